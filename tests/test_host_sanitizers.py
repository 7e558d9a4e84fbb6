"""The host-side parsers of caller-supplied data under AddressSanitizer and
UndefinedBehaviorSanitizer (CPU only).

tests/host_fuzz.cpp drives the ncnn .param graph checks, the ModelBin section walks,
the graph/weight file readers (host/block_files.cpp, and host/component_files.cpp for the
DiT heads and text blocks), SHA-256, pad_text,
dit_constants and FlowSchedule::turbo with seeded mutations of the reference's own
graph fixtures and of well-formed weight files. Every input must either pass the
checks or raise a C++ exception; any sanitizer report aborts the run.
"""
import os
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HOST = ROOT / "ernie-image-ncnn-vulkan_amd" / "host"
SOURCES = [ROOT / "tests" / "host_fuzz.cpp"] + [HOST / f for f in
                                                 ("block_files.cpp", "component_files.cpp", "sha256.cpp",
                                                  "conditioning.cpp", "latent_ops.cpp")]


@pytest.fixture(scope="module")
def fuzz_binary(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    out = tmp_path_factory.mktemp("asan") / "host_fuzz"
    # Host code only: the device half of these files (uploads) is dropped by the linker.
    cmd = ["g++", "-std=c++17", "-O1", "-g", "-fno-omit-frame-pointer", "-fsanitize=address,undefined",
           "-fno-sanitize-recover=all", "-ffunction-sections", "-fdata-sections", "-ffp-contract=off",
           f"-I{ROOT / 'include'}", f"-I{HOST}", "-I/opt/rocm/include", "-D__HIP_PLATFORM_AMD__",
           *map(str, SOURCES), "-Wl,--gc-sections", "-o", str(out)]
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    assert proc.returncode == 0, proc.stdout
    return out


@pytest.mark.parametrize("seed", [1, 7])
def test_host_parsers_clean_under_sanitizers(fuzz_binary, tmp_path, seed):
    env = dict(os.environ, ASAN_OPTIONS="halt_on_error=1:detect_leaks=1:abort_on_error=0",
               UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")
    proc = subprocess.run([str(fuzz_binary), str(ROOT / "tests" / "golden"), str(tmp_path), "600", str(seed)],
                          stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, env=env, timeout=300)
    assert proc.returncode == 0, proc.stdout[-4000:]
    assert "ERROR: AddressSanitizer" not in proc.stdout and "runtime error" not in proc.stdout, proc.stdout[-4000:]
    line = [l for l in proc.stdout.splitlines() if l.startswith("host_fuzz:")]
    assert line, proc.stdout[-2000:]
    # Both outcomes occur: the mutations are not all rejected, nor all accepted.
    parts = line[0].split()
    accepted, rejected = int(parts[3]), int(parts[5])
    assert accepted > 0 and rejected > 0, line[0]
