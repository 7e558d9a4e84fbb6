"""Build the gfx950 HIP library and the C++ host facade in-tree.

    lib/libernie_hip.so  kernels + extern "C" ABI (include/ernie_hip.h), hipcc
    lib/libernie.so      C++ facade mirroring the reference's block-runner /
                         DiT / denoise API, g++, linked against libernie_hip.so
    lib/ernie-block-runner, lib/ernie-denoise-runner
                         command-line runners with the reference probes' flags
                         (probes/block_runner.cpp, probes/denoise_runner.cpp), g++

Usage: python build.py [--jobs N]
"""
import argparse
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
HOST = PKG / "host"
RUNNERS = PKG / "runners"
LIB = PKG / "lib"
OBJ = LIB / "obj"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))

HIP_SOURCES = ["gemm.hip", "gemm16_pp.hip", "sdpa.hip", "sdpa16_dl.hip", "pointwise.hip", "noalloc.hip", "mfma_rate.hip",
               "ernie_hip.cpp"]
HOST_SOURCES = ["runtime.cpp", "conditioning.cpp", "latent_ops.cpp", "denoiser.cpp", "block_sequence.cpp", "dit.cpp", "ops.cpp",
                "sha256.cpp", "block_files.cpp", "block_upload.cpp", "component_files.cpp", "text_encoder.cpp", "capi.cpp"]

# Packed-FP32 VALU forms are disabled for every HIP translation unit.
HIPCC_FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++17", "-fPIC", "-Wall", "-Xclang", "-target-feature",
               "-Xclang", "-packed-fp32-ops", f"-I{ROOT / 'include'}", f"-I{CSRC}"]
# The facade restates the reference's FP32 host arithmetic (schedule, time
# features, RoPE tables), which the reference compiles with -ffp-contract=off.
CXX_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-Wall", "-Wextra", "-ffp-contract=off", f"-I{ROOT / 'include'}",
             f"-I{HOST}", f"-I{ROCM / 'include'}", "-D__HIP_PLATFORM_AMD__"]


def run(cmd):
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(map(str, cmd))}\n{out}")
    return out


def build(jobs=8, verbose=False):
    OBJ.mkdir(parents=True, exist_ok=True)
    hipcc = str(ROCM / "bin" / "hipcc")

    def hip_obj(src):
        obj = OBJ / (src + ".o")
        return run([hipcc, *HIPCC_FLAGS, "-c", str(CSRC / src), "-o", str(obj)]), obj

    def host_obj(src):
        obj = OBJ / (src + ".o")
        return run(["g++", *CXX_FLAGS, "-c", str(HOST / src), "-o", str(obj)]), obj

    with ThreadPoolExecutor(max_workers=jobs) as pool:
        hip_results = list(pool.map(hip_obj, HIP_SOURCES))
        host_results = list(pool.map(host_obj, HOST_SOURCES))
    for out, _ in hip_results + host_results:
        if verbose and out.strip():
            print(out)
    hip_so = LIB / "libernie_hip.so"
    tmp = LIB / "libernie_hip.so.tmp"
    run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(tmp), *[str(o) for _, o in hip_results]])
    os.replace(tmp, hip_so)
    host_so = LIB / "libernie.so"
    tmp = LIB / "libernie.so.tmp"
    run(["g++", "-shared", "-fPIC", "-o", str(tmp), *[str(o) for _, o in host_results], f"-L{LIB}", "-lernie_hip",
         "-Wl,-rpath,$ORIGIN", "-Wl,--no-as-needed"])
    os.replace(tmp, host_so)

    def runner(name, src):
        exe = LIB / name
        tmp = LIB / (name + ".tmp")
        run(["g++", *CXX_FLAGS, f"-I{RUNNERS}", str(RUNNERS / src), "-o", str(tmp), f"-L{LIB}", "-lernie",
             "-lernie_hip", "-Wl,-rpath,$ORIGIN"])
        os.replace(tmp, exe)
        return exe

    with ThreadPoolExecutor(max_workers=2) as pool:
        runners = list(pool.map(lambda a: runner(*a), (("ernie-block-runner", "block_runner.cpp"),
                                                       ("ernie-denoise-runner", "denoise_runner.cpp"))))
    return (hip_so, host_so, *runners)


if __name__ == "__main__":
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--jobs", type=int, default=8)
    ap.add_argument("-v", "--verbose", action="store_true")
    args = ap.parse_args()
    for p in build(args.jobs, args.verbose):
        print(p)
    sys.exit(0)
