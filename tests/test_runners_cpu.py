"""The command-line runners' argument handling and their device-free paths, on the CPU.

ernie-block-runner and ernie-denoise-runner keep the flags of the reference's probes
(probes/block_runner.cpp:41-90, probes/denoise_runner.cpp:42-100): usage errors exit 2
(block runner) or 1 (denoise runner) before any device work; inputs of the wrong size, a
graph whose static token count differs and a per-query mask are refused; the denoise
runner's --timestep mode writes the time features without a device.
"""
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import ernie_amd as E
import oracle as O

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "ernie-image-ncnn-vulkan_amd" / "lib"
BLOCK = LIB / "ernie-block-runner"
DENOISE = LIB / "ernie-denoise-runner"
GOLDEN = Path(__file__).with_name("golden")


def run(exe, *args):
    return subprocess.run([str(exe), *map(str, args)], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                          timeout=120)


@pytest.mark.parametrize("args", [
    [],
    ["--model", "m", "--fixture", "f", "--tokens", "288", "--output", "o", "--backend", "cpu"],
    ["--model", "m", "--fixture", "f", "--tokens", "288", "--output", "o", "--repeat", "21"],
    ["--model", "m", "--fixture", "f", "--tokens", "0", "--output", "o"],
    ["--model", "m", "--fixture", "f", "--tokens", "28x", "--output", "o"],
    ["--model", "m", "--fixture", "f", "--tokens", "288", "--output", "o", "--precision", "fp8"],
    ["--model", "m", "--fixture", "f", "--tokens", "288", "--output", "o", "--output-blob", "15"],
    ["--model", "m", "--fixture", "f", "--tokens", "288", "--output", "o", "--bogus", "1"],
    ["--model"],
])
def test_block_runner_usage(args):
    p = run(BLOCK, *args)
    assert p.returncode == 2 and "Usage: ernie-block-runner" in p.stderr, (p.returncode, p.stderr)


def _block_fixture(tmp_path, tokens=288, dim=4096, mask=None):
    model, fixture = tmp_path / "model", tmp_path / "fixture"
    model.mkdir(parents=True)
    fixture.mkdir(parents=True)
    (model / "block.ncnn.param").write_bytes((GOLDEN / "block_component_s288.ncnn.param").read_bytes())
    np.zeros((tokens, dim), "<f4").tofile(fixture / "in0.f32")
    for i in range(1, 7):
        np.zeros(dim, "<f4").tofile(fixture / f"in{i}.f32")
    np.zeros((tokens, 128), "<f4").tofile(fixture / "in7.f32")
    np.zeros((tokens, 128), "<f4").tofile(fixture / "in8.f32")
    (np.zeros((tokens, tokens), "<f4") if mask is None else mask.astype("<f4")).tofile(fixture / "in9.f32")
    return model, fixture


def test_block_runner_refuses_bad_inputs_before_the_device(tmp_path):
    model, fixture = _block_fixture(tmp_path)
    out = tmp_path / "out.f32"
    p = run(BLOCK, "--model", model, "--fixture", fixture, "--tokens", 100, "--output", out)
    assert p.returncode == 1 and "static at 288 tokens" in p.stderr, p.stderr
    (fixture / "in7.f32").write_bytes(b"\0" * 12)
    p = run(BLOCK, "--model", model, "--fixture", fixture, "--tokens", 288, "--output", out)
    assert p.returncode == 1 and "byte count mismatch" in p.stderr and "in7.f32" in p.stderr, p.stderr
    # A mask that differs between query rows is not the block's broadcast mask.
    mask = np.zeros((288, 288), np.float32)
    mask[5, 200:] = -1e30
    model2, fixture2 = _block_fixture(tmp_path / "b", mask=mask)
    p = run(BLOCK, "--model", model2, "--fixture", fixture2, "--tokens", 288, "--output", out)
    assert p.returncode == 1 and "mask row 5 differs" in p.stderr, p.stderr
    # An existing output is never overwritten.
    out.write_bytes(b"x")
    p = run(BLOCK, "--model", model2, "--fixture", fixture2, "--tokens", 288, "--output", out)
    assert p.returncode == 1 and "Output exists" in p.stderr
    assert not list(tmp_path.glob("*.tmp"))


@pytest.mark.parametrize("t", [0.0, 363.63638, 1000.0])
def test_denoise_runner_time_features_without_a_device(tmp_path, t):
    out = tmp_path / "features"
    p = run(DENOISE, "--output", out, "--timestep", repr(t))
    assert p.returncode == 0, p.stderr
    got = np.fromfile(out / "features.f32", "<f4")
    np.testing.assert_array_equal(got, E.timestep_features(t))
    np.testing.assert_array_equal(got, O.timestep_features(t))
    p = run(DENOISE, "--output", out, "--timestep", repr(t))
    assert p.returncode == 1 and "new --output" in p.stderr


@pytest.mark.parametrize("args,message", [
    (["--timestep", "1000.5"], "Timestep must be finite and in [0,1000]"),
    (["--timestep", "5x"], "Invalid timestep"),
    (["--fixture", "f", "--width", "4", "--height", "4", "--text-tokens", "8", "--model", "m",
      "--input-head", "i", "--output-head", "o", "--backend", "cpu"], "device only"),
    (["--fixture", "f", "--width", "4", "--height", "4", "--text-tokens", "8", "--input-head", "i",
      "--output-head", "o"], "Require heads, blocks"),
    (["--fixture", "f", "--width", "257", "--height", "4", "--text-tokens", "8", "--model", "m",
      "--input-head", "i", "--output-head", "o"], "Require heads, blocks"),
    (["--steps", "x"], "Invalid integer for --steps"),
    (["--bogus", "1"], "Unknown argument: --bogus"),
])
def test_denoise_runner_usage(tmp_path, args, message):
    p = run(DENOISE, "--output", tmp_path / "o", *args)
    assert p.returncode == 1 and message in p.stderr, (p.returncode, p.stderr)
    assert not (tmp_path / "o").exists()
