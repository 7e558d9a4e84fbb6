"""The command-line runners on the device: ernie-block-runner on a full-width block in
the reviewed component graph (288 tokens: 4x4 latent grid, 272 text slots, 270 valid,
the layout of the reference's own block fixture), against the oracle under the block
gates; ernie-denoise-runner on that block with both heads loaded from their files,
against the facade's denoise on the same weights (bitwise) and the oracle (denoiser gate).
The fixtures are written here in the probes' file layout (in0..in9.f32).
"""
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

import ernie_amd as E
import kat
import oracle as O
from gpu_util import NAMES, dev, empty, host
from test_block_files import exact_weights, write_block_bin
from test_component_files import exact_head_weights, write_head_bin

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parent.parent
LIB = ROOT / "ernie-image-ncnn-vulkan_amd" / "lib"
GOLDEN = Path(__file__).with_name("golden")
DIM, FFN, W, H, TEXT, VALID = 4096, 12288, 4, 4, 272, 270
S = W * H + TEXT


@pytest.fixture(scope="module")
def block_dir(tmp_path_factory):
    d = tmp_path_factory.mktemp("block")
    w = exact_weights(DIM, FFN, seed=8)
    (d / "block.ncnn.param").write_bytes((GOLDEN / "block_component_s288.ncnn.param").read_bytes())
    write_block_bin(d / "block.ncnn.bin", w, E.BF16)
    return d, w


def run(*args):
    p = subprocess.run([str(a) for a in args], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                       timeout=600)
    print(p.stderr[-2000:], flush=True)
    return p


@pytest.mark.parametrize("dt", [E.FP16, E.BF16], ids=lambda d: NAMES[d])
def test_block_runner_against_oracle(tmp_path, block_dir, dt):
    model, w = block_dir
    fixture = tmp_path / "fixture"
    fixture.mkdir()
    cos, sin, mask = O.dit_constants(O.rope_frequencies(), W, H, VALID, TEXT)
    x = O.normal((S, DIM), 9)
    mods = O.normal((6, DIM), 10, std=0.5)
    x.astype("<f4").tofile(fixture / "in0.f32")
    for i in range(6):
        mods[i].astype("<f4").tofile(fixture / f"in{i + 1}.f32")
    cos.astype("<f4").tofile(fixture / "in7.f32")
    sin.astype("<f4").tofile(fixture / "in8.f32")
    np.broadcast_to(mask, (S, S)).astype("<f4").tofile(fixture / "in9.f32")
    out = tmp_path / "actual.f32"
    p = run(LIB / "ernie-block-runner", "--model", model, "--fixture", fixture, "--tokens", S, "--output", out,
            "--backend", "vulkan", "--precision", NAMES[dt], "--repeat", 2, "--trace-attention")
    assert p.returncode == 0, p.stderr
    info = json.loads([l for l in p.stdout.splitlines() if l.startswith("{")][-1])
    assert (info["tokens"], info["dim"], info["repeat_max_abs"], info["valid_keys"]) == (S, DIM, 0, W * H + VALID)
    assert len(info["run_seconds"]) == 2 and info["attention_diagnostic"]["flash_calls"] == 2
    got = np.fromfile(out, "<f4").reshape(S, DIM)
    ref = O.block_forward(w, x, mods, cos, sin, mask)
    g = kat.gate(got, ref, *kat.BLOCK_GATES[NAMES[dt]])
    assert g["passed"], g


def test_denoise_runner_against_facade_and_oracle(tmp_path, block_dir):
    import torch
    model, wb = block_dir
    steps, dt = 2, E.FP16
    heads = exact_head_weights(DIM, 128, 3072, seed=17)
    dirs = {}
    for kind in ("input", "output"):
        dirs[kind] = tmp_path / kind
        dirs[kind].mkdir()
        (dirs[kind] / "head.ncnn.param").write_bytes((GOLDEN / f"head_{kind}_s288.ncnn.param").read_bytes())
        write_head_bin(dirs[kind] / "head.ncnn.bin", kind, heads, E.BF16)
    fixture = tmp_path / "fixture"
    fixture.mkdir()
    latent = O.normal((128, H, W), 18)
    text = O.normal((TEXT, 3072), 19)
    text[VALID:] = 0.0
    cos, sin, mask = O.dit_constants(O.rope_frequencies(), W, H, VALID, TEXT)
    latent.astype("<f4").tofile(fixture / "in0.f32")
    text.astype("<f4").tofile(fixture / "in1.f32")
    cos.astype("<f4").tofile(fixture / "in3.f32")
    sin.astype("<f4").tofile(fixture / "in4.f32")
    np.broadcast_to(mask, (S, S)).astype("<f4").tofile(fixture / "in5.f32")
    out = tmp_path / "out"
    p = run(LIB / "ernie-denoise-runner", "--model", model, "--input-head", dirs["input"], "--output-head",
            dirs["output"], "--fixture", fixture, "--width", W, "--height", H, "--text-tokens", TEXT, "--steps",
            steps, "--output", out, "--backend", "hip", "--precision", "fp16", "--trace")
    assert p.returncode == 0, p.stderr
    lines = [json.loads(l) for l in p.stdout.splitlines() if l.startswith("{")]
    sig, ts = O.flow_schedule_turbo(steps)
    assert [l["step"] for l in lines[:-1]] == list(range(steps))
    assert [np.float32(l["timestep"]) for l in lines[:-1]] == list(ts[:steps])
    assert all(l["elapsed_seconds"] > 0 and l["block_compute_seconds"] > 0 for l in lines[:-1])
    assert lines[-1]["complete"] and lines[-1]["steps"] == steps and lines[-1]["blocks"] == 1
    final = np.fromfile(out / "final.f32", "<f4").reshape(latent.shape)
    np.testing.assert_array_equal(np.fromfile(out / f"step-{steps - 1}.f32", "<f4").reshape(latent.shape), final)
    # The facade in this process, on the same weights uploaded from host arrays.
    fac = E.Facade(0)
    try:
        fac.hip.heads_upload(heads, DIM, 128, 3072, dt)
        fac.hip.block_upload(0, wb, DIM, FFN, dt)
        lat = dev(latent)
        fac.denoise([0], lat, H, W, dev(text), TEXT, dev(cos), dev(sin), dev(mask), W * H + VALID, steps, dtype=dt)
        np.testing.assert_array_equal(final, host(lat))
    finally:
        torch.cuda.synchronize()
        fac.close()
    # The oracle's two steps.
    ref = latent.copy()
    out_w = {"mod_w": heads["out_mod_w"], "mod_b": heads["out_mod_b"], "proj_w": heads["proj_w"],
             "proj_b": heads["proj_b"]}
    for i in range(steps):
        x, c, mods = O.input_head({k: heads[k] for k in O.INPUT_HEAD_FIELDS}, ref, text,
                                  O.timestep_features(float(ts[i])))
        x = O.block_forward(wb, x, mods, cos, sin, mask)
        pred = O.output_head(out_w, x, c, W * H).reshape(ref.shape)
        ref = O.euler_step(ref, pred, sig[i + 1] - sig[i])
    nrmse, rtol, atol = kat.DENOISER_GATES["fp16"]
    g = kat.gate(final, ref, atol, rtol, nrmse)
    assert g["passed"], g
