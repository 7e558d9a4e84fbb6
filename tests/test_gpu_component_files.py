"""DiT heads and text blocks loaded from their .param + .bin files compute exactly what
the same weights uploaded from host arrays compute (the head and text-block halves of
load_component, src/dit.cpp:22-45 and src/text_encoder.cpp:30-40).

The weights are exact in FP32, BF16 and FP16, so every ModelBin storage tag describes
the same values and the device outputs must agree bitwise.
"""
import numpy as np
import pytest

import ernie_amd as E
import oracle as O
from gpu_util import NAMES, ALL_DT, dev, empty, host
from test_oracle import small_block
from test_component_files import (exact_head_weights, exact_text_weights, head_graph, text_graph, write_head_bin,
                                  write_text_bin, GOLDEN)

pytestmark = pytest.mark.gpu


def run_heads(ctx, dim, latent, text_dim, H, W, T, seed=5):
    """Input head then output head on fixed inputs; returns x, c, mods, prediction (host)."""
    hw = H * W
    lat = O.normal((latent, H, W), seed)
    tx = O.normal((T, text_dim), seed + 1)
    feat = O.normal((dim,), seed + 2)
    x, c, mods = empty((hw + T, dim)), empty((dim,)), empty((6, dim))
    ctx.input_head(dev(lat), hw, dev(tx), T, dev(feat), x, c, mods)
    pred = empty((latent, H, W))
    ctx.output_head(x, hw + T, hw, c, pred)
    return host(x), host(c), host(mods), host(pred)


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_loaded_heads_match_uploaded_heads(tmp_path, dt):
    dim, latent, text_dim, H, W, T = 256, 32, 64, 2, 4, 8
    fac = E.Facade(0)
    try:
        w = exact_head_weights(dim, latent, text_dim, seed=11)
        fac.hip.heads_upload(w, dim, latent, text_dim, dt)
        assert fac.hip.heads_loaded() == E.HEAD_INPUT | E.HEAD_OUTPUT
        ref = run_heads(fac.hip, dim, latent, text_dim, H, W, T)
        assert all(np.isfinite(r).all() for r in ref)
        graphs = {}
        for kind in ("input", "output"):
            graphs[kind] = tmp_path / f"{kind}.ncnn.param"
            graphs[kind].write_text(head_graph(kind, dim, latent, text_dim, W, H, T))
        for storage in (E.FP32, E.BF16, E.FP16):
            bins = {}
            for kind in ("input", "output"):
                bins[kind] = tmp_path / f"{kind}_{NAMES[storage]}.ncnn.bin"
                write_head_bin(bins[kind], kind, w, storage)
            info_in = fac.head_load(graphs["input"], bins["input"], dt, allow_unreviewed=True)
            info_out = fac.head_load(graphs["output"], bins["output"], dt, allow_unreviewed=True)
            assert (info_in["part"], info_out["part"]) == (E.HEAD_INPUT, E.HEAD_OUTPUT)
            assert fac.hip.heads_loaded() == E.HEAD_INPUT | E.HEAD_OUTPUT
            got = run_heads(fac.hip, dim, latent, text_dim, H, W, T)
            for name, g, r in zip(("x", "c", "mods", "prediction"), got, ref):
                np.testing.assert_array_equal(g, r, err_msg=f"{name} from {NAMES[storage]} files")
        # An output head of another width cannot sit beside the resident input head.
        other = tmp_path / "other.ncnn.param"
        other.write_text(head_graph("output", 384, latent, text_dim, W, H, T))
        ob = tmp_path / "other.ncnn.bin"
        write_head_bin(ob, "output", exact_head_weights(384, latent, text_dim, seed=12), E.FP32)
        with pytest.raises(E.ErnieError, match="width"):
            fac.head_load(other, ob, dt, allow_unreviewed=True)
        # An unreviewed graph is refused unless the caller opts in; the heads stay loaded.
        with pytest.raises(E.ErnieInvalidRequest):
            fac.head_load(graphs["input"], tmp_path / "input_fp32.ncnn.bin", dt)
        np.testing.assert_array_equal(run_heads(fac.hip, dim, latent, text_dim, H, W, T)[3], ref[3])
    finally:
        fac.close()


def test_denoise_on_file_loaded_heads(tmp_path):
    # The facade's denoise (src/denoiser.h:13-44) at the reference's head widths (dim 4096,
    # 128 latent channels, 3072-wide text) with the heads loaded from BF16 files, against
    # the same weights uploaded from host arrays: bitwise the same latent after two steps.
    import torch
    dim, latent, text_dim, ffn = 4096, 128, 3072, 512
    H = W = 4
    T, valid = 8, 5
    fac = E.Facade(0)
    try:
        lat0 = O.normal((latent, H, W), 31)
        tx = O.normal((T, text_dim), 32)
        tx[valid:] = 0.0
        cos, sin, mask = O.dit_constants(O.rope_frequencies(), W, H, valid, T)
        args = (dev(tx), T, dev(cos), dev(sin), dev(mask), H * W + valid, 2)
        # No heads resident: the request is rejected before any device work.
        fac.hip.block_upload(0, small_block(dim, ffn, seed=34), dim, ffn, E.FP16)
        with pytest.raises(E.ErnieInvalidRequest, match="head"):
            fac.denoise([0], dev(lat0), H, W, *args, dtype=E.FP16)
        w = exact_head_weights(dim, latent, text_dim, seed=33)
        fac.hip.heads_upload(w, dim, latent, text_dim, E.FP16)
        ref = dev(lat0)
        fac.denoise([0], ref, H, W, *args, dtype=E.FP16)
        ref = host(ref)
        assert np.isfinite(ref).all()
        fac.hip.heads_init_random(dim, latent, text_dim, E.FP16, seed=99)  # something else resident first
        for kind, graph in (("input", GOLDEN / "head_input_s288.ncnn.param"),
                            ("output", GOLDEN / "head_output_s288.ncnn.param")):
            b = tmp_path / f"{kind}.ncnn.bin"
            write_head_bin(b, kind, w, E.BF16)
            info = fac.head_load(graph, b, E.FP16)
            assert info["reviewed"] and info["dim"] == dim
            b.unlink()
        got = dev(lat0)
        fac.denoise([0], got, H, W, *args, dtype=E.FP16)
        np.testing.assert_array_equal(host(got), ref)
    finally:
        torch.cuda.synchronize()
        fac.close()


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_loaded_text_block_matches_uploaded_block(tmp_path, dt):
    hidden, heads, kv, ffn, S = 512, 4, 2, 1024, 16
    fac = E.Facade(0)
    try:
        w = exact_text_weights(hidden, heads, kv, ffn, seed=21)
        fac.hip.text_block_upload(0, w, hidden, heads, kv, ffn, dt)
        freqs = (1.0 / (1e6 ** (np.arange(0, 128, 2) / 128.0))).astype(np.float32)
        cos, sin, mask = O.text_constants(freqs, S)
        x = O.normal((S, hidden), 22, std=0.2)

        def forward(slot):
            out = empty((S, hidden))
            fac.hip.text_block_forward(slot, dev(x), out, dev(cos), dev(sin), S, causal=True)
            return host(out)

        ref = forward(0)
        assert np.isfinite(ref).all()
        g = tmp_path / "text.ncnn.param"
        g.write_text(text_graph(hidden, heads, kv, ffn, S))
        for i, storage in enumerate((E.FP32, E.BF16, E.FP16), start=1):
            b = tmp_path / f"text_{NAMES[storage]}.ncnn.bin"
            write_text_bin(b, w, storage)
            info = fac.text_block_load(i, g, b, dt, allow_unreviewed=True)
            assert (info["hidden"], info["heads"], info["kv_heads"], info["ffn"], info["tokens"]) == \
                (hidden, heads, kv, ffn, S)
            np.testing.assert_array_equal(forward(i), ref, err_msg=NAMES[storage])
        with pytest.raises(E.ErnieInvalidRequest):
            fac.text_block_load(5, g, tmp_path / "text_bf16.ncnn.bin", dt)
        for i in range(4):
            fac.hip.call("text_block_release", i)
    finally:
        fac.close()
