"""Pins the CPU oracle (oracle/) before it is trusted as the parity reference.

Every oracle function is checked against the reference's own known-answer
tests (ported in kat.py), closed forms, library routines in FP64 (PyTorch on
the CPU), or invariants chosen so that a dropped term, wrong sign or transposed
operand fails.
"""
import hashlib
import json
import math
from pathlib import Path

import numpy as np
import pytest

import kat
import oracle as O

GOLDEN = Path(__file__).with_name("golden")


# ---- synthetic generator -------------------------------------------------------------
def test_normal_generator_moments_and_slices():
    x = O.normal((400000,), seed=11)
    assert abs(float(x.mean())) < 5e-3 and abs(float(x.std()) - 1.0) < 5e-3
    # Counter-based: any slice regenerates alone; seeds differ.
    np.testing.assert_array_equal(O.normal((100,), 11, offset=1234), x[1234:1334])
    assert not np.array_equal(O.normal((100,), 12), x[:100])
    y = O.normal((1000,), 3, mean=1.0, std=0.02)
    assert abs(float(y.mean()) - 1.0) < 3e-3 and abs(float(y.std()) - 0.02) < 3e-3


# ---- closed forms ------------------------------------------------------------------------
def test_flow_schedule_contract():
    # tests/test_latent_contract.cpp:19-28
    with pytest.raises(ValueError):
        O.flow_schedule_turbo(0)
    with pytest.raises(ValueError):
        O.flow_schedule_turbo(1001)
    sig, ts = O.flow_schedule_turbo(8)
    assert sig[0] == 1.0 and sig[-1] == 0.0
    assert all(sig[i + 1] - sig[i] < 0 for i in range(8))
    np.testing.assert_array_equal(ts, (np.float32(1000.0) * sig[:8]).astype(np.float32))
    # FP64 closed form: s = 1 - i/S, sigma = 4s / (1 + 3s).
    for steps in (1, 2, 7, 8, 50, 1000):
        sig, _ = O.flow_schedule_turbo(steps)
        s = 1.0 - np.arange(steps) / steps
        np.testing.assert_allclose(sig[:steps], 4 * s / (1 + 3 * s), rtol=4e-7, atol=1e-7)


def test_timestep_features_closed_form():
    with pytest.raises(ValueError):
        O.timestep_features(-1.0)
    with pytest.raises(ValueError):
        O.timestep_features(1000.5)
    with pytest.raises(ValueError):
        O.timestep_features(float("nan"))
    f0 = O.timestep_features(0.0)
    assert np.all(f0[:2048] == 0.0) and np.all(f0[2048:] == 1.0)
    for t in (1000.0, 500.0, 363.63638, 1.0):
        f = O.timestep_features(t)
        phase = t * np.exp(-math.log(10000.0) * np.arange(2048) / 2048.0)
        # FP32 phase rounding bounds the error: |d phase| <= t * 2^-23 ~ 1.2e-4 at t = 1000
        # (the reference's own time-feature gate is max_abs 1.3e-4, tools/validate_denoiser.py:55).
        np.testing.assert_allclose(f[:2048], np.sin(phase), atol=1.3e-4)
        np.testing.assert_allclose(f[2048:], np.cos(phase), atol=1.3e-4)


def test_euler_independent_recurrence():
    # tests/test_memory_execution.cpp:323-330: a tiny denoiser v = 0.125 x through
    # real Euler steps against an independent FP32 recurrence (<= 3e-7).
    steps = 4
    sig, _ = O.flow_schedule_turbo(steps)
    x0 = O.normal((128, 3, 5), 21)
    x = x0.copy()
    for i in range(steps):
        x = O.euler_step(x, np.float32(0.125) * x, sig[i + 1] - sig[i])
    expected = x0.astype(np.float64)
    for i in range(steps):
        expected = expected + float(np.float32(sig[i + 1] - sig[i])) * (expected * 0.125)
    assert np.max(np.abs(x - expected)) <= 3e-7 * max(1.0, float(np.abs(expected).max()))
    # Alias-safe consume-and-replace (tests/test_latent_contract.cpp:41-45): 1 + (-1 * 1) = 0.
    ones = np.ones((128, 15), np.float32)
    assert np.all(O.euler_step(ones, ones, -1.0) == 0.0)


def test_rope_frequencies_match_torch_fixture():
    fixture = np.fromfile(GOLDEN / "rope_inv_freq.f32", dtype="<f4")
    ours = O.rope_frequencies()
    assert fixture.shape == (64,)
    # Same FP32 formula through two libm implementations: within one ulp.
    ulp = np.spacing(fixture)
    assert np.all(np.abs(ours - fixture) <= ulp)
    # Closed form structure: axis blocks of 16, 24, 24 starting at 1.
    assert ours[0] == 1.0 and ours[16] == 1.0 and ours[40] == 1.0
    np.testing.assert_allclose(ours[:16], 256.0 ** (-np.arange(0, 32, 2) / 32.0), rtol=2e-7)


def test_dit_constants_brute_force():
    freqs = np.fromfile(GOLDEN / "rope_inv_freq.f32", dtype="<f4")
    w, h, valid, text = 5, 3, 4, 7
    cos, sin, mask = O.dit_constants(freqs, w, h, valid, text)
    S = w * h + text
    assert cos.shape == (S, 128)
    for i in range(S):
        pos = (valid, i // w, i % w) if i < w * h else (i - w * h, 0, 0)
        for j in range(64):
            axis = 0 if j < 16 else (1 if j < 40 else 2)
            phase = np.float32(np.float32(pos[axis]) * freqs[j])
            assert cos[i, 2 * j] == cos[i, 2 * j + 1] and sin[i, 2 * j] == sin[i, 2 * j + 1]
            assert abs(cos[i, 2 * j] - math.cos(float(phase))) <= 6e-8
            assert abs(sin[i, 2 * j] - math.sin(float(phase))) <= 6e-8
    np.testing.assert_array_equal(mask, np.where(np.arange(S) >= w * h + valid, -1e30, 0.0).astype(np.float32))
    for bad in ((0, 3, 1, 2), (5, 3, 0, 2), (5, 3, 3, 2), (5, 3, 1, 2049)):
        with pytest.raises(ValueError):
            O.dit_constants(freqs, *bad)


def _official_block00():
    """The reference's block-0 fixture record: layout and SHA-256 of the official inputs
    (artifacts/2026-09-05/components/blocks/block-00/runtime/fixture.json)."""
    fx = json.loads((GOLDEN / "block00_runtime_fixture.json").read_text())
    w, h = fx["grid"]
    assert fx["tokens"] == w * h + fx["text_tokens"]
    return fx, w, h


def _sha256_f32(a):
    return hashlib.sha256(np.ascontiguousarray(a, "<f4").tobytes()).hexdigest()


def test_dit_mask_reproduces_official_in9():
    # in9 is the official dense [S][S] additive mask of a 4x4 grid with 272 text slots,
    # 270 valid; the oracle's one-row mask broadcast over the queries is bitwise that tensor.
    fx, w, h = _official_block00()
    S = fx["tokens"]
    _, _, mask = O.dit_constants(O.rope_frequencies(), w, h, fx["valid_text"], fx["text_tokens"])
    assert fx["inputs"]["in9"]["shape"] == [S, S]
    assert _sha256_f32(np.broadcast_to(mask.reshape(1, S), (S, S))) == fx["inputs"]["in9"]["sha256"]


def test_dit_rope_layout_reproduces_official_in7_in8():
    # in7 / in8 are the official model's position embeddings. PyTorch FP32 cos / sin of
    # position x frequency, with image token i at (valid, i / w, i % w), text token j at
    # (j, 0, 0), axes of 16 / 24 / 24 frequencies and each value duplicated into columns
    # 2j and 2j + 1, reproduce both hashes bitwise: that pins the position layout, the axis
    # split and the column duplication to the official model. The oracle's table (glibc
    # cosf / sinf of the same FP32 phases) is then within one ulp of it everywhere.
    torch = pytest.importorskip("torch")
    fx, w, h = _official_block00()
    S, valid, image = fx["tokens"], fx["valid_text"], w * h
    freqs = O.rope_frequencies()
    pos = np.array([(valid, i // w, i % w) if i < image else (i - image, 0, 0) for i in range(S)], np.float32)
    axis = np.array([0 if j < 16 else 1 if j < 40 else 2 for j in range(64)])
    phase = torch.from_numpy(np.ascontiguousarray(pos[:, axis])) * torch.from_numpy(freqs)[None, :]
    tc = torch.cos(phase).repeat_interleave(2, dim=1).numpy()
    ts = torch.sin(phase).repeat_interleave(2, dim=1).numpy()
    assert _sha256_f32(tc) == fx["inputs"]["in7"]["sha256"]
    assert _sha256_f32(ts) == fx["inputs"]["in8"]["sha256"]
    cos, sin, _ = O.dit_constants(freqs, w, h, valid, fx["text_tokens"])
    for ours, official in ((cos, tc), (sin, ts)):
        assert np.all(np.abs(ours.astype(np.float64) - official) <= np.spacing(np.abs(official)))
        assert np.mean(ours == official) > 0.95


# ---- operators -----------------------------------------------------------------------------
@pytest.mark.parametrize("width", [128, 3072, 4096])
@pytest.mark.parametrize("scale", [1.0, 512.0])
def test_rmsnorm_probe_kat(width, scale):
    x, gamma, expected = kat.rmsnorm_kat_case(width, scale)
    out = O.rmsnorm(x, gamma)
    assert np.max(np.abs(out - expected)) <= kat.RMSNORM_LIMITS["fp32"]


@pytest.mark.parametrize("scale", [1.0, 1024.0])
def test_layernorm_probe_kat(scale):
    x, _, expected = kat.rmsnorm_kat_case(4096, scale, centered=True)
    assert np.max(np.abs(O.layernorm(x) - expected)) <= kat.RMSNORM_LIMITS["fp32"]


@pytest.mark.parametrize("shape", [0, 1])
def test_gelu_probe_kat(shape):
    x = kat.gelu_kat_input(shape)
    assert np.max(np.abs(O.gelu(x) - kat.gelu_expected(x))) <= kat.GELU_LIMITS["fp32"]


def test_modulate_is_the_graph_binary_ops():
    h = O.normal((3, 8), 1)
    shift, scale = O.normal((8,), 2), O.normal((8,), 3)
    out = O.modulate(h, shift, scale)
    np.testing.assert_array_equal(out, (h * (scale + np.float32(1.0)) + shift).astype(np.float32))


@pytest.mark.parametrize("name,m,n,k,bias", kat.GEMM_KAT_SHAPES)
def test_gemm_exact_products_kat(name, m, n, k, bias):
    a, w, b = kat.gemm_kat_case(m, n, k)
    out = O.gemm_nt(a, w, b if bias else None)
    ref = a.astype(np.float64) @ w.astype(np.float64).T + (b.astype(np.float64) if bias else 0.0)
    # Operands are multiples of 1/8: every FP32 product and partial sum is exact.
    np.testing.assert_array_equal(out.astype(np.float64), ref)
    np.testing.assert_array_equal(kat.rne_bf16(out), kat.rne_bf16(ref.astype(np.float32)))


def test_gemm_random_against_fp64():
    a = O.normal((70, 96), 5)
    w = O.normal((50, 96), 6, std=0.02)
    ref = a.astype(np.float64) @ w.astype(np.float64).T
    np.testing.assert_allclose(O.gemm_nt(a, w), ref, rtol=1e-5, atol=1e-6)


def test_rope_rows_matches_torch_rotary():
    import torch
    x = O.normal((6, 128), 9)
    ang = O.normal((6, 128), 10)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    t = torch.from_numpy(x).double()
    c, s = torch.from_numpy(cos).double(), torch.from_numpy(sin).double()
    # tools/export_dit_block.py:39-47 with explicit halves.
    ref = torch.cat((t[:, :64] * c[:, :64] - t[:, 64:] * s[:, :64], t[:, 64:] * c[:, 64:] + t[:, :64] * s[:, 64:]),
                    dim=-1)
    np.testing.assert_allclose(O.rope_rows(x, cos, sin), ref.numpy(), atol=1e-6)


@pytest.mark.parametrize("mask_heads", [1, 2])
@pytest.mark.parametrize("queries,keys,width", [(3, 17, 128), (257, 65, 128), (3, 17, 124)])
def test_attention_mask_kat(queries, keys, width, mask_heads):
    for shift in (0, 3):
        q, k, v, row, dense = kat.attention_mask_case(queries, keys, mask_heads, width, shift)
        a = O.sdpa(q, k, v, mask=dense, precise=True)
        b = O.sdpa(q, k, v, mask=row, precise=True)
        np.testing.assert_array_equal(a, b)  # row mask == dense mask, bitwise
        expected = kat.attention_mask_expected(q, k, v, keys, mask_heads, shift)
        assert np.max(np.abs(b - expected)) < 3e-6


def test_attention_accuracy_probe():
    q, k, v, mask, expected, _ = kat.attention_accuracy_case()
    out = O.sdpa(q, k, v, mask=mask, precise=True)
    g = kat.attention_accuracy_gate(out, expected)
    assert g["passed"], g


def test_sdpa_matches_torch_fp64():
    import torch
    q, k, v = O.normal((3, 20, 128), 1), O.normal((3, 33, 128), 2), O.normal((3, 33, 128), 3)
    mask = np.zeros(33, np.float32)
    mask[29:] = -1e30
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).double(), torch.from_numpy(k).double(), torch.from_numpy(v).double(),
        attn_mask=torch.from_numpy(mask).double().expand(20, 33))
    np.testing.assert_allclose(O.sdpa(q, k, v, mask=mask), ref.numpy(), atol=2e-6)
    # The fast (FP32) mode stays within FP32 accumulation error of it.
    np.testing.assert_allclose(O.sdpa(q, k, v, mask=mask, precise=False), ref.numpy(), atol=2e-5)
    # q_range computes only the requested rows.
    part = O.sdpa(q, k, v, mask=mask, q_range=(5, 9))
    np.testing.assert_array_equal(part[:, 5:9], O.sdpa(q, k, v, mask=mask)[:, 5:9])
    assert np.all(part[:, :5] == 0)


# ---- block and heads against PyTorch FP64 library routines ----------------------------------
def small_block(dim=256, ffn=512, seed=0, std=0.02, block=0):
    """One block's weights in .bin order; block b of a stack draws sub-streams 16b + i of the seed."""
    shapes = {"norm1": (dim,), "wq": (dim, dim), "wk": (dim, dim), "wv": (dim, dim), "norm_q": (128,),
              "norm_k": (128,), "wo": (dim, dim), "norm2": (dim,), "w_up": (ffn, dim), "w_gate": (ffn, dim),
              "w_down": (dim, ffn)}
    w = {}
    for i, (name, shape) in enumerate(shapes.items()):
        mean = 1.0 if name.startswith("norm") else 0.0
        w[name] = O.normal(shape, seed, offset=(16 * block + i) << 40, mean=mean, std=std)
    return w


def torch_block_fp64(w, x, mods, cos, sin, mask):
    """tools/export_dit_block.py:49-68 with torch.nn.functional in FP64."""
    import torch
    F = torch.nn.functional
    T = {k: torch.from_numpy(np.asarray(v)).double() for k, v in w.items()}
    x = torch.from_numpy(x).double()
    dim = x.shape[1]
    heads = dim // 128
    sh_sa, sc_sa, g_sa, sh_mlp, sc_mlp, g_mlp = torch.from_numpy(mods).double()
    c, s = torch.from_numpy(cos).double()[:, None], torch.from_numpy(sin).double()[:, None]

    def rotary(t):
        a, b = t[..., :64], t[..., 64:]
        return torch.cat((a * c[..., :64] - b * s[..., :64], b * c[..., 64:] + a * s[..., 64:]), dim=-1)

    h = F.rms_norm(x, (dim,), T["norm1"], 1e-6) * (1.0 + sc_sa) + sh_sa
    q = F.linear(h, T["wq"]).reshape(-1, heads, 128)
    k = F.linear(h, T["wk"]).reshape(-1, heads, 128)
    v = F.linear(h, T["wv"]).reshape(-1, heads, 128)
    q = rotary(F.rms_norm(q, (128,), T["norm_q"], 1e-6)).transpose(0, 1)
    k = rotary(F.rms_norm(k, (128,), T["norm_k"], 1e-6)).transpose(0, 1)
    m = torch.from_numpy(mask).double().expand(x.shape[0], -1)
    a = F.scaled_dot_product_attention(q, k, v.transpose(0, 1), attn_mask=m).transpose(0, 1).reshape(-1, dim)
    x1 = x + g_sa * F.linear(a, T["wo"])
    h2 = F.rms_norm(x1, (dim,), T["norm2"], 1e-6) * (1.0 + sc_mlp) + sh_mlp
    p = F.linear(h2, T["w_up"]) * F.gelu(F.linear(h2, T["w_gate"]), approximate="none")
    return (x1 + g_mlp * F.linear(p, T["w_down"])).numpy()


def small_inputs(S=40, dim=256, image=(4, 8), valid=5, seed=1):
    freqs = O.rope_frequencies()
    w_, h_ = image
    text = S - w_ * h_
    cos, sin, mask = O.dit_constants(freqs, w_, h_, valid, text)
    x = O.normal((S, dim), seed)
    mods = O.normal((6, dim), seed + 100, std=0.5)
    return x, mods, cos, sin, mask


def test_block_matches_torch_fp64():
    w = small_block()
    x, mods, cos, sin, mask = small_inputs()
    out = O.block_forward(w, x, mods, cos, sin, mask)
    ref = torch_block_fp64(w, x, mods, cos, sin, mask)
    m = kat.fp32_block_rule(out, ref)
    assert m["passed"] and m["nrmse"] < 2e-6, m


def test_block_zero_gates_is_identity():
    w = small_block()
    x, mods, cos, sin, mask = small_inputs()
    mods[2] = 0.0
    mods[5] = 0.0
    np.testing.assert_array_equal(O.block_forward(w, x, mods, cos, sin, mask), x)


def test_block_head_permutation_symmetry():
    w = small_block(dim=384)
    x, mods, cos, sin, mask = small_inputs(dim=384)
    perm = [2, 0, 1]
    idx = np.concatenate([np.arange(p * 128, (p + 1) * 128) for p in perm])
    w2 = dict(w)
    for name in ("wq", "wk", "wv"):
        w2[name] = w[name][idx]
    w2["wo"] = w["wo"][:, idx]
    a = O.block_forward(w, x, mods, cos, sin, mask)
    b = O.block_forward(w2, x, mods, cos, sin, mask)
    np.testing.assert_allclose(a, b, rtol=1e-5, atol=1e-5)


def small_heads(dim=256, latent_ch=128, text_dim=3072 // 8, seed=7):
    shapes = {"x_w": (dim, latent_ch), "x_b": (dim,), "text_w": (dim, text_dim), "t1_w": (dim, dim), "t1_b": (dim,),
              "t2_w": (dim, dim), "t2_b": (dim,), "mod_w": (6 * dim, dim), "mod_b": (6 * dim,),
              "out_mod_w": (2 * dim, dim), "out_mod_b": (2 * dim,), "proj_w": (latent_ch, dim),
              "proj_b": (latent_ch,)}
    return {n: O.normal(s, seed, offset=i << 40, std=0.02) for i, (n, s) in enumerate(shapes.items())}


def test_heads_match_torch_fp64():
    import torch
    F = torch.nn.functional
    hw_ = small_heads()
    dim = 256
    latent = O.normal((128, 6, 5), 3)
    text = O.normal((4, 3072 // 8), 4)
    feat = O.timestep_features(500.0)[:dim].copy()
    x, c, mods = O.input_head({k: hw_[k] for k in O.INPUT_HEAD_FIELDS}, latent, text, feat)
    T = {k: torch.from_numpy(v).double() for k, v in hw_.items()}
    lat = torch.from_numpy(latent).double().reshape(128, -1).T
    xr = torch.cat([F.linear(lat, T["x_w"], T["x_b"]), F.linear(torch.from_numpy(text).double(), T["text_w"])])
    cr = F.linear(F.silu(F.linear(torch.from_numpy(feat).double(), T["t1_w"], T["t1_b"])), T["t2_w"], T["t2_b"])
    mr = F.linear(F.silu(cr), T["mod_w"], T["mod_b"]).reshape(6, dim)
    np.testing.assert_allclose(x, xr.numpy(), atol=2e-5, rtol=1e-5)
    np.testing.assert_allclose(c, cr.numpy(), atol=2e-6, rtol=1e-5)
    np.testing.assert_allclose(mods, mr.numpy(), atol=2e-6, rtol=1e-5)
    out_w = {"mod_w": hw_["out_mod_w"], "mod_b": hw_["out_mod_b"], "proj_w": hw_["proj_w"], "proj_b": hw_["proj_b"]}
    pred = O.output_head(out_w, x, c, 30)
    mm = F.linear(torch.from_numpy(c).double(), T["out_mod_w"], T["out_mod_b"])
    y = F.layer_norm(torch.from_numpy(x[:30]).double(), (dim,), eps=1e-6) * (1 + mm[:dim]) + mm[dim:]
    pr = F.linear(y, T["proj_w"], T["proj_b"]).T
    np.testing.assert_allclose(pred, pr.numpy(), atol=2e-5, rtol=1e-5)
