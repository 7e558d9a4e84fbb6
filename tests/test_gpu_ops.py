"""Operator parity on the device: each ernie_hip op against the oracle and the
reference's own known-answer tests (ported in kat.py)."""
import numpy as np
import pytest

import ernie_amd as E
import kat
import oracle as O
from gpu_util import ALL_DT, NAMES, dev, empty, host, stored

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("width", [128, 3072, 4096])
@pytest.mark.parametrize("scale", [1.0, 512.0])
def test_rmsnorm_probe_kat(ctx, dt, width, scale):
    # probes/rmsnorm_probe.cpp: inputs and weights exact in every storage type.
    x, gamma, expected = kat.rmsnorm_kat_case(width, scale)
    xd, out = dev(x, dt), empty(x.shape, dt)
    ctx.rmsnorm(xd, dt, dev(gamma), x.shape[0], width, out, dt)
    err = np.max(np.abs(host(out) - expected))
    assert err <= kat.RMSNORM_LIMITS[NAMES[dt]], err


@pytest.mark.parametrize("scale", [1.0, 1024.0])
def test_layernorm_probe_kat(ctx, scale):
    x, _, expected = kat.rmsnorm_kat_case(4096, scale, centered=True)
    zeros = dev(np.zeros(4096, np.float32))
    out = empty(x.shape)
    ctx.layernorm_modulate(dev(x), zeros, zeros, x.shape[0], 4096, out, E.FP32)
    assert np.max(np.abs(host(out) - expected)) <= kat.RMSNORM_LIMITS["fp32"]


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("shape", [0, 1])
def test_gelu_probe_kat(ctx, dt, shape):
    x = kat.gelu_kat_input(shape)
    xd = dev(x, dt)
    ctx.gelu(xd, dt, x.size)
    err = np.max(np.abs(host(xd) - kat.gelu_expected(x)))
    assert err <= kat.GELU_LIMITS[NAMES[dt]], err


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_residual_contract(ctx, dt):
    # tests/test_residual_contract.cpp: |a| >= 70000 adds exactly in FP32, and the
    # low-storage normalized projection of the sum stays within .001 / .004.
    a, b = kat.residual_case()
    out = empty(a.shape)
    ctx.residual_add(dev(a), E.FP32, dev(b, dt), dt, out, a.size)
    s = host(out)
    np.testing.assert_array_equal(s, (a + b).astype(np.float32))
    norm = empty(a.shape, dt)
    ctx.rmsnorm(out, E.FP32, dev(np.ones(4096, np.float32)), 4, 4096, norm, dt)
    sd = s.astype(np.float64)
    expected = sd / np.sqrt((sd * sd).mean(axis=1, keepdims=True) + 1e-6)
    limit = {E.FP32: 1e-6, E.FP16: 0.001, E.BF16: 0.004}[dt]
    assert np.max(np.abs(host(norm) - expected)) <= limit


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("name,m,n,k,bias", kat.GEMM_KAT_SHAPES)
def test_gemm_exact_products_kat(ctx, dt, name, m, n, k, bias):
    # tests/test_bf16_gemm.cpp: multiples of 1/8, exact FP32 products and sums;
    # the low-precision result must equal round-to-nearest-even of the FP64 sum.
    a, w, b = kat.gemm_kat_case(m, n, k)
    ref = a.astype(np.float64) @ w.astype(np.float64).T + (b.astype(np.float64) if bias else 0.0)
    ad, wd = dev(a, dt), dev(w, dt)
    bd = dev(b) if bias else None
    c32 = empty((m, n))
    ctx.gemm(ad, k, wd, k, c32, n, m, n, k, dt, E.FP32, bias=bd)
    np.testing.assert_array_equal(host(c32).astype(np.float64), ref)
    if dt != E.FP32:
        c16 = empty((m, n), dt)
        ctx.gemm(ad, k, wd, k, c16, n, m, n, k, dt, dt, bias=bd)
        np.testing.assert_array_equal(host(c16), stored(ref.astype(np.float32), dt))


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("m,n,k", [(300, 520, 256), (4160, 256, 512), (33, 4096, 128), (1056, 96, 4096),
                                   (4160, 4096, 256), (4120, 4096, 256)])
def test_gemm_random_against_oracle(ctx, dt, m, n, k):
    # 4160 / 4120 x 4096: 256 full tiles and a 64- or 24-row tail row; the 16-bit kernel
    # computes the tail in 16-row chunks inside full tiles (light tiles), one per
    # workgroup at most.
    a = O.normal((m, k), 1)
    w = O.normal((n, k), 2, std=0.02)
    a_s, w_s = stored(a, dt), stored(w, dt)
    ref = O.gemm_nt(a_s, w_s).astype(np.float64)
    c = empty((m, n))
    ctx.gemm(dev(a, dt), k, dev(w, dt), k, c, n, m, n, k, dt, E.FP32)
    g = kat.gate(host(c), ref, 0, 1e-5, 1e-5)
    assert g["passed"], g


def test_gemm_rejects_unsupported_shapes(ctx):
    a, c = empty((4, 40), E.FP16), empty((4, 8))
    with pytest.raises(E.ErnieError):
        ctx.gemm(a, 40, a, 40, c, 8, 4, 8, 40, E.FP16, E.FP32)  # K % 32 != 0


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("mask_heads", [1, 2])
@pytest.mark.parametrize("queries,keys,width", [(3, 17, 128), (257, 65, 128), (3, 17, 124)])
def test_attention_mask_kat(ctx, dt, queries, keys, width, mask_heads):
    # tests/test_attention_mask.cpp: row mask == dense mask bitwise, repeated
    # runs identical, FP32 against FP64 with the mask as a visible-key count.
    heads = 2
    for shift in (0, 3):
        q, k, v, row, dense = kat.attention_mask_case(queries, keys, mask_heads, width, shift)
        qd, kd, vd = dev(q, dt), dev(k, dt), dev(v, dt)
        strides = (queries * width, width, keys * width, width, keys * width, width, queries * width, width)
        outs = []
        for rep, mask in enumerate((dense, row, row)):
            o = empty((heads, queries, width), dt)
            ctx.sdpa(qd, kd, vd, o, dt, heads, 1, queries, keys, width, strides, mask=dev(mask),
                     mask_heads=mask_heads, mask_rows=mask.shape[1])
            outs.append(host(o))
        np.testing.assert_array_equal(outs[0], outs[1])
        np.testing.assert_array_equal(outs[1], outs[2])
        expected = kat.attention_mask_expected(stored(q, dt), stored(k, dt), stored(v, dt), keys, mask_heads, shift)
        limit = {E.FP32: 3e-6, E.FP16: 4e-3, E.BF16: 3e-2}[dt]
        assert np.max(np.abs(outs[1] - expected)) < limit


def test_attention_accuracy_probe(ctx):
    # probes/attention_accuracy_probe.cpp: 4160 keys (4128 visible); a constant V
    # column must stay 1 within 5e-7; max error 3e-6 and nrmse 5e-7 vs FP64.
    q, k, v, mask, expected, _ = kat.attention_accuracy_case()
    H, Sq, d = q.shape
    Sk = k.shape[1]
    o = empty(q.shape)
    strides = (Sq * d, d, Sk * d, d, Sk * d, d, Sq * d, d)
    ctx.sdpa(dev(q), dev(k), dev(v), o, E.FP32, H, H, Sq, Sk, d, strides, mask=dev(mask), mask_heads=1,
             mask_rows=Sq)
    g = kat.attention_accuracy_gate(host(o), expected)
    assert g["passed"], g


@pytest.mark.parametrize("dt", [E.FP32, E.FP16, E.BF16], ids=lambda d: NAMES[d])
def test_sdpa_full_size_rows_against_oracle(ctx, dt):
    # SDPA alone at S=4160, 32 heads x 128, last 24 text keys padded; token-major
    # [S][4096] layout as the block uses it. Rows checked: the first query tile,
    # a middle one and the partial last tile, all heads.
    S, H, d, valid = 4160, 32, 128, 4136
    q = O.normal((S, H * d), 2)
    k = O.normal((S, H * d), 3)
    v = O.normal((S, H * d), 4)
    qd, kd, vd = dev(q, dt), dev(k, dt), dev(v, dt)
    o = empty((S, H * d), dt)
    strides = (d, H * d, d, H * d, d, H * d, d, H * d)
    ctx.sdpa(qd, kd, vd, o, dt, H, H, S, S, d, strides, valid_keys=valid)
    out = host(o).reshape(S, H, d).transpose(1, 0, 2)
    qs, ks, vs = (stored(t, dt).reshape(S, H, d).transpose(1, 0, 2).copy() for t in (q, k, v))
    mask = np.zeros(S, np.float32)
    mask[valid:] = -1e30
    # Rows 2240..2303 are the last two waves of their 128-query workgroup.
    for r0, r1 in ((0, 64), (2048, 2112), (2240, 2304), (4096, 4160)):
        ref = O.sdpa(qs, ks, vs, mask=mask, q_range=(r0, r1))[:, r0:r1]
        got = out[:, r0:r1]
        if dt == E.FP32:
            m = kat.fp32_block_rule(got, ref)
            assert m["passed"] and m["nrmse"] < 1e-6, m
        else:
            g = kat.gate(got, ref, *kat.BLOCK_GATES[NAMES[dt]])
            assert g["passed"], g


@pytest.mark.parametrize("dt", [E.FP16, E.BF16], ids=lambda d: NAMES[d])
@pytest.mark.parametrize("S,H,valid", [(256, 2, 256), (512, 3, 500), (1280, 2, 1270), (456, 2, 456), (300, 1, 290),
                                         (1088, 2, 1060)])
def test_sdpa_full_tiles_and_remainder(ctx, dt, S, H, valid):
    # Unmasked attention at lengths around the kernel's workgroup tiles: whole
    # 256-query tiles (the 8-wave form: 256, 512, 1280), 128-query tiles with a partial
    # last tile of 72 / 44 / 64 queries (split along the keys into parts that a second
    # launch merges; its waves past the last query only load and keep the barriers),
    # and valid-key counts that are not multiples of 64. Every row of every head is
    # compared with the oracle.
    d = 128
    q = O.normal((S, H * d), 21)
    k = O.normal((S, H * d), 22)
    v = O.normal((S, H * d), 23)
    o = empty((S, H * d), dt)
    strides = (d, H * d, d, H * d, d, H * d, d, H * d)
    ctx.sdpa(dev(q, dt), dev(k, dt), dev(v, dt), o, dt, H, H, S, S, d, strides, valid_keys=valid)
    out = host(o).reshape(S, H, d).transpose(1, 0, 2)
    qs, ks, vs = (stored(t, dt).reshape(S, H, d).transpose(1, 0, 2).copy() for t in (q, k, v))
    mask = np.zeros(S, np.float32)
    mask[valid:] = -1e30
    ref = O.sdpa(qs, ks, vs, mask=mask)
    g = kat.gate(out, ref, *kat.BLOCK_GATES[NAMES[dt]])
    assert g["passed"], g


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_qk_norm_rope_against_oracle(ctx, dt):
    S, H = 70, 3
    x = O.normal((S, 3 * H * 128), 5)
    gamma = O.normal((128,), 6, mean=1.0, std=0.1)
    ang = O.normal((S, 128), 7)
    cos, sin = np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)
    xd = dev(x, dt)
    ctx.qk_norm_rope(xd, dt, S, H, 3 * H * 128, dev(gamma), dev(cos), dev(sin))
    got = host(xd)
    xs = stored(x, dt)
    ref = xs.copy()
    for h in range(H):
        sl = xs[:, h * 128:(h + 1) * 128]
        ref[:, h * 128:(h + 1) * 128] = O.rope_rows(O.rmsnorm(sl, gamma), cos, sin)
    tol = {E.FP32: 2e-6, E.FP16: 4e-3, E.BF16: 3e-2}[dt]
    assert np.max(np.abs(got - ref)) <= tol * max(1.0, float(np.abs(ref).max()))
    # Columns outside the first H heads (the V block) are untouched.
    np.testing.assert_array_equal(got[:, H * 128:], xs[:, H * 128:])


@pytest.mark.slow
@pytest.mark.parametrize("dt", [E.FP32, E.FP16, E.BF16], ids=lambda d: NAMES[d])
def test_sdpa_config1_every_row_against_oracle(ctx, dt):
    # The standalone SDPA workload at full size: 32 heads x 128, S = 4160 (4096 image
    # tokens + a 64-token text bucket whose last 24 keys are padding), Q/K/V ~ N(0,1), scale
    # 1/sqrt(128), head-major [32][S][128]. Every query row of every head is compared with
    # the oracle (FP64 sums), so the full query tiles, both rounds of them and the key-split
    # partial last tile are all covered.
    S, H, d, valid = 4160, 32, 128, 4136
    q = O.normal((H, S, d), 2)
    k = O.normal((H, S, d), 3)
    v = O.normal((H, S, d), 4)
    o = empty((H, S, d), dt)
    strides = (S * d, d, S * d, d, S * d, d, S * d, d)
    ctx.sdpa(dev(q, dt), dev(k, dt), dev(v, dt), o, dt, H, H, S, S, d, strides, valid_keys=valid)
    got = host(o)
    mask = np.zeros(S, np.float32)
    mask[valid:] = -1e30
    ref = O.sdpa(stored(q, dt), stored(k, dt), stored(v, dt), mask=mask)
    if dt == E.FP32:
        m = kat.fp32_block_rule(got, ref)
        assert m["passed"] and m["nrmse"] < 1e-6, m
    else:
        g = kat.gate(got, ref, *kat.BLOCK_GATES[NAMES[dt]])
        assert g["passed"], g
        # Per-row error bound as well (the gate's atol + rtol max|ref|), so that a few wrong
        # rows cannot hide in the norm.
        atol, rtol, _ = kat.BLOCK_GATES[NAMES[dt]]
        row_err = np.abs(got - ref).max(axis=2)
        assert float(row_err.max()) <= atol + rtol * float(np.abs(ref).max()), float(row_err.max())


def test_euler_and_finite_contracts(ctx):
    # src/latent_ops.cpp:72-92 and tests/test_latent_contract.cpp.
    x = O.normal((128, 5, 3), 9)
    v = O.normal((128, 5, 3), 10)
    xd, vd, out = dev(x), dev(v), empty(x.shape)
    # Each delta of the 8-step turbo schedule (none a power of two): x + (delta * v) rounded
    # twice, bitwise the oracle's -ffp-contract=off product and sum. A fused multiply-add
    # (one rounding) gives different bits for some elements at these deltas, so the test
    # sees a contraction.
    sig, _ = O.flow_schedule_turbo(8)
    contraction_visible = False
    for i in range(8):
        delta = np.float32(sig[i + 1] - sig[i])
        ctx.euler_step(xd, vd, float(delta), x.size, out)
        ref = O.euler_step(x, v, delta)
        np.testing.assert_array_equal(host(out), ref)
        fused = (x.astype(np.float64) + np.float64(delta) * v.astype(np.float64)).astype(np.float32)
        contraction_visible |= bool(np.any(fused != ref))
    assert contraction_visible
    ctx.euler_step(xd, vd, -0.0625, x.size, out)
    np.testing.assert_array_equal(host(out), O.euler_step(x, v, -0.0625))
    for bad in (0.0, 0.5, -1.5, float("nan")):
        with pytest.raises(E.ErnieError):
            ctx.euler_step(xd, vd, bad, x.size, out)
    ones = dev(np.ones((128, 15), np.float32))
    ctx.euler_step(ones, ones, -1.0, 128 * 15, ones)  # aliased consume-and-replace
    assert np.all(host(ones) == 0.0)
    assert ctx.finite(xd, x.size)
    for bad in (float("inf"), float("nan")):
        y = x.copy()
        y[42, 2, 1] = bad
        assert not ctx.finite(dev(y), y.size)


def test_query_rows_compatibility(ctx):
    for rows in (128, 64, 32, 16):
        ctx.call("set_attention_query_rows", rows)
    with pytest.raises(E.ErnieError):
        ctx.call("set_attention_query_rows", 48)
    assert ctx.L.ernie_hip_attention_internal_submissions(ctx.ctx) == 0
