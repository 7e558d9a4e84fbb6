"""Mistral text path on the device: the causal GQA attention probe, rotary-only
Q/K, one text block at the reference's width (hidden 3072, 32 heads over 8 K/V
heads, ffn 9216) and a block sequence through the C ABI and the facade, against
the oracle under the reference's text gates (tools/validate_text.py:53-54)."""
import numpy as np
import pytest

import ernie_amd as E
import kat
import oracle as O
from gpu_util import ALL_DT, NAMES, dev, empty, host, stored
from test_text_cpu import small_text_block, yarn_like_frequencies

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("length", [32, 65, 200])
def test_gqa_causal_attention_probe(ctx, dt, length):
    # probes/attention_probe.cpp: 32 query heads over 8 K/V heads, causal -1e30 mask,
    # against the FP64 visible-key oracle, under the probe's operator gates.
    q, k, v, mask = kat.gqa_causal_case(length, 11)
    d = 128
    o = empty(q.shape, dt)
    strides = (length * d, d, length * d, d, length * d, d, length * d, d)
    ctx.sdpa(dev(q, dt), dev(k, dt), dev(v, dt), o, dt, 32, 8, length, length, d, strides, mask=dev(mask),
             mask_heads=1, mask_rows=length)
    got = host(o)
    ref = kat.gqa_causal_expected(stored(q, dt), stored(k, dt), stored(v, dt))
    m = kat.metrics(got, ref)
    atol, nrmse = kat.GQA_PROBE_LIMITS[NAMES[dt]]
    assert m["finite"] and m["max_abs_error"] <= atol and m["nrmse"] <= nrmse, m
    # The same attention applied by position (no mask tensor; tiles above the diagonal skipped).
    o2 = empty(q.shape, dt)
    ctx.sdpa_causal(dev(q, dt), dev(k, dt), dev(v, dt), o2, dt, 32, 8, length, length, d, strides)
    m2 = kat.metrics(host(o2), ref)
    assert m2["finite"] and m2["max_abs_error"] <= atol and m2["nrmse"] <= nrmse, m2


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_gqa_causal_queries_after_a_prefix(ctx, dt):
    # The probe's growth case (probes/attention_probe.cpp:326): queries at positions
    # 34..64 over all 65 keys, key k visible iff k <= q + (sk - sq).
    sk, sq, d = 65, 31, 128
    q, k, v, _ = kat.gqa_causal_case(sk, 83)
    ref = kat.gqa_causal_expected(stored(q, dt), stored(k, dt), stored(v, dt))[:, sk - sq:]
    qt = np.ascontiguousarray(q[:, sk - sq:])
    o = empty(qt.shape, dt)
    strides = (sq * d, d, sk * d, d, sk * d, d, sq * d, d)
    ctx.sdpa_causal(dev(qt, dt), dev(k, dt), dev(v, dt), o, dt, 32, 8, sq, sk, d, strides)
    m = kat.metrics(host(o), ref)
    atol, nrmse = kat.GQA_PROBE_LIMITS[NAMES[dt]]
    assert m["finite"] and m["max_abs_error"] <= atol and m["nrmse"] <= nrmse, m


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_rotary_only_matches_oracle(ctx, dt):
    # Text q/k path (text-s64.ncnn.param lines 18-44): rotary without a norm, gamma NULL.
    S, heads = 40, 5
    cos, sin, _ = O.text_constants(yarn_like_frequencies(), S)
    x = O.normal((S, heads * 128), 3)
    xd = dev(x, dt)
    ctx.qk_norm_rope(xd, dt, S, heads, heads * 128, None, dev(cos), dev(sin))
    got = host(xd)
    base = stored(x, dt)
    ref = np.concatenate([O.rope_rows(base[:, h * 128:(h + 1) * 128], cos, sin) for h in range(heads)], axis=1)
    limit = {E.FP32: 1e-6, E.FP16: 4e-3, E.BF16: 3e-2}[dt]
    assert np.max(np.abs(got - ref)) <= limit * max(1.0, np.max(np.abs(ref)))


def run_text_block(ctx, index, x, cos, sin, mask, causal=False):
    S, hidden = x.shape
    out = empty((S, hidden))
    ctx.text_block_forward(index, dev(x), out, dev(cos), dev(sin), S, mask=None if mask is None else dev(mask),
                           causal=causal)
    return host(out)


@pytest.fixture(scope="module")
def full_text_block():
    # The reference text block's shape: hidden 3072, 32 heads x 128 over 8 K/V heads,
    # ffn 9216; weights N(0, 0.02), gammas 1 + N(0, 0.02).
    return small_text_block(seed=40, hidden=3072, heads=32, kv_heads=8, ffn=9216, std=0.02)


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("S", [64, 33, 2048])
def test_text_block_full_width_against_oracle(ctx, full_text_block, dt, S):
    # S = 64 is a reference text bucket (tests/fixtures/text-s64.ncnn.param); 33 leaves
    # a ragged key tile; at 2048 the up/gate GEMM has 8 x 72 = 576 tiles, so its last
    # 64 run split along K, and the o_proj / down GEMMs split every tile. x ~ 0.2 N(0, 1)
    # as tools/export_text_block.py:74.
    w = full_text_block
    ctx.text_block_upload(3, w, 3072, 32, 8, 9216, dt)
    cos, sin, mask = O.text_constants(yarn_like_frequencies(), S)
    x = O.normal((S, 3072), 41, std=0.2)
    got = run_text_block(ctx, 3, x, cos, sin, mask)
    ref = O.text_block_forward(w, x, cos, sin, mask, 32, 8)
    g = kat.gate(got, ref, *kat.TEXT_GATES[NAMES[dt]])
    assert g["passed"], g
    if dt == E.FP32:
        m = kat.fp32_block_rule(got, ref)
        assert m["passed"], m
    np.testing.assert_array_equal(run_text_block(ctx, 3, x, cos, sin, mask), got)  # repeat-deterministic
    # Causal by position instead of the mask tensor.
    gc = kat.gate(run_text_block(ctx, 3, x, cos, sin, None, causal=True), ref, *kat.TEXT_GATES[NAMES[dt]])
    assert gc["passed"], gc
    ctx.call("text_block_release", 3)


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_text_block_ragged_tiles_against_oracle(ctx, dt):
    # 300 tokens: a partial 256-row GEMM tile (split-K tail) and a partial 128-query
    # attention tile (key-range split), at a narrower width.
    hidden, heads, kv, ffn, S = 512, 8, 2, 1024, 300
    w = small_text_block(seed=44, hidden=hidden, heads=heads, kv_heads=kv, ffn=ffn)
    ctx.text_block_upload(4, w, hidden, heads, kv, ffn, dt)
    cos, sin, mask = O.text_constants(yarn_like_frequencies(), S)
    x = O.normal((S, hidden), 45, std=0.2)
    got = run_text_block(ctx, 4, x, cos, sin, None, causal=True)
    ref = O.text_block_forward(w, x, cos, sin, mask, heads, kv)
    g = kat.gate(got, ref, *kat.TEXT_GATES[NAMES[dt]])
    assert g["passed"], g
    ctx.call("text_block_release", 4)


def test_text_sequence_and_facade_against_oracle(ctx):
    # Three blocks (run_text_blocks, src/text_encoder.cpp:119-180) at FP16, chained
    # through the C ABI and through the facade, against the chained oracle.
    hidden, heads, kv, ffn, S = 512, 8, 2, 1024, 64
    ws = [small_text_block(seed=50 + i, hidden=hidden, heads=heads, kv_heads=kv, ffn=ffn) for i in range(3)]
    fac = E.Facade(0)
    try:
        for i, w in enumerate(ws):
            fac.hip.text_block_upload(10 + i, w, hidden, heads, kv, ffn, E.FP16)
        cos, sin, mask = O.text_constants(yarn_like_frequencies(), S)
        x = O.normal((S, hidden), 51, std=0.2)
        ref = x
        for w in ws:
            ref = O.text_block_forward(w, ref, cos, sin, mask, heads, kv)
        xd, cd, sd, md = dev(x), dev(cos), dev(sin), dev(mask)
        out = empty((S, hidden))
        secs = fac.hip.text_block_sequence([10, 11, 12], xd, out, cd, sd, S, mask=md, timing=True)
        got = host(out)
        assert np.all(secs > 0)
        g = kat.gate(got, ref, *kat.TEXT_GATES["fp16"])
        assert g["passed"], g
        out2 = empty((S, hidden))
        fac.run_text_blocks([10, 11, 12], xd, S, hidden, cd, sd, md, out2, dtype=E.FP16)
        np.testing.assert_array_equal(host(out2), got)
        # The facade's causal mask (as upload_text_constants marks it) runs by position.
        fac.hip.text_block_sequence([10, 11, 12], xd, out, cd, sd, S, causal=True)
        fac.run_text_blocks([10, 11, 12], xd, S, hidden, cd, sd, md, out2, dtype=E.FP16, causal=True)
        np.testing.assert_array_equal(host(out2), host(out))
        gc = kat.gate(host(out), ref, *kat.TEXT_GATES["fp16"])
        assert gc["passed"], gc
        # src/text_encoder.cpp:41-45: 1..25 blocks and exactly the three constants.
        with pytest.raises(E.ErnieInvalidRequest):
            fac.run_text_blocks([], xd, S, hidden, cd, sd, md, out2, dtype=E.FP16)
        with pytest.raises(E.ErnieInvalidRequest):
            fac.run_text_blocks([10] * 26, xd, S, hidden, cd, sd, md, out2, dtype=E.FP16)
        with pytest.raises(E.ErnieError):
            fac.hip.text_block_sequence([10, 13], xd, out, cd, sd, S, mask=md)  # slot 13 not loaded
    finally:
        fac.close()
