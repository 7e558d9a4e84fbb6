"""Block, sequence, heads, DiT and denoise parity on the device against the
oracle, under the reference's own per-precision gates (kat.py)."""
import numpy as np
import pytest

import ernie_amd as E
import kat
import oracle as O
from gpu_util import ALL_DT, NAMES, dev, empty, host
from test_oracle import small_block, small_heads, small_inputs

pytestmark = pytest.mark.gpu

BLOCK_FIELDS = O.BLOCK_FIELDS


def run_block(ctx, index, x, mods, cos, sin, mask, valid):
    S, dim = x.shape
    xd, out = dev(x), empty((S, dim))
    ctx.block_forward(index, xd, out, dev(mods), dev(cos), dev(sin), S, mask=dev(mask), valid_keys=valid)
    return host(out)


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_block_small_against_oracle(ctx, dt):
    w = small_block(dim=256, ffn=512)
    x, mods, cos, sin, mask = small_inputs(S=40, dim=256)
    ctx.block_upload(0, w, 256, 512, dt)
    valid = int(np.sum(mask == 0))
    got = run_block(ctx, 0, x, mods, cos, sin, mask, valid)
    ref = O.block_forward(w, x, mods, cos, sin, mask)
    g = kat.gate(got, ref, *kat.BLOCK_GATES[NAMES[dt]])
    assert g["passed"], g
    if dt == E.FP32:
        assert kat.fp32_block_rule(got, ref)["passed"]
    # The mask alone (valid_keys = 0) and the count alone give the same block.
    again = run_block(ctx, 0, x, mods, cos, sin, mask, 0)
    g2 = kat.gate(again, ref, *kat.BLOCK_GATES[NAMES[dt]])
    assert g2["passed"], g2


@pytest.mark.parametrize("dt", [E.FP16, E.BF16], ids=lambda d: NAMES[d])
def test_block_last_round_split_against_oracle(ctx, dt):
    # Width 1024 (8 heads), FFN 4096, S = 2368 = 9 x 256 + 64 (48 x 44 image tokens,
    # 256 text slots, 200 valid). The up/gate GEMM has 9 x 32 = 288 full 256 x 256
    # tiles, 32 more than one round of 256 workgroups: those 32 are split along K,
    # next to the split 64-row tail row. The narrower projections split every tile.
    dim, ffn = 1024, 4096
    w = small_block(dim=dim, ffn=ffn, seed=7)
    x, mods, cos, sin, mask = small_inputs(S=2368, dim=dim, image=(48, 44), valid=200, seed=8)
    ctx.block_upload(5, w, dim, ffn, dt)
    valid = int(np.sum(mask == 0))
    got = run_block(ctx, 5, x, mods, cos, sin, mask, valid)
    ref = O.block_forward(w, x, mods, cos, sin, mask)
    g = kat.gate(got, ref, *kat.BLOCK_GATES[NAMES[dt]])
    assert g["passed"], g
    np.testing.assert_array_equal(run_block(ctx, 5, x, mods, cos, sin, mask, valid), got)  # repeat-deterministic
    ctx.call("block_release", 5)


@pytest.mark.parametrize("dt", [E.FP16, E.BF16], ids=lambda d: NAMES[d])
def test_block_heavy_tail_tiles_against_oracle(ctx, dt):
    # Width 1024 (8 heads), FFN 4096, S = 5160 = 20 x 256 + 40 (64 x 80 image tokens,
    # 40 text slots, 30 valid). The up/gate GEMM has 20 x 32 = 640 full tiles, two and a
    # half rounds of 256 workgroups, so its last row of tiles takes the 40 tail rows as
    # 320-row tiles (rows past S are computed and not stored) instead of a split tail
    # row; the other GEMMs have too few tiles for that and keep their split tails.
    dim, ffn = 1024, 4096
    w = small_block(dim=dim, ffn=ffn, seed=11)
    x, mods, cos, sin, mask = small_inputs(S=5160, dim=dim, image=(64, 80), valid=30, seed=12)
    ctx.block_upload(6, w, dim, ffn, dt)
    valid = int(np.sum(mask == 0))
    got = run_block(ctx, 6, x, mods, cos, sin, mask, valid)
    ref = O.block_forward(w, x, mods, cos, sin, mask)
    g = kat.gate(got, ref, *kat.BLOCK_GATES[NAMES[dt]])
    assert g["passed"], g
    np.testing.assert_array_equal(run_block(ctx, 6, x, mods, cos, sin, mask, valid), got)  # repeat-deterministic
    ctx.call("block_release", 6)


@pytest.mark.parametrize("ffn", [2048, 4096])
@pytest.mark.parametrize("dt", [E.FP16, E.BF16], ids=lambda d: NAMES[d])
def test_block_light_tail_tiles_against_oracle(ctx, dt, ffn):
    # Width 1024, S = 4136 = 16 x 256 + 40. FFN 2048: the up/gate GEMM has 16 x 16 = 256
    # full tiles, one round, and the 40 tail rows go as three 16-row chunks (the last one
    # 8 rows past S) into 48 of those tiles. FFN 4096: 512 full tiles, two rounds, and
    # the tail goes as two 32-row chunks (24 rows past S) into 64 tiles. Either way at
    # most one chunk per workgroup, with the GEGLU epilogue applied to each chunk in the
    # tile that computed it.
    dim = 1024
    w = small_block(dim=dim, ffn=ffn, seed=13)
    x, mods, cos, sin, mask = small_inputs(S=4136, dim=dim, image=(64, 64), valid=30, seed=14)
    ctx.block_upload(7, w, dim, ffn, dt)
    valid = int(np.sum(mask == 0))
    got = run_block(ctx, 7, x, mods, cos, sin, mask, valid)
    ref = O.block_forward(w, x, mods, cos, sin, mask)
    g = kat.gate(got, ref, *kat.BLOCK_GATES[NAMES[dt]])
    assert g["passed"], g
    np.testing.assert_array_equal(run_block(ctx, 7, x, mods, cos, sin, mask, valid), got)  # repeat-deterministic
    ctx.call("block_release", 7)


_CONFIG0_MODS = []


def config0_modulations():
    """Time MLP + adaLN of synthetic heads (N(0, 0.02), seed 0) on timestep_features(500)."""
    if not _CONFIG0_MODS:
        heads = small_heads(dim=4096, latent_ch=128, text_dim=3072, seed=0)
        # Only the time path matters here; one latent token and no text rows.
        _, c, mods = O.input_head({k: heads[k] for k in O.INPUT_HEAD_FIELDS}, np.zeros((128, 1, 1), np.float32),
                                  np.zeros((0, 3072), np.float32), O.timestep_features(500.0))
        assert np.isfinite(mods).all() and float(np.abs(mods).max()) > 0
        _CONFIG0_MODS.append(mods)
    return _CONFIG0_MODS[0]


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_block_config0_against_oracle(ctx, dt):
    # One ERNIE block at full width (4096, 32 heads, FFN 12288), S = 1056
    # (32x32 image tokens + 32 text tokens, all valid), weights N(0, 0.02) from seed 0,
    # x N(0, 1) from seed 1. The six modulations come from the input head's time MLP
    # (4096 -> 4096, SiLU, 4096 -> 4096, SiLU, 4096 -> 6 x 4096;
    # heads/input/head.ncnn.param lines 9-17) on timestep_features(500), t = 0.5.
    dim, ffn = 4096, 12288
    w = small_block(dim=dim, ffn=ffn, seed=0)
    x, _, cos, sin, mask = small_inputs(S=1056, dim=dim, image=(32, 32), valid=32, seed=1)
    mods = config0_modulations()
    ctx.block_upload(1, w, dim, ffn, dt)
    got = run_block(ctx, 1, x, mods, cos, sin, mask, 1056)
    ref = O.block_forward(w, x, mods, cos, sin, mask)
    g = kat.gate(got, ref, *kat.BLOCK_GATES[NAMES[dt]])
    assert g["passed"], g
    if dt == E.FP32:
        m = kat.fp32_block_rule(got, ref)
        assert m["passed"], m
    # Repeat-determinism (probes/block_runner.cpp:196-203): bitwise identical.
    np.testing.assert_array_equal(run_block(ctx, 1, x, mods, cos, sin, mask, 1056), got)
    ctx.call("block_release", 1)


def test_block_zero_gates_is_identity_full_size(ctx):
    # S = 4160 fp16 (the 1024x1024 token count); gate_sa = gate_mlp = 0 leaves x untouched.
    S, dim, ffn = 4160, 4096, 12288
    ctx.block_init_random(2, dim, ffn, E.FP16, seed=5)
    x = O.normal((S, dim), 3)
    mods = O.normal((6, dim), 4, std=0.5)
    mods[2] = 0.0
    mods[5] = 0.0
    freqs = O.rope_frequencies()
    cos, sin, mask = O.dit_constants(freqs, 64, 64, 40, 64)
    got = run_block(ctx, 2, x, mods, cos, sin, mask, 4136)
    np.testing.assert_array_equal(got, x)
    # With gates on, the output is finite, deterministic and differs from x.
    mods = O.normal((6, dim), 4, std=0.5)
    a = run_block(ctx, 2, x, mods, cos, sin, mask, 4136)
    b = run_block(ctx, 2, x, mods, cos, sin, mask, 4136)
    assert np.isfinite(a).all() and not np.array_equal(a, x)
    np.testing.assert_array_equal(a, b)
    ctx.call("block_release", 2)


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_block_sequence_against_oracle(ctx, dt):
    dim, ffn = 256, 512
    ws = [small_block(dim, ffn, seed=10 + i) for i in range(3)]
    for i, w in enumerate(ws):
        ctx.block_upload(10 + i, w, dim, ffn, dt)
    x, mods, cos, sin, mask = small_inputs(S=40, dim=dim)
    valid = int(np.sum(mask == 0))
    xd, out = dev(x), empty(x.shape)
    secs = ctx.block_sequence([10, 11, 12], xd, out, dev(mods), dev(cos), dev(sin), 40, mask=dev(mask),
                              valid_keys=valid, timing=True)
    assert secs.shape == (3,) and np.all(secs > 0)
    ref = x
    for w in ws:
        ref = O.block_forward(w, ref, mods, cos, sin, mask)
    g = kat.gate(host(out), ref, *kat.SEQUENCE_GATES[NAMES[dt]])
    assert g["passed"], g


def test_block_call_validation(ctx):
    x = empty((8, 256))
    with pytest.raises(E.ErnieError):
        ctx.block_forward(999, x, x, x, x, x, 8)  # not loaded
    with pytest.raises(E.ErnieError):
        ctx.block_sequence([], x, x, x, x, x, 8)
    with pytest.raises(E.ErnieError):
        ctx.block_init_random(3, 200, 512, E.FP16, 1)  # width not a multiple of 128


def heads_for(dim):
    return small_heads(dim=dim, latent_ch=128, text_dim=3072)


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_heads_against_oracle(ctx, dt):
    dim = 256
    hw_ = heads_for(dim)
    ctx.heads_upload(hw_, dim, 128, 3072, dt)
    latent = O.normal((128, 6, 5), 3)
    text = O.normal((8, 3072), 4)
    feat = O.timestep_features(500.0)[:dim].copy()
    S = 30 + 8
    x, c, mods = empty((S, dim)), empty((dim,)), empty((6, dim))
    ctx.input_head(dev(latent), 30, dev(text), 8, dev(feat), x, c, mods)
    xr, cr, mr = O.input_head({k: hw_[k] for k in O.INPUT_HEAD_FIELDS}, latent, text, feat)
    gates = kat.HEAD_GATES[NAMES[dt]]
    for got, ref in ((x, xr), (c, cr), (mods, mr)):
        g = kat.gate(host(got), ref, *gates)
        assert g["passed"], g
    pred = empty((128, 30))
    ctx.output_head(dev(xr), S, 30, dev(cr), pred)
    out_w = {"mod_w": hw_["out_mod_w"], "mod_b": hw_["out_mod_b"], "proj_w": hw_["proj_w"], "proj_b": hw_["proj_b"]}
    g = kat.gate(host(pred), O.output_head(out_w, xr, cr, 30), *gates)
    assert g["passed"], g


@pytest.mark.parametrize("dt", [E.FP16, E.BF16], ids=lambda d: NAMES[d])
def test_heads_full_size_against_oracle(ctx, dt):
    # The 1024x1024 heads: 64x64 latent tokens and 64 text rows at width 4096. The
    # 4096 -> 128 output projection has 16 tiles and splits every tile along K; the
    # 64 text rows are one split partial row of tiles; the time MLP and both adaLN
    # projections run in the four-row GEMV.
    dim = 4096
    hw_ = heads_for(dim)
    ctx.heads_upload(hw_, dim, 128, 3072, dt)
    latent = O.normal((128, 64, 64), 13)
    text = O.normal((64, 3072), 14)
    feat = O.timestep_features(875.0)[:dim].copy()
    S = 4096 + 64
    x, c, mods = empty((S, dim)), empty((dim,)), empty((6, dim))
    ctx.input_head(dev(latent), 4096, dev(text), 64, dev(feat), x, c, mods)
    xr, cr, mr = O.input_head({k: hw_[k] for k in O.INPUT_HEAD_FIELDS}, latent, text, feat)
    gates = kat.HEAD_GATES[NAMES[dt]]
    for got, ref in ((x, xr), (c, cr), (mods, mr)):
        g = kat.gate(host(got), ref, *gates)
        assert g["passed"], g
    pred = empty((128, 4096))
    ctx.output_head(dev(xr), S, 4096, dev(cr), pred)
    out_w = {"mod_w": hw_["out_mod_w"], "mod_b": hw_["out_mod_b"], "proj_w": hw_["proj_w"], "proj_b": hw_["proj_b"]}
    g = kat.gate(host(pred), O.output_head(out_w, xr, cr, 4096), *gates)
    assert g["passed"], g


def oracle_dit(blocks_w, heads_w, latent, text, feat, cos, sin, mask):
    x, c, mods = O.input_head({k: heads_w[k] for k in O.INPUT_HEAD_FIELDS}, latent, text, feat)
    for w in blocks_w:
        x = O.block_forward(w, x, mods, cos, sin, mask)
    out_w = {"mod_w": heads_w["out_mod_w"], "mod_b": heads_w["out_mod_b"], "proj_w": heads_w["proj_w"],
             "proj_b": heads_w["proj_b"]}
    hw = latent[0].size
    return O.output_head(out_w, x, c, hw).reshape(latent.shape)


def dit_setup(ctx, dt, nblocks=2, dim=256, ffn=512, grid=(4, 4), text=8, valid=5):
    hw_ = heads_for(dim)
    ctx.heads_upload(hw_, dim, 128, 3072, dt)
    ws = [small_block(dim, ffn, seed=20 + i) for i in range(nblocks)]
    for i, w in enumerate(ws):
        ctx.block_upload(20 + i, w, dim, ffn, dt)
    H, W = grid
    latent = O.normal((128, H, W), 31)
    tx = O.normal((text, 3072), 32)
    tx[valid:] = 0.0  # pad_text zero rows
    cos, sin, mask = O.dit_constants(O.rope_frequencies(), W, H, valid, text)
    return hw_, ws, latent, tx, cos, sin, mask


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_dit_forward_against_oracle(ctx, dt):
    dim = 256
    hw_, ws, latent, tx, cos, sin, mask = dit_setup(ctx, dt)
    feat = O.timestep_features(705.8824)[:dim].copy()
    pred = empty(latent.shape)
    valid = int(np.sum(mask == 0))
    ctx.dit_forward(dev(latent), 16, dev(tx), tx.shape[0], dev(feat), dev(cos), dev(sin), [20, 21], pred,
                    mask=dev(mask), valid_keys=valid)
    ref = oracle_dit(ws, hw_, latent, tx, feat, cos, sin, mask)
    g = kat.gate(host(pred), ref, *kat.SEQUENCE_GATES[NAMES[dt]])
    assert g["passed"], g


@pytest.mark.parametrize("dt", [E.FP32, E.FP16], ids=lambda d: NAMES[d])
def test_facade_denoise_against_oracle(dt):
    # denoise (src/denoiser.cpp:41-86) through the C++ facade: schedule, time
    # features, run_dit, Euler and the finite check; 3 of 4 steps from start_step 1.
    import torch
    fac = E.Facade(0)
    dim = 4096  # time features are 4096 wide (ERNIE Timesteps(4096))
    ffn = 512
    hw_ = small_heads(dim=dim, latent_ch=128, text_dim=3072, seed=40)
    fac.hip.heads_upload(hw_, dim, 128, 3072, dt)
    ws = [small_block(dim, ffn, seed=41)]
    fac.hip.block_upload(0, ws[0], dim, ffn, dt)
    H = W = 4
    text, valid = 8, 5
    latent = O.normal((128, H, W), 43)
    tx = O.normal((text, 3072), 44)
    tx[valid:] = 0.0
    cos, sin, mask = O.dit_constants(O.rope_frequencies(), W, H, valid, text)
    steps, start = 4, 1
    lat = dev(latent)
    secs, ts = fac.denoise([0], lat, H, W, dev(tx), text, dev(cos), dev(sin), dev(mask), H * W + valid, steps,
                           start_step=start, dtype=dt)
    sig, tsteps = O.flow_schedule_turbo(steps)
    np.testing.assert_array_equal(ts, tsteps[start:])
    assert np.all(secs > 0)
    ref = latent.copy()
    for i in range(start, steps):
        pred = oracle_dit(ws, hw_, ref, tx, O.timestep_features(float(tsteps[i])), cos, sin, mask)
        ref = O.euler_step(ref, pred, sig[i + 1] - sig[i])
    nrmse, rtol, atol = kat.DENOISER_GATES[NAMES[dt]]
    g = kat.gate(host(lat), ref, atol, rtol, nrmse)
    assert g["passed"], g
    # Argument contracts of the facade (src/denoiser.cpp:12-19, 50-51).
    with pytest.raises(E.ErnieInvalidRequest):
        fac.denoise([0], lat, H, W, dev(tx), text, dev(cos), dev(sin), dev(mask), 0, steps, start_step=5, dtype=dt)
    with pytest.raises(E.ErnieInvalidRequest):
        fac.denoise([], lat, H, W, dev(tx), text, dev(cos), dev(sin), dev(mask), 0, steps, dtype=dt)
    torch.cuda.synchronize()
    fac.close()


def test_facade_block_sequence_validation_and_parity():
    fac = E.Facade(0)
    dim, ffn = 256, 512
    w = small_block(dim, ffn, seed=50)
    fac.hip.block_upload(0, w, dim, ffn, E.FP32)
    x, mods, cos, sin, mask = small_inputs(S=40, dim=dim)
    md = [dev(m) for m in mods]
    out = empty(x.shape)
    valid = int(np.sum(mask == 0))
    secs = fac.run_block_sequence([0], dev(x), 40, dim, md, dev(cos), dev(sin), out, mask=dev(mask),
                                  valid_prefix=valid)
    assert secs.shape == (1,) and secs[0] > 0
    m = kat.fp32_block_rule(host(out), O.block_forward(w, x, mods, cos, sin, mask))
    assert m["passed"], m
    with pytest.raises(E.ErnieInvalidRequest):
        fac.run_block_sequence([0] * 37, dev(x), 40, dim, md, dev(cos), dev(sin), out)
    with pytest.raises(E.ErnieInvalidRequest):
        fac.run_block_sequence([], dev(x), 40, dim, md, dev(cos), dev(sin), out)
    fac.close()


@pytest.mark.parametrize("dim,ffn,S,image,valid", [(4096, 1024, 4160, (64, 64), 40), (1024, 2048, 4136, (64, 64), 20)],
                         ids=["light-tail-tiles", "split-tail"])
@pytest.mark.parametrize("dt", [E.FP16, E.BF16], ids=lambda d: NAMES[d])
def test_qk_rounding_orders(ctx, dt, dim, ffn, S, image, valid):
    # 16-bit blocks normalise and rotate Q and K from the QKV GEMM's FP32 accumulators
    # (ERNIE_QK_ROUND_FUSED, the default); ERNIE_QK_ROUND_STORAGE first rounds the
    # projections to the storage dtype, as the reference graph does (gemm_0/gemm_1 ->
    # rmsn_9/rmsn_10). At 4160 tokens and width 4096 the Q/K/V GEMM finishes its 64 tail
    # rows in light tiles; at width 1024 and 4136 tokens (192 full tiles) in a split tail
    # row, whose rows take the storage order in both modes. (GEMMs of at most 128 tiles
    # split every tile along K and so always take the storage order.) The two orders
    # differ by one rounding of Q and K: their block outputs are held to each other by the
    # reference's block gate for the dtype and by NRMSE <= 1e-3 (FP16) / 8e-3 (BF16), an
    # eighth and a quarter of that gate, and to the oracle by the gate where the oracle
    # runs (the narrower case).
    w = small_block(dim=dim, ffn=ffn, seed=15)
    x, mods, cos, sin, mask = small_inputs(S=S, dim=dim, image=image, valid=valid, seed=16)
    ctx.block_upload(8, w, dim, ffn, dt)
    keys = int(np.sum(mask == 0))
    fused = run_block(ctx, 8, x, mods, cos, sin, mask, keys)
    ctx.call("set_qk_rounding", 1)
    try:
        storage = run_block(ctx, 8, x, mods, cos, sin, mask, keys)
        np.testing.assert_array_equal(run_block(ctx, 8, x, mods, cos, sin, mask, keys), storage)
    finally:
        ctx.call("set_qk_rounding", 0)
    np.testing.assert_array_equal(run_block(ctx, 8, x, mods, cos, sin, mask, keys), fused)
    assert not np.array_equal(fused, storage)
    g = kat.gate(fused, storage, *kat.BLOCK_GATES[NAMES[dt]])
    print(f"qk rounding orders {NAMES[dt]} S={S}: max|d| {g['max_abs_error']:.3g} nrmse {g['nrmse']:.3g}", flush=True)
    assert g["passed"] and g["nrmse"] <= (1e-3 if dt == E.FP16 else 8e-3), g
    if dim <= 1024:
        ref = O.block_forward(w, x, mods, cos, sin, mask)
        for name, got in (("fused", fused), ("storage", storage)):
            go = kat.gate(got, ref, *kat.BLOCK_GATES[NAMES[dt]])
            assert go["passed"], (name, go)
    with pytest.raises(E.ErnieError):
        ctx.call("set_qk_rounding", 2)
    ctx.call("block_release", 8)


@pytest.mark.parametrize("dt", [E.FP16, E.BF16], ids=lambda d: NAMES[d])
def test_rotary_pairs_must_repeat(ctx, dt):
    # 16-bit blocks read each rotary angle once from its pair of columns (2k, 2k + 1). The
    # reference's tables repeat every angle there (src/conditioning.cpp:34-37); a table
    # whose pair columns differ makes the output non-finite instead of silently using one
    # of the two values.
    w = small_block(dim=256, ffn=512, seed=21)
    x, mods, cos, sin, mask = small_inputs(S=300, dim=256, image=(16, 16), valid=30, seed=22)
    ctx.block_upload(9, w, 256, 512, dt)
    keys = int(np.sum(mask == 0))
    good = run_block(ctx, 9, x, mods, cos, sin, mask, keys)
    assert np.isfinite(good).all()
    ref = O.block_forward(w, x, mods, cos, sin, mask)
    g = kat.gate(good, ref, *kat.BLOCK_GATES[NAMES[dt]])
    assert g["passed"], g
    bad = cos.copy()
    bad[7, 11] += 0.25  # column 11 no longer repeats column 10 in row 7
    assert not np.isfinite(run_block(ctx, 9, x, mods, bad, sin, mask, keys)).all()
    np.testing.assert_array_equal(run_block(ctx, 9, x, mods, cos, sin, mask, keys), good)
    ctx.call("block_release", 9)
