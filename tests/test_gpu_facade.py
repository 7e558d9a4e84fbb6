"""The facade's queueing contracts on the device: the asynchronous finite check and
stream markers, the block cache's trim, run_dit's per-block observer and timing, and
a denoise whose finiteness is read one step behind (src/denoiser.cpp:41-86 reports
each step, observes each step and names the failing step; src/dit.cpp:126 ->
src/block_sequence.cpp:89 observes every block)."""
import ctypes

import numpy as np
import pytest

import ernie_amd as E
import kat
import oracle as O
from gpu_util import dev, empty, host
from test_oracle import small_block, small_heads

pytestmark = pytest.mark.gpu


def device_copy(ctx, ptr, count):
    """FP32 values at a device address, read on the context stream."""
    out = np.empty(count, np.float32)
    ctx.call("memcpy_d2h", out.ctypes.data, ctypes.c_void_p(ptr), count * 4)
    return out


def test_finite_check_in_flight_on_two_slots(ctx):
    good = dev(O.normal((1000,), 5))
    bad_host = O.normal((1000,), 6)
    bad_host[777] = np.inf
    bad = dev(bad_host)
    ctx.marker(0)
    ctx.finite_begin(good, 1000, 0)
    ctx.finite_begin(bad, 1000, 1)
    ctx.marker(1)
    assert ctx.finite_end(1) is False
    assert ctx.finite_end(0) is True
    assert ctx.marker_elapsed(0, 1) >= 0.0
    # A slot is free again after its end; ending it twice is an error, as is a bad slot.
    with pytest.raises(E.ErnieError):
        ctx.finite_end(0)
    with pytest.raises(E.ErnieError):
        ctx.finite_begin(good, 1000, E_SLOTS + E_SLOTS_RESERVED)
    with pytest.raises(E.ErnieError):
        ctx.finite_begin(good, 1000, -1)
    nan_host = np.zeros(64, np.float32)
    nan_host[0] = np.nan
    ctx.finite_begin(dev(nan_host), 64, 2)
    assert ctx.finite_end(2) is False
    # The synchronous check agrees.
    assert ctx.finite(good, 1000) and not ctx.finite(bad, 1000)
    with pytest.raises(E.ErnieError):
        ctx.marker_elapsed(0, 63)  # never recorded


E_SLOTS = 4           # ERNIE_FINITE_SLOTS: the callers' slots
E_SLOTS_RESERVED = 3  # ERNIE_FINITE_SLOTS_RESERVED: the facade's, after them


def test_upload_async_copies_before_the_source_is_reused(ctx):
    import torch
    dst = torch.empty(3 * 4096, dtype=torch.float32, device="cuda")
    src = np.arange(4096, dtype=np.float32)
    for k in range(3):
        ctx.call("upload_async", ctypes.c_void_p(dst.data_ptr() + k * 4096 * 4), src.ctypes.data, 4096 * 4)
        src += 4096  # the caller's buffer changes right away
    np.testing.assert_array_equal(host(dst), np.arange(3 * 4096, dtype=np.float32))


def test_trim_releases_freed_blocks():
    import torch
    fac = E.Facade(0)
    try:
        c = fac.hip
        p = ctypes.c_void_p()
        c.call("malloc", 3 << 20, ctypes.byref(p))
        c.call("free", p)
        assert c.trim() >= 3 << 20
        assert c.trim() == 0
    finally:
        torch.cuda.synchronize()
        fac.close()


def dit_fixture(fac, dt, nblocks=3, dim=256, ffn=512):
    heads = small_heads(dim=dim, latent_ch=128, text_dim=3072, seed=70)
    fac.hip.heads_upload(heads, dim, 128, 3072, dt)
    ws = [small_block(dim, ffn, seed=71 + i) for i in range(nblocks)]
    for i, w in enumerate(ws):
        fac.hip.block_upload(i, w, dim, ffn, dt)
    H, W, text, valid = 4, 5, 8, 6
    latent = O.normal((128, H, W), 81)
    tx = O.normal((text, 3072), 82)
    tx[valid:] = 0.0
    cos, sin, mask = O.dit_constants(O.rope_frequencies(), W, H, valid, text)
    return heads, ws, latent, tx, cos, sin, mask, H, W, text, H * W + valid


def test_run_dit_observes_every_block():
    import torch
    dim = 256
    fac = E.Facade(0)
    try:
        heads, ws, latent, tx, cos, sin, mask, H, W, text, valid = dit_fixture(fac, E.FP32)
        feat = O.timestep_features(612.5)[:dim].copy()
        seen = {}

        def observer(stage, ptr, w, h, c):
            seen[stage] = device_copy(fac.hip, ptr, w * h * c).reshape(-1, w) if h * c > 1 else \
                device_copy(fac.hip, ptr, w)

        pred = empty(latent.shape)
        secs = fac.run_dit([0, 1, 2], dev(latent), H, W, dev(tx), text, dev(feat), dim, dev(cos), dev(sin), pred,
                           mask=dev(mask), valid_prefix=valid, dtype=E.FP32, timing=True, observer=observer)
        assert list(seen) == [f"head-{i}" for i in range(8)] + ["block-0", "block-1", "block-2"]
        assert secs.shape == (3,) and np.all(secs > 0)
        # Each observed stage against the oracle's own chain.
        x, c, mods = O.input_head({k: heads[k] for k in O.INPUT_HEAD_FIELDS}, latent, tx, feat)
        g = kat.gate(seen["head-0"], x, *kat.HEAD_GATES["fp32"])
        assert g["passed"], g
        for i in range(6):
            g = kat.gate(seen[f"head-{i + 2}"], mods[i], *kat.HEAD_GATES["fp32"])
            assert g["passed"], (i, g)
        for i, w in enumerate(ws):
            ref = O.block_forward(w, seen["head-0"] if i == 0 else seen[f"block-{i - 1}"], mods, cos, sin, mask)
            m = kat.fp32_block_rule(seen[f"block-{i}"], ref)
            assert m["passed"], (i, m)
        # Without observer or timing the same prediction comes back (one queued call).
        pred2 = empty(latent.shape)
        assert fac.run_dit([0, 1, 2], dev(latent), H, W, dev(tx), text, dev(feat), dim, dev(cos), dev(sin), pred2,
                           mask=dev(mask), valid_prefix=valid, dtype=E.FP32) is None
        np.testing.assert_array_equal(host(pred2), host(pred))
    finally:
        torch.cuda.synchronize()
        fac.close()


@pytest.mark.parametrize("details", [False, True], ids=["queued", "collect_details"])
def test_denoise_observer_sees_each_step(details):
    # dim 4096 (the time features' width), FFN 512, one block; 4 steps from step 1.
    import torch
    dim, ffn = 4096, 512
    fac = E.Facade(0)
    try:
        heads = small_heads(dim=dim, latent_ch=128, text_dim=3072, seed=90)
        fac.hip.heads_upload(heads, dim, 128, 3072, E.FP32)
        w = small_block(dim, ffn, seed=91)
        fac.hip.block_upload(0, w, dim, ffn, E.FP32)
        H = W = 4
        text, valid = 8, 5
        latent = O.normal((128, H, W), 92)
        tx = O.normal((text, 3072), 93)
        tx[valid:] = 0.0
        cos, sin, mask = O.dit_constants(O.rope_frequencies(), W, H, valid, text)
        seen = []

        def observer(step, pred_ptr, sample_ptr, count):
            seen.append((step, device_copy(fac.hip, pred_ptr, count), device_copy(fac.hip, sample_ptr, count)))

        steps, start = 4, 1
        lat = dev(latent)
        secs, ts = fac.denoise_observed([0], lat, H, W, dev(tx), text, dev(cos), dev(sin), dev(mask), H * W + valid,
                                        steps, start_step=start, dtype=E.FP32, collect_details=details,
                                        observer=observer)
        assert [s for s, _, _ in seen] == [1, 2, 3]
        assert secs.shape == (3,) and np.all(secs > 0)
        sig, tsteps = O.flow_schedule_turbo(steps)
        np.testing.assert_array_equal(ts, tsteps[start:])
        ref = latent.copy()
        nrmse, rtol, atol = kat.DENOISER_GATES["fp32"]
        for (step, pred, sample), i in zip(seen, range(start, steps)):
            out_w = {"mod_w": heads["out_mod_w"], "mod_b": heads["out_mod_b"], "proj_w": heads["proj_w"],
                     "proj_b": heads["proj_b"]}
            x, c, mods = O.input_head({k: heads[k] for k in O.INPUT_HEAD_FIELDS}, ref, tx,
                                      O.timestep_features(float(tsteps[i])))
            x = O.block_forward(w, x, mods, cos, sin, mask)
            p = O.output_head(out_w, x, c, H * W).reshape(ref.shape)
            ref = O.euler_step(ref, p, sig[i + 1] - sig[i])
            g = kat.gate(pred.reshape(ref.shape), p, atol, rtol, nrmse)
            assert g["passed"], (step, g)
            g = kat.gate(sample.reshape(ref.shape), ref, atol, rtol, nrmse)
            assert g["passed"], (step, g)
        np.testing.assert_array_equal(host(lat), seen[-1][2].reshape(ref.shape))
    finally:
        torch.cuda.synchronize()
        fac.close()


@pytest.mark.parametrize("start", [0, 2])
def test_denoise_names_the_non_finite_step(start):
    # A NaN output-projection bias makes the first executed step's prediction NaN: its
    # check, read while the next step is queued, must still name that step.
    import torch
    dim, ffn = 4096, 512
    fac = E.Facade(0)
    try:
        heads = small_heads(dim=dim, latent_ch=128, text_dim=3072, seed=95)
        heads["proj_b"] = heads["proj_b"].copy()
        heads["proj_b"][3] = np.nan
        fac.hip.heads_upload(heads, dim, 128, 3072, E.FP16)
        fac.hip.block_upload(0, small_block(dim, ffn, seed=96), dim, ffn, E.FP16)
        H = W = 4
        text, valid = 8, 5
        tx = O.normal((text, 3072), 97)
        cos, sin, mask = O.dit_constants(O.rope_frequencies(), W, H, valid, text)
        seen = []
        with pytest.raises(E.ErnieError, match=f"Non-finite latent after denoise step {start + 1}$"):
            fac.denoise_observed([0], dev(O.normal((128, H, W), 98)), H, W, dev(tx), text, dev(cos), dev(sin),
                                 dev(mask), H * W + valid, 4, start_step=start, dtype=E.FP16,
                                 observer=lambda *a: seen.append(a[0]))
        assert seen == []
        # A non-finite initial latent is rejected as an invalid request (src/denoiser.cpp:56-57).
        bad = O.normal((128, H, W), 98)
        bad[5, 1, 2] = np.inf
        with pytest.raises(E.ErnieInvalidRequest, match="Initial latent is not finite"):
            fac.denoise_observed([0], dev(bad), H, W, dev(tx), text, dev(cos), dev(sin), dev(mask), H * W + valid, 4,
                                 start_step=start, dtype=E.FP16, observer=lambda *a: seen.append(a[0]))
        assert seen == []
    finally:
        torch.cuda.synchronize()
        fac.close()


def test_denoise_reports_a_later_steps_own_failure():
    # Step k's DiT fails (its block was released by the observer of step k - 2, after the
    # device had finished with it) while step k - 1's finite check is still pending. That
    # check passes, so the error that comes back is step k's own device error, not
    # a finite-check or timing error, and every earlier step was observed.
    import torch
    dim, ffn = 4096, 512
    fac = E.Facade(0)
    try:
        fac.hip.heads_upload(small_heads(dim=dim, latent_ch=128, text_dim=3072, seed=60), dim, 128, 3072, E.FP16)
        fac.hip.block_upload(0, small_block(dim, ffn, seed=61), dim, ffn, E.FP16)
        H = W = 4
        text, valid = 8, 5
        tx = O.normal((text, 3072), 62)
        cos, sin, mask = O.dit_constants(O.rope_frequencies(), W, H, valid, text)
        seen = []

        def observer(step, *_):
            seen.append(step)
            if step == 0:
                fac.hip.synchronize()  # step 1 is queued on the block: let it finish first
                fac.hip.call("block_release", 0)

        with pytest.raises(E.ErnieError, match="not loaded") as info:
            fac.denoise_observed([0], dev(O.normal((128, H, W), 63)), H, W, dev(tx), text, dev(cos), dev(sin),
                                 dev(mask), H * W + valid, 4, dtype=E.FP16, observer=observer)
        assert type(info.value) is E.ErnieError  # neither an allocation error nor a rejected request
        assert seen == [0, 1]
    finally:
        torch.cuda.synchronize()
        fac.close()
