"""The register_layers plugin seam (src/ernie_gelu.cpp:108-116) on the device: each
registered op is driven as a one-layer graph would drive it, by its .param parameter
ids and .bin weights, on the reference's own known-answer tests
(probes/rmsnorm_probe.cpp:40-107, probes/gelu_probe.cpp:152-196,
tests/test_residual_contract.cpp, tests/test_attention_mask.cpp:18-105,
tests/test_bf16_gemm.cpp:17-214)."""
import numpy as np
import pytest

import ernie_amd as E
import kat
from gpu_util import ALL_DT, NAMES, dev, empty, host, stored

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fac():
    import torch
    f = E.Facade(0)
    yield f
    torch.cuda.synchronize()
    f.close()


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("width", [128, 3072, 4096])
def test_rmsnorm_layer(fac, dt, width):
    # "RMSNorm norm 1 1 in0 out0 0=<width> 1=0.000001 2=1" with the probe's weights; the
    # Q/K-norm width is a 3D blob [8][5][128], the hidden widths 2D [8][width].
    for scale in (1.0, 512.0):
        x, gamma, expected = kat.rmsnorm_kat_case(width, scale)
        c, h = (8, 5) if width == 128 else (1, 8)
        xd = dev(x, dt)
        fac.op_forward("RMSNorm", f"0={width} 1=0.000001 2=1", [(xd, dt, width, h, c)], weights=gamma)
        err = np.max(np.abs(host(xd) - expected))  # in place: one blob
        assert err <= kat.RMSNORM_LIMITS[NAMES[dt]], (scale, err)


def test_layernorm_layer(fac):
    for scale in (1.0, 1024.0):
        x, _, expected = kat.rmsnorm_kat_case(4096, scale, centered=True)
        out = empty(x.shape)
        fac.op_forward("LayerNorm", "0=4096 1=0.000001 2=0", [(dev(x), E.FP32, 4096, 8, 1)],
                       [(out, E.FP32, 4096, 8, 1)])
        assert np.max(np.abs(host(out) - expected)) <= kat.RMSNORM_LIMITS["fp32"]


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_gelu_layer(fac, dt):
    for shape, dims in ((0, (4096, 16, 1)), (1, (128, 257, 3))):
        x = kat.gelu_kat_input(shape)
        xd = dev(x, dt)
        fac.op_forward("ErnieGELU", "", [(xd, dt) + dims])
        err = np.max(np.abs(host(xd) - kat.gelu_expected(x)))
        assert err <= kat.GELU_LIMITS[NAMES[dt]], (shape, err)


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_residual_layer(fac, dt):
    # "ErnieResidualAdd add_16 2 1 ... 0=0": FP32 result whatever the operand storage.
    a, b = kat.residual_case()
    out = empty(a.shape)
    shape = (a.shape[1], a.shape[0], 1)
    fac.op_forward("ErnieResidualAdd", "0=0", [(dev(a), E.FP32) + shape, (dev(b, dt), dt) + shape],
                   [(out, E.FP32) + shape])
    np.testing.assert_array_equal(host(out), (a + stored(b, dt)).astype(np.float32))


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_sdpa_layer_mask_kat(fac, dt):
    # "SDPA sdpa_22 4 1 q k v mask out 5=1": row mask and dense mask agree bitwise.
    queries, keys, width, heads = 257, 65, 128, 2
    for mask_heads in (1, 2):
        q, k, v, row, dense = kat.attention_mask_case(queries, keys, mask_heads, width, 0)
        qd, kd, vd = dev(q, dt), dev(k, dt), dev(v, dt)
        outs = []
        for mask in (dense, row):
            o = empty((heads, queries, width), dt)
            fac.op_forward("SDPA", "5=1", [(qd, dt, width, queries, heads), (kd, dt, width, keys, 1),
                                           (vd, dt, width, keys, 1),
                                           (dev(mask), E.FP32, keys, mask.shape[1], mask_heads)],
                           [(o, dt, width, queries, heads)])
            outs.append(host(o))
        np.testing.assert_array_equal(outs[0], outs[1])
        expected = kat.attention_mask_expected(stored(q, dt), stored(k, dt), stored(v, dt), keys, mask_heads, 0)
        limit = {E.FP32: 3e-6, E.FP16: 4e-3, E.BF16: 3e-2}[dt]
        assert np.max(np.abs(outs[1] - expected)) < limit


# tests/test_bf16_gemm.cpp:196-201: name, M, N, K, transA, transB, bias type, output
# transpose, output N1M, output elempack.
GEMM_SHAPES = [("projection", 32, 48, 64, 0, 1, -1, 0, 0, 4),
               ("single_row_bias", 1, 48, 32, 0, 1, 4, 0, 0, 1),
               ("odd_transpose", 17, 19, 32, 1, 0, 4, 1, 1, 1),
               ("matrix_bias", 32, 48, 64, 1, 1, 3, 1, 1, 4)]


def gemm_case(m, n, k, ta, tb, bias):
    """The test's input blob, .bin weights (B then C) and the FP64 product + bias."""
    r = np.arange(m)[:, None]
    i = np.arange(k)[None, :]
    a = (((r * 13 + i * 7) % 17 - 3) * np.where(r % 3 == 0, -0.125, 0.125)).astype(np.float32)  # [m][k]
    ii = np.arange(k)[:, None]
    col = np.arange(n)[None, :]
    w_kn = (((ii * 5 + col * 11) % 9 - 2) * 0.125).astype(np.float32)  # weight_value(inner, column)
    rows = np.arange(m)[:, None]
    c_mn = ((((rows * 3) if bias == 3 else 0) + col) % 5 - 2) * 0.125 if bias != -1 else np.zeros((m, n))
    weights = [w_kn.T if tb else w_kn]
    if bias == 4:
        weights.append(c_mn[0])
    elif bias == 3:
        weights.append(c_mn)
    blob = a.T if ta else a
    expected = a.astype(np.float64) @ w_kn.astype(np.float64) + c_mn
    return np.ascontiguousarray(blob), np.concatenate([np.ravel(x) for x in weights]).astype(np.float32), expected


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
@pytest.mark.parametrize("shape", GEMM_SHAPES, ids=lambda s: s[0])
def test_gemm_layer_exact_products(fac, dt, shape):
    _, m, n, k, ta, tb, bias, tout, n1m, pack = shape
    blob, weights, expected = gemm_case(m, n, k, ta, tb, bias)
    params = (f"0=1.0 1=1.0 2={ta} 3={tb} 4=0 5=1 6=1 7={m} 8={n} 9={k} 10={bias} 11={n1m} 12={pack} "
              f"14={tout}")
    want = expected.T if tout else expected
    rows, w = want.shape
    out_dims = (w, 1, rows) if n1m else (w, rows, 1)
    for out_dt in sorted({E.FP32, dt}):
        out = empty((rows, w), out_dt)
        fac.op_forward("Gemm", params, [(dev(blob, dt), dt, blob.shape[1], blob.shape[0], 1)],
                       [(out, out_dt) + out_dims], weights=weights)
        # Exact: every product and partial sum is a multiple of 1/64 within FP32 range,
        # so the result is the one rounding of the FP64 sum to the output precision.
        np.testing.assert_array_equal(host(out), stored(want.astype(np.float32), out_dt))


def test_registry_rejections(fac):
    x = empty((8, 4096))
    blob = [(x, E.FP32, 4096, 8, 1)]
    gamma = np.ones(4096, np.float32)
    with pytest.raises(E.ErnieError):  # unregistered type
        fac.op_forward("Softmax", "0=1", blob)
    with pytest.raises(E.ErnieError):  # RMSNorm widths are 128 / 3072 / 4096
        fac.op_forward("RMSNorm", "0=1000 1=0.000001 2=1", [(x, E.FP32, 1000, 8, 1)], weights=gamma[:1000])
    with pytest.raises(E.ErnieError):  # non-affine RMSNorm is not an ERNIE layer
        fac.op_forward("RMSNorm", "0=4096 1=0.000001 2=0", blob, weights=gamma)
    with pytest.raises(E.ErnieError):  # residual adds only (0=0), without a scalar (1=0)
        fac.op_forward("ErnieResidualAdd", "0=2", blob + blob, blob)
    with pytest.raises(E.ErnieError):  # alpha other than 1
        fac.op_forward("Gemm", "0=2.0 3=1 5=1 8=16 9=4096", blob, [(empty((8, 16)), E.FP32, 16, 8, 1)],
                       weights=np.zeros(16 * 4096, np.float32))
    with pytest.raises(E.ErnieInvalidRequest):  # malformed parameter text
        fac.op_forward("RMSNorm", "0=", blob, weights=gamma)
    with pytest.raises(E.ErnieInvalidRequest):
        fac.op_forward("RMSNorm", "0=4096 x=1", blob, weights=gamma)
