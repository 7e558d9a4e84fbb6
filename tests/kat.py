"""Known-answer inputs and gates ported from the reference's own tests.

Each generator reproduces the closed-form integer-pattern inputs of the named
reference test/probe, so the same FP64 expectations apply here.
"""
import math

import numpy as np

# ---- gates -----------------------------------------------------------------------
# tools/validate_dit_block.py:108-120 (max |d| <= atol + rtol * max|ref| AND nrmse),
# gate values fixed in tools/export_dit_block.py:163-165 (block) and
# tools/validate_block_sequence.py:37-39 / tools/validate_dit.py:58-60 (sequence).
BLOCK_GATES = {"fp32": (2e-4, 2e-4, 2e-5), "fp16": (0.02, 0.02, 0.01), "bf16": (0.15, 0.08, 0.03)}
SEQUENCE_GATES = {"fp32": (2e-4, 2e-4, 2e-4), "fp16": (0.03, 0.03, 0.03), "bf16": (0.2, 0.2, 0.12)}
HEAD_GATES = {"fp32": (2e-4, 2e-4, 2e-5), "fp16": (0.03, 0.03, 0.02), "bf16": (0.2, 0.2, 0.1)}
# tools/validate_text.py:53-54: text block / text stack gates as (atol, rtol, nrmse).
TEXT_GATES = {"fp32": (2e-4, 2e-4, 2e-4), "fp16": (0.03, 0.03, 0.03), "bf16": (0.2, 0.2, 0.15)}
# tools/validate_denoiser.py:53-55 as (nrmse, global_rtol, atol); the reference has no BF16 denoiser gate.
DENOISER_GATES = {"fp32": (0.002, 0.002, 0.0002), "fp16": (0.1, 0.1, 0.03)}


def metrics(actual, ref):
    a = np.asarray(actual, np.float64).ravel()
    r = np.asarray(ref, np.float64).ravel()
    d = a - r
    return {"max_abs_error": float(np.max(np.abs(d))) if d.size else 0.0,
            "nrmse": float(np.linalg.norm(d) / max(np.linalg.norm(r), 1e-30)),
            "reference_max_abs": float(np.max(np.abs(r))) if r.size else 0.0,
            "finite": bool(np.isfinite(a).all())}


def gate(actual, ref, atol, rtol, nrmse):
    m = metrics(actual, ref)
    limit = atol + rtol * m["reference_max_abs"]
    m.update(max_abs_limit=limit, nrmse_limit=nrmse,
             passed=m["finite"] and m["max_abs_error"] <= limit and m["nrmse"] <= nrmse)
    return m


def fp32_block_rule(actual, ref):
    """FP32 block rule: max |d| <= 1e-4 * max |ref|."""
    m = metrics(actual, ref)
    m["passed"] = m["finite"] and m["max_abs_error"] <= 1e-4 * m["reference_max_abs"]
    return m


# ---- probes/rmsnorm_probe.cpp:40-107 -----------------------------------------------
RMSNORM_LIMITS = {"fp32": 2e-6, "fp16": 0.002, "bf16": 0.01}


def rmsnorm_kat_case(width, scale, centered=False):
    """Returns (x [rows][width] float32, gamma, expected FP64). Q/K norm width 128 is [8][5][128]."""
    channels, rows = (8, 5) if width == 128 else (1, 8)
    weight = np.array([.5 + (i % 8) * .0625 for i in range(width)], np.float32)
    x = np.empty((channels, rows, width), np.float32)
    for c in range(channels):
        for r in range(rows):
            for i in range(width):
                x[c, r, i] = scale * (.5 + ((i + r + c) % 8) * .125)
    x = x.reshape(-1, width)
    xd = x.astype(np.float64)
    mean = xd.mean(axis=1, keepdims=True) if centered else 0.0
    d = xd - mean
    inv = 1.0 / np.sqrt((d * d).sum(axis=1, keepdims=True) / width + 1e-6)
    expected = d * inv * (1.0 if centered else weight.astype(np.float64))
    return x, weight, expected


# ---- probes/gelu_probe.cpp:152-196 -------------------------------------------------
GELU_LIMITS = {"fp32": 2e-6, "fp16": 0.008, "bf16": 0.064}


def gelu_kat_input(shape):
    """shape 0: [16][4096]; shape 1: [3][257][128]; linspace over [-12, 12]."""
    dims = (1, 16, 4096) if shape == 0 else (3, 257, 128)
    count = int(np.prod(dims))
    c, plane = dims[0], dims[1] * dims[2]
    x = np.empty(count, np.float32)
    for ch in range(c):
        i = np.arange(plane, dtype=np.int64)
        x[ch * plane:(ch + 1) * plane] = (-12.0 + 24.0 * (i + ch * plane).astype(np.float32) / np.float32(count - 1)
                                          ).astype(np.float32)
    return x


def gelu_expected(x):
    from scipy.special import erfc
    xd = np.asarray(x, np.float64)
    return 0.5 * xd * erfc(-xd / math.sqrt(2.0))


# ---- tests/test_attention_mask.cpp:18-105 -----------------------------------------
def attention_mask_case(queries, keys, mask_heads, width=128, shift=0):
    heads = 2
    i = np.arange(queries)[:, None]
    d = np.arange(width)[None, :]
    q = np.stack([((i * 3 + d * 7 + h) % 17 - 8) / 32.0 for h in range(heads)]).astype(np.float32)
    j = np.arange(keys)[:, None]
    k = (((j * 7 + d) % 19 - 9) / 32.0).astype(np.float32)[None]
    v = (((j * 3 + d * 5) % 23 - 11) / 16.0).astype(np.float32)[None]
    row = np.zeros((mask_heads, 1, keys), np.float32)
    for h in range(mask_heads):
        row[h, 0, keys - 4 - shift - h:] = -1e30
    dense = np.repeat(row, queries, axis=1)
    return q, k, v, row, dense


def attention_mask_expected(q, k, v, keys, mask_heads, shift):
    """FP64 attention with the mask as an exact visible-key count."""
    heads, queries, width = q.shape
    out = np.empty((heads, queries, width), np.float64)
    for h in range(heads):
        visible = keys - 4 - shift - (0 if mask_heads == 1 else h)
        dots = q[h].astype(np.float64) @ k[0, :visible].astype(np.float64).T
        p = np.exp(dots / math.sqrt(width))
        out[h] = (p @ v[0, :visible].astype(np.float64)) / p.sum(axis=1, keepdims=True)
    return out


# ---- probes/attention_accuracy_probe.cpp:22-80 --------------------------------------
def attention_accuracy_case():
    width, queries, keys, heads, visible = 128, 5, 4160, 2, 4128
    q = np.empty((heads, queries, width), np.float32)
    k = np.empty((heads, keys, width), np.float32)
    v = np.empty((heads, keys, width), np.float32)
    d = np.arange(width)
    j = np.arange(keys)[:, None]
    for h in range(heads):
        for i in range(queries):
            q[h, i] = 0.0 if i == 0 else ((d * 17 + i * 13 + h) % 41 - 20) / 40.0
        k[h] = ((j * 7 + d[None] * 19 + h * 11) % 101 - 50) / 64.0
        v[h] = ((j * 47 + d[None] * 13 + h * 31) % 257 - 128) / 128.0
        v[h, :, 0] = 1.0
    mask = np.zeros((queries, keys), np.float32)
    mask[:, visible:] = -1e30
    expected = np.empty((heads, queries, width), np.float64)
    for h in range(heads):
        s = q[h].astype(np.float64) @ k[h, :visible].astype(np.float64).T / math.sqrt(width)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        expected[h] = (p @ v[h, :visible].astype(np.float64)) / p.sum(axis=1, keepdims=True)
    return q, k, v, mask, expected.astype(np.float32), visible


def attention_accuracy_gate(actual, expected):
    a = np.asarray(actual, np.float64)
    b = np.asarray(expected, np.float64)
    err = a - b
    nrmse = math.sqrt((err ** 2).sum() / (b ** 2).sum())
    maximum = float(np.abs(err).max())
    constant = float(np.abs(a[:, :, 0] - 1.0).max())
    return {"max_abs_error": maximum, "constant_error": constant, "nrmse": nrmse,
            "passed": maximum <= 3e-6 and constant <= 5e-7 and nrmse <= 5e-7}


# ---- tests/test_bf16_gemm.cpp:17-214 -------------------------------------------------
GEMM_KAT_SHAPES = [("projection", 32, 48, 64, False), ("single_row_bias", 1, 48, 32, True),
                   ("odd_transpose", 17, 19, 32, True), ("matrix", 32, 48, 64, False)]


def gemm_kat_case(m, n, k):
    r = np.arange(m)[:, None]
    i = np.arange(k)[None, :]
    a = (((r * 13 + i * 7) % 17 - 3) * np.where(r % 3 == 0, -0.125, 0.125)).astype(np.float32)
    ii = np.arange(k)[:, None]
    col = np.arange(n)[None, :]
    w_kn = (((ii * 5 + col * 11) % 9 - 2) * 0.125).astype(np.float32)  # [k][n]
    bias = (((np.arange(n)) % 5 - 2) * 0.125).astype(np.float32)
    return a, np.ascontiguousarray(w_kn.T), bias


def rne_bf16(x):
    """Round FP32 values to BF16 (nearest-even), returned as FP32."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    b = (b + 0x7FFF + ((b >> 16) & 1)) & 0xFFFF0000
    return b.astype(np.uint32).view(np.float32)


# ---- tests/test_residual_contract.cpp:44-60 -------------------------------------------
def residual_case():
    y = np.arange(4)[:, None]
    i = np.arange(4096)[None, :]
    a = (np.where(i % 2 == 1, -1.0, 1.0) * (70000.0 + y * 128.0)).astype(np.float32)
    b = ((i % 8) * 128.0 + 0 * y).astype(np.float32)
    return a, b


# ---- probes/attention_probe.cpp:20-112: causal GQA attention ----------------------
# 32 query heads over 8 key/value heads, head_dim 128; inputs are a hash of
# (head, position, dim, seed) in [-1, 1); the mask is 0 for visible keys and
# -1e30 past the query's position; the expectation is an FP64 softmax over
# exactly the visible keys. Operator gates (max abs, nrmse) from suite(), lines 321-323.
GQA_PROBE_LIMITS = {"fp32": (2e-5, 2e-5), "fp16": (0.002, 0.005), "bf16": (0.015, 0.03)}


def gqa_sample(heads, length, start, seed, head_dim=128):
    h = np.arange(heads, dtype=np.uint64)[:, None, None]
    p = np.arange(start, start + length, dtype=np.uint64)[None, :, None]
    d = np.arange(head_dim, dtype=np.uint64)[None, None, :]
    m = np.uint64(0xFFFFFFFF)
    x = (np.uint64(seed) ^ ((h + 1) * np.uint64(0x9E3779B9) & m) ^ ((p + 1) * np.uint64(0x85EBCA6B) & m)
         ^ ((d + 1) * np.uint64(0xC2B2AE35) & m)) & m
    x ^= x >> np.uint64(16)
    x = (x * np.uint64(0x7FEB352D)) & m
    x ^= x >> np.uint64(15)
    return (((x & np.uint64(65535)).astype(np.int64) - 32768) / 32768.0).astype(np.float32)


def gqa_causal_case(length, seed, q_heads=32, kv_heads=8):
    q = gqa_sample(q_heads, length, 0, seed)
    k = gqa_sample(kv_heads, length, 0, seed + 1)
    v = gqa_sample(kv_heads, length, 0, seed + 2)
    pos = np.arange(length)
    mask = np.where(pos[None, :] <= pos[:, None], 0.0, -1e30).astype(np.float32)
    return q, k, v, mask


def gqa_causal_expected(q, k, v):
    q_heads, length, width = q.shape
    group = q_heads // k.shape[0]
    out = np.empty(q.shape, np.float64)
    for h in range(q_heads):
        kh, vh = k[h // group].astype(np.float64), v[h // group].astype(np.float64)
        for p in range(length):
            s = kh[:p + 1] @ q[h, p].astype(np.float64) / math.sqrt(width)
            w = np.exp(s - s.max())
            out[h, p] = (w @ vh[:p + 1]) / w.sum()
    return out
