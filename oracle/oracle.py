"""ctypes binding of the CPU oracle (test infrastructure only).

Loaded by the test suite, the smoke check and the CPU-baseline leg of the
benchmark -- never by the product library. Each wrapper names the reference
function it restates (see oracle.h for the file:line citations).
"""
import ctypes
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "liboracle.so"

_f32p = ctypes.POINTER(ctypes.c_float)
_lib = None


def build():
    subprocess.run(["make", "-s", "-C", str(HERE), "-j4"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        L = _lib
        L.orc_normal_fill.argtypes = [_f32p, ctypes.c_size_t, ctypes.c_uint64, ctypes.c_uint64, ctypes.c_float,
                                      ctypes.c_float]
        L.orc_timestep_features.argtypes = [ctypes.c_float, _f32p]
        L.orc_flow_schedule_turbo.argtypes = [ctypes.c_int, _f32p, _f32p]
        L.orc_euler_step.argtypes = [_f32p, _f32p, ctypes.c_float, ctypes.c_size_t, _f32p]
        L.orc_rope_frequencies.argtypes = [_f32p]
        L.orc_dit_constants.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, _f32p,
                                        _f32p]
        L.orc_rmsnorm.argtypes = [_f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, _f32p]
        L.orc_layernorm.argtypes = [_f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, _f32p]
        L.orc_modulate.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int]
        L.orc_gemm_nt.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int]
        L.orc_gelu.argtypes = [_f32p, ctypes.c_size_t, _f32p]
        L.orc_rope_rows.argtypes = [_f32p, _f32p, _f32p, ctypes.c_int, ctypes.c_long, ctypes.c_long]
        L.orc_sdpa.argtypes = [_f32p, _f32p, _f32p, _f32p] + [ctypes.c_int] * 5 + [ctypes.c_long] * 6 + [
            _f32p, ctypes.c_int, ctypes.c_int, ctypes.c_float, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_block_forward.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _f32p, _f32p, _f32p, _f32p, _f32p,
                                        ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int]
        L.orc_input_head.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int,
                                     _f32p, ctypes.c_int, _f32p, _f32p, _f32p, _f32p, ctypes.c_int]
        L.orc_output_head.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int,
                                      _f32p, _f32p, ctypes.c_int]
        L.orc_silu.argtypes = [_f32p, ctypes.c_size_t, _f32p]
        L.orc_text_constants.argtypes = [_f32p, ctypes.c_int, _f32p, _f32p, _f32p]
        L.orc_text_block_forward.argtypes = [ctypes.c_void_p] + [ctypes.c_int] * 4 + [_f32p] * 4 + [
            ctypes.c_int, _f32p, ctypes.c_int, ctypes.c_int]
        for name in ("orc_timestep_features", "orc_flow_schedule_turbo", "orc_dit_constants", "orc_block_forward",
                     "orc_input_head", "orc_output_head", "orc_text_constants", "orc_text_block_forward"):
            getattr(L, name).restype = ctypes.c_int
    return _lib


def _p(a):
    if a is None:
        return None
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], (a.dtype, a.flags)
    return a.ctypes.data_as(_f32p)


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- synthetic inputs -----------------------------------------------------
def normal(shape, seed, offset=0, mean=0.0, std=1.0):
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    lib().orc_normal_fill(_p(out), n, seed, offset, mean, std)
    return out.reshape(shape)


# ---- closed forms ------------------------------------------------------------
def timestep_features(t):
    out = np.empty(4096, np.float32)
    if lib().orc_timestep_features(float(t), _p(out)) != 0:
        raise ValueError("Timestep must be finite and in [0,1000]")
    return out


def flow_schedule_turbo(steps=8):
    sig = np.empty(steps + 1, np.float32)
    ts = np.empty(max(steps, 1), np.float32)
    if lib().orc_flow_schedule_turbo(steps, _p(sig), _p(ts)) != 0:
        raise ValueError("Steps must be in [1,1000]")
    return sig, ts[:steps]


def euler_step(x, v, delta):
    x, v = f32(x), f32(v)
    out = np.empty_like(x)
    lib().orc_euler_step(_p(x), _p(v), float(delta), x.size, _p(out))
    return out


def rope_frequencies():
    out = np.empty(64, np.float32)
    lib().orc_rope_frequencies(_p(out))
    return out


def dit_constants(freqs, w, h, valid, text):
    S = w * h + text
    cos = np.empty((S, 128), np.float32)
    sin = np.empty((S, 128), np.float32)
    mask = np.empty(S, np.float32)
    if lib().orc_dit_constants(_p(f32(freqs)), w, h, valid, text, _p(cos), _p(sin), _p(mask)) != 0:
        raise ValueError("Invalid DiT position dimensions or frequency table")
    return cos, sin, mask


# ---- operators -----------------------------------------------------------------
def rmsnorm(x, gamma, eps=1e-6):
    x = f32(x)
    width = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_rmsnorm(_p(x), _p(f32(gamma)) if gamma is not None else None, x.size // width, width, eps, _p(out))
    return out


def layernorm(x, eps=1e-6):
    x = f32(x)
    width = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_layernorm(_p(x), x.size // width, width, eps, _p(out))
    return out


def modulate(h, shift, scale):
    h = f32(h).copy()
    width = h.shape[-1]
    lib().orc_modulate(_p(h), _p(f32(shift)), _p(f32(scale)), h.size // width, width)
    return h


def gemm_nt(a, w, bias=None, threads=0):
    a, w = f32(a), f32(w)
    M, K = a.shape
    N = w.shape[0]
    assert w.shape[1] == K
    c = np.empty((M, N), np.float32)
    lib().orc_gemm_nt(_p(a), _p(w), _p(f32(bias)) if bias is not None else None, M, N, K, _p(c), threads)
    return c


def gelu(x):
    x = f32(x)
    out = np.empty_like(x)
    lib().orc_gelu(_p(x), x.size, _p(out))
    return out


def rope_rows(x, cos, sin):
    """x [rows][128] rotated with tables [rows][128]."""
    x = f32(x).copy()
    lib().orc_rope_rows(_p(x), _p(f32(cos)), _p(f32(sin)), x.shape[0], 128, 128)
    return x


def sdpa(q, k, v, mask=None, scale=None, q_range=None, precise=True, threads=0):
    """q [H][Sq][d], k/v [Hkv][Sk][d]; mask [mask_heads][rows][Sk] additive (rows 1 = broadcast)."""
    q, k, v = f32(q), f32(k), f32(v)
    H, Sq, d = q.shape
    Hkv, Sk, _ = k.shape
    scale = 1.0 / np.sqrt(d) if scale is None else scale
    q0, q1 = (0, Sq) if q_range is None else q_range
    out = np.zeros((H, Sq, d), np.float32)
    mh = mr = 1
    mp = None
    if mask is not None:
        mask = f32(mask)
        if mask.ndim == 1:
            mask = mask.reshape(1, 1, -1)
        elif mask.ndim == 2:
            mask = mask.reshape(1, *mask.shape)
        mh, mr = mask.shape[0], mask.shape[1]
        mp = _p(mask)
    lib().orc_sdpa(_p(q), _p(k), _p(v), _p(out), H, Hkv, Sq, Sk, d, Sq * d, d, Sk * d, d, Sq * d, d, mp, mh, mr,
                   float(scale), q0, q1, 1 if precise else 0, threads)
    return out


BLOCK_FIELDS = ("norm1", "wq", "wk", "wv", "norm_q", "norm_k", "wo", "norm2", "w_up", "w_gate", "w_down")


class _BlockWeights(ctypes.Structure):
    _fields_ = [(n, _f32p) for n in BLOCK_FIELDS]


def block_forward(weights, x, mods, cos, sin, mask, precise=True, threads=0):
    """weights: dict with BLOCK_FIELDS (FP32 arrays, [out][in] for matrices)."""
    keep = {n: f32(weights[n]) for n in BLOCK_FIELDS}
    st = _BlockWeights(*[_p(keep[n]) for n in BLOCK_FIELDS])
    x = f32(x)
    S, dim = x.shape
    ffn = keep["w_up"].shape[0]
    out = np.empty_like(x)
    rc = lib().orc_block_forward(ctypes.byref(st), dim, ffn, _p(x), _p(f32(mods)), _p(f32(cos)), _p(f32(sin)),
                                 _p(f32(mask)), S, _p(out), 1 if precise else 0, threads)
    if rc:
        raise ValueError("block_forward rejected its arguments")
    return out


INPUT_HEAD_FIELDS = ("x_w", "x_b", "text_w", "t1_w", "t1_b", "t2_w", "t2_b", "mod_w", "mod_b")
OUTPUT_HEAD_FIELDS = ("mod_w", "mod_b", "proj_w", "proj_b")


class _InputHead(ctypes.Structure):
    _fields_ = [(n, _f32p) for n in INPUT_HEAD_FIELDS]


class _OutputHead(ctypes.Structure):
    _fields_ = [(n, _f32p) for n in OUTPUT_HEAD_FIELDS]


def input_head(weights, latent, text, time_features, threads=0):
    keep = {n: f32(weights[n]) for n in INPUT_HEAD_FIELDS}
    st = _InputHead(*[_p(keep[n]) for n in INPUT_HEAD_FIELDS])
    latent, text = f32(latent), f32(text)
    ch = latent.shape[0]
    hw = latent[0].size
    dim = keep["x_w"].shape[0]
    T, text_dim = text.shape
    x = np.empty((hw + T, dim), np.float32)
    c = np.empty(dim, np.float32)
    mods = np.empty((6, dim), np.float32)
    rc = lib().orc_input_head(ctypes.byref(st), dim, ch, text_dim, _p(latent), hw, _p(text), T,
                              _p(f32(time_features)), _p(x), _p(c), _p(mods), threads)
    if rc:
        raise ValueError("input_head rejected its arguments")
    return x, c, mods


def output_head(weights, x, c, hw, threads=0):
    keep = {n: f32(weights[n]) for n in OUTPUT_HEAD_FIELDS}
    st = _OutputHead(*[_p(keep[n]) for n in OUTPUT_HEAD_FIELDS])
    x = f32(x)
    S, dim = x.shape
    ch = keep["proj_w"].shape[0]
    pred = np.empty((ch, hw), np.float32)
    rc = lib().orc_output_head(ctypes.byref(st), dim, ch, _p(x), S, hw, _p(f32(c)), _p(pred), threads)
    if rc:
        raise ValueError("output_head rejected its arguments")
    return pred


def silu(x):
    x = f32(x)
    out = np.empty_like(x)
    lib().orc_silu(_p(x), x.size, _p(out))
    return out


def text_constants(freqs, bucket):
    """64 YaRN inverse frequencies -> cos, sin [bucket][128], causal mask [bucket][bucket]."""
    cos = np.empty((bucket, 128), np.float32)
    sin = np.empty((bucket, 128), np.float32)
    mask = np.empty((bucket, bucket), np.float32)
    if lib().orc_text_constants(_p(f32(freqs)), bucket, _p(cos), _p(sin), _p(mask)):
        raise ValueError("text_constants rejected its arguments")
    return cos, sin, mask


TEXT_FIELDS = ("norm1", "wq", "wk", "wv", "wo", "norm2", "w_gate", "w_up", "w_down")


class _TextWeights(ctypes.Structure):
    _fields_ = [(n, _f32p) for n in TEXT_FIELDS]


def text_block_forward(weights, x, cos, sin, mask, heads, kv_heads, precise=True, threads=0):
    """weights: dict with TEXT_FIELDS (FP32, [out][in] for matrices); mask [S][S] or None."""
    keep = {n: f32(weights[n]) for n in TEXT_FIELDS}
    st = _TextWeights(*[_p(keep[n]) for n in TEXT_FIELDS])
    x = f32(x)
    S, hidden = x.shape
    ffn = keep["w_up"].shape[0]
    out = np.empty_like(x)
    rc = lib().orc_text_block_forward(ctypes.byref(st), hidden, heads, kv_heads, ffn, _p(x), _p(f32(cos)),
                                      _p(f32(sin)), None if mask is None else _p(f32(mask)), S, _p(out),
                                      1 if precise else 0, threads)
    if rc:
        raise ValueError("text_block_forward rejected its arguments")
    return out
