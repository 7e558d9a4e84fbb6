"""ctypes binding of the ernie_hip C ABI (include/ernie_hip.h) and the C entry
points of the C++ facade (include/ernie.h).

Device buffers are torch tensors on the HIP device (torch is only the
allocator/stream plumbing here); every computation runs in the in-tree gfx950
library. Loading fails loudly when the library has not been built -- there is
no other implementation behind this module.
"""
import ctypes
import re
from pathlib import Path

PKG = Path(__file__).resolve().parent.parent
ROOT = PKG.parent
LIB_DIR = PKG / "lib"
HIP_LIB = LIB_DIR / "libernie_hip.so"
FACADE_LIB = LIB_DIR / "libernie.so"
HEADERS = [ROOT / "include" / "ernie_hip.h", ROOT / "include" / "ernie.h"]

FP32, FP16, BF16 = 0, 1, 2
OK, ERROR, ALLOCATION_FAILED, INVALID_REQUEST = 0, -1, -100, -22
PROFILE_CLASSES = ("gemm_qkv", "sdpa", "gemm_out", "gemm_up_gate", "gemm_down", "rmsnorm_modulate", "qk_norm_rope",
                   "heads")

_hip = None
_facade = None

c_int, c_long, c_float, c_double, c_size_t, c_u64, c_vp = (ctypes.c_int, ctypes.c_long, ctypes.c_float,
                                                          ctypes.c_double, ctypes.c_size_t, ctypes.c_uint64,
                                                          ctypes.c_void_p)


class ErnieError(RuntimeError):
    def __init__(self, status, message):
        super().__init__(f"status {status}: {message}")
        self.status = status


class ErnieAllocationError(ErnieError):
    pass


class ErnieInvalidRequest(ErnieError, ValueError):
    pass


def build():
    import importlib.util
    spec = importlib.util.spec_from_file_location("ernie_build", PKG / "build.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.build()


def declared_functions():
    """Every function name declared in the public headers."""
    names = []
    for h in HEADERS:
        text = h.read_text()
        names += re.findall(r"^[A-Za-z_][\w\s\*]*?\b(ernie_\w+)\s*\(", text, flags=re.M)
    return sorted(set(names))


def hip():
    global _hip
    if _hip is None:
        if not HIP_LIB.exists():
            raise RuntimeError(f"{HIP_LIB} is missing: run `python {PKG / 'build.py'}` first")
        L = ctypes.CDLL(str(HIP_LIB), mode=ctypes.RTLD_GLOBAL)
        sig = {
            "ernie_hip_create": (c_int, [c_int, ctypes.POINTER(c_vp)]),
            "ernie_hip_destroy": (None, [c_vp]),
            "ernie_hip_last_error": (ctypes.c_char_p, [c_vp]),
            "ernie_hip_set_stream": (c_int, [c_vp, c_vp]),
            "ernie_hip_get_stream": (c_vp, [c_vp]),
            "ernie_hip_own_stream": (c_vp, [c_vp]),
            "ernie_hip_synchronize": (c_int, [c_vp]),
            "ernie_hip_malloc": (c_int, [c_vp, c_size_t, ctypes.POINTER(c_vp)]),
            "ernie_hip_free": (c_int, [c_vp, c_vp]),
            "ernie_hip_memcpy_h2d": (c_int, [c_vp, c_vp, c_vp, c_size_t]),
            "ernie_hip_memcpy_d2h": (c_int, [c_vp, c_vp, c_vp, c_size_t]),
            "ernie_hip_rmsnorm": (c_int, [c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_int, c_int, c_float, c_vp, c_int]),
            "ernie_hip_layernorm_modulate": (c_int, [c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_float, c_vp, c_int]),
            "ernie_hip_gelu": (c_int, [c_vp, c_vp, c_int, c_size_t]),
            "ernie_hip_residual_add": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_vp, c_size_t]),
            "ernie_hip_gemm": (c_int, [c_vp, c_vp, c_long, c_vp, c_long, c_vp, c_vp, c_long, c_int, c_int, c_int,
                                       c_int, c_int]),
            "ernie_hip_sdpa": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int] +
                               [c_long] * 8 + [c_vp, c_int, c_int, c_int, c_float]),
            "ernie_hip_set_attention_query_rows": (c_int, [c_vp, c_int]),
            "ernie_hip_attention_internal_submissions": (c_u64, [c_vp]),
            "ernie_hip_qk_norm_rope": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_long, c_vp, c_vp, c_vp]),
            "ernie_hip_euler_step": (c_int, [c_vp, c_vp, c_vp, c_float, c_size_t, c_vp]),
            "ernie_hip_finite": (c_int, [c_vp, c_vp, c_size_t, ctypes.POINTER(c_int)]),
            "ernie_hip_finite_begin": (c_int, [c_vp, c_vp, c_size_t, c_int]),
            "ernie_hip_finite_end": (c_int, [c_vp, c_int, ctypes.POINTER(c_int)]),
            "ernie_hip_marker_record": (c_int, [c_vp, c_int]),
            "ernie_hip_marker_elapsed": (c_int, [c_vp, c_int, c_int, ctypes.POINTER(c_double)]),
            "ernie_hip_trim": (c_size_t, [c_vp]),
            "ernie_hip_upload_async": (c_int, [c_vp, c_vp, c_vp, c_size_t]),
            "ernie_hip_transpose": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_vp]),
            "ernie_hip_fill_normal": (c_int, [c_vp, c_vp, c_int, c_size_t, c_u64, c_u64, c_float, c_float]),
            "ernie_hip_convert": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_size_t]),
            "ernie_hip_block_upload": (c_int, [c_vp, c_int, c_vp, c_int, c_int, c_int]),
            "ernie_hip_block_upload_tensors": (c_int, [c_vp, c_int, c_vp, c_int, c_int, c_int]),
            "ernie_hip_block_init_random": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_u64, c_float]),
            "ernie_hip_block_release": (c_int, [c_vp, c_int]),
            "ernie_hip_block_count": (c_int, [c_vp]),
            "ernie_hip_block_forward": (c_int, [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int]),
            "ernie_hip_block_sequence": (c_int, [c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int,
                                                 c_vp]),
            "ernie_hip_text_block_upload_tensors": (c_int, [c_vp, c_int, c_vp, c_int, c_int, c_int, c_int, c_int]),
            "ernie_hip_text_block_init_random": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_int, c_int, c_u64,
                                                         c_float]),
            "ernie_hip_text_block_release": (c_int, [c_vp, c_int]),
            "ernie_hip_text_block_forward_noalloc": (c_int, [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int,
                                                             c_int]),
            "ernie_hip_text_block_forward": (c_int, [c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int]),
            "ernie_hip_text_block_sequence": (c_int, [c_vp, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int,
                                                      c_vp]),
            "ernie_hip_sdpa_causal": (c_int, [c_vp, c_vp, c_vp, c_vp, c_vp, c_int, c_int, c_int, c_int, c_int, c_int] +
                                      [c_long] * 8 + [c_float]),
            "ernie_hip_heads_upload": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_int]),
            "ernie_hip_heads_init_random": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_u64, c_float]),
            "ernie_hip_input_head": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_vp]),
            "ernie_hip_output_head": (c_int, [c_vp, c_vp, c_int, c_int, c_vp, c_vp]),
            "ernie_hip_dit_forward": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_vp, c_int, c_vp,
                                              c_int, c_vp]),
            "ernie_hip_profile_enable": (c_int, [c_vp, c_int]),
            "ernie_hip_profile_classes": (c_int, [c_vp, ctypes.c_uint]),
            "ernie_hip_profile_stride": (c_int, [c_vp, c_int]),
            "ernie_hip_profile_collect": (c_int, [c_vp]),
            "ernie_hip_profile_reset": (c_int, [c_vp]),
            "ernie_hip_profile_query": (c_int, [c_vp, c_int, ctypes.POINTER(c_long), ctypes.POINTER(c_double),
                                                ctypes.POINTER(c_double), ctypes.POINTER(c_double)]),
            "ernie_hip_heads_upload_tensors": (c_int, [c_vp, c_vp, c_int, c_int, c_int, c_int, c_int]),
            "ernie_hip_heads_loaded": (c_int, [c_vp]),
            "ernie_hip_set_qk_rounding": (c_int, [c_vp, c_int]),
            "ernie_hip_mfma_rate": (c_int, [c_vp, c_int, c_int, ctypes.POINTER(c_double), ctypes.POINTER(c_double),
                                            ctypes.POINTER(c_double)]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _hip = L
    return _hip


class BlockFileInfo(ctypes.Structure):
    """ernie_block_file_info (include/ernie.h)."""
    _fields_ = [("tokens", c_int), ("dim", c_int), ("ffn", c_int), ("contract", c_int),
                ("component_sha256", ctypes.c_char * 65), ("runtime_sha256", ctypes.c_char * 65),
                ("bin_bytes", c_size_t), ("section_count", c_int), ("section_dtype", c_int * 11),
                ("section_begin", c_size_t * 11), ("section_data", c_size_t * 11), ("section_end", c_size_t * 11)]

    def as_dict(self):
        n = self.section_count
        return {"tokens": self.tokens, "dim": self.dim, "ffn": self.ffn,
                "contract": GRAPH_CONTRACTS[self.contract],
                "component_sha256": self.component_sha256.decode(), "runtime_sha256": self.runtime_sha256.decode(),
                "bin_bytes": self.bin_bytes,
                "sections": [{"layer": BLOCK_WEIGHT_LAYERS[i], "dtype": self.section_dtype[i],
                              "begin": self.section_begin[i], "data": self.section_data[i],
                              "end": self.section_end[i]} for i in range(n)]}


class HostTensor(ctypes.Structure):
    """ernie_host_tensor (include/ernie_hip.h)."""
    _fields_ = [("data", c_vp), ("dtype", c_int)]


class OpBlob(ctypes.Structure):
    """ernie_op_blob (include/ernie.h)."""
    _fields_ = [("data", c_vp), ("dtype", c_int), ("w", c_int), ("h", c_int), ("c", c_int)]


# ernie_stage_observer / ernie_step_observer (include/ernie.h).
STAGE_OBSERVER = ctypes.CFUNCTYPE(None, ctypes.c_char_p, c_vp, c_int, c_int, c_int, c_vp)
STEP_OBSERVER = ctypes.CFUNCTYPE(None, c_int, c_vp, c_vp, c_size_t, c_vp)

GRAPH_CONTRACTS = ("unreviewed", "component", "runtime")
# Weighted layers of a block graph in .bin order (tools/build_dit_weights.py:19-31).
BLOCK_WEIGHT_LAYERS = ("rmsn_8", "gemm_0", "gemm_1", "gemm_2", "rmsn_9", "rmsn_10", "gemm_3", "rmsn_11", "gemm_4",
                       "gemm_5", "gemm_6")


def facade():
    global _facade
    if _facade is None:
        hip()
        if not FACADE_LIB.exists():
            raise RuntimeError(f"{FACADE_LIB} is missing: run `python {PKG / 'build.py'}` first")
        L = ctypes.CDLL(str(FACADE_LIB))
        cp = ctypes.c_char_p
        sig = {
            "ernie_device_create": (c_int, [c_int, ctypes.POINTER(c_vp)]),
            "ernie_device_destroy": (None, [c_vp]),
            "ernie_device_ctx": (c_vp, [c_vp]),
            "ernie_timestep_features": (c_int, [c_float, c_vp, cp, c_size_t]),
            "ernie_flow_schedule_turbo": (c_int, [c_int, c_vp, c_vp, cp, c_size_t]),
            "ernie_rope_frequencies": (c_int, [c_vp]),
            "ernie_dit_constants": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_vp, c_vp, c_vp, cp, c_size_t]),
            "ernie_dit_constants_file": (c_int, [ctypes.c_char_p, c_int, c_int, c_int, c_int, c_vp, c_vp, c_vp, cp,
                                                 c_size_t]),
            "ernie_pad_text": (c_int, [c_vp, c_int, c_int, c_vp, cp, c_size_t]),
            "ernie_run_block_sequence": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_int, c_vp, c_vp, c_vp, c_vp, c_int,
                                                 c_int, c_vp, c_vp, cp, c_size_t]),
            "ernie_denoise": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_int, c_vp, c_int, c_vp, c_vp, c_vp, c_int,
                                      c_int, c_int, c_int, c_vp, c_vp, cp, c_size_t]),
            "ernie_denoise_observed": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_int, c_vp, c_int, c_vp, c_vp, c_vp,
                                               c_int, c_int, c_int, c_int, c_int, c_vp, c_vp, STEP_OBSERVER, c_vp,
                                               cp, c_size_t]),
            "ernie_run_dit": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_int, c_vp, c_int, c_vp, c_int, c_vp, c_vp,
                                      c_vp, c_int, c_int, c_vp, c_vp, STAGE_OBSERVER, c_vp, cp, c_size_t]),
            "ernie_op_forward": (c_int, [c_vp, cp, cp, c_vp, c_size_t, ctypes.POINTER(OpBlob), c_int,
                                         ctypes.POINTER(OpBlob), c_int, cp, c_size_t]),
            "ernie_text_constants": (c_int, [c_vp, c_int, c_vp, c_vp, c_vp, cp, c_size_t]),
            "ernie_text_embeddings": (c_int, [c_vp, c_size_t, c_int, c_vp, c_int, c_int, c_vp, cp, c_size_t]),
            "ernie_run_text_blocks": (c_int, [c_vp, c_vp, c_int, c_vp, c_int, c_int, c_vp, c_vp, c_vp, c_int, c_int,
                                              c_vp, c_vp, cp, c_size_t]),
            "ernie_sha256_hex": (c_int, [c_vp, c_size_t, cp]),
            "ernie_block_file_inspect": (c_int, [cp, cp, c_int, cp, ctypes.POINTER(BlockFileInfo), cp, c_size_t]),
            "ernie_block_load": (c_int, [c_vp, c_int, cp, cp, c_int, c_int, cp, ctypes.POINTER(BlockFileInfo), cp,
                                         c_size_t]),
            "ernie_head_file_inspect": (c_int, [cp, cp, c_int, cp, ctypes.POINTER(HeadFileInfo), cp, c_size_t]),
            "ernie_head_load": (c_int, [c_vp, cp, cp, c_int, c_int, cp, ctypes.POINTER(HeadFileInfo), cp, c_size_t]),
            "ernie_text_block_file_inspect": (c_int, [cp, cp, c_int, cp, ctypes.POINTER(TextBlockFileInfo), cp,
                                                      c_size_t]),
            "ernie_text_block_load": (c_int, [c_vp, c_int, cp, cp, c_int, c_int, cp,
                                              ctypes.POINTER(TextBlockFileInfo), cp, c_size_t]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _facade = L
    return _facade


def _raise(status, message):
    msg = message.decode() if isinstance(message, bytes) else str(message)
    if status == ALLOCATION_FAILED:
        raise ErnieAllocationError(status, msg)
    if status == INVALID_REQUEST:
        raise ErnieInvalidRequest(status, msg)
    raise ErnieError(status, msg)


def ptr(t):
    """Device (or host numpy) pointer of a tensor / array, None passes through."""
    if t is None:
        return None
    if isinstance(t, int):
        return t
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


# ---- host helpers of the facade (no device needed) -------------------------------
def _err():
    return ctypes.create_string_buffer(512)


def timestep_features(t):
    import numpy as np
    out = np.empty(4096, np.float32)
    e = _err()
    rc = facade().ernie_timestep_features(float(t), out.ctypes.data, e, 512)
    if rc:
        _raise(rc, e.value)
    return out


def flow_schedule_turbo(steps=8):
    import numpy as np
    sig = np.empty(steps + 1 if steps > 0 else 1, np.float32)
    ts = np.empty(max(steps, 1), np.float32)
    e = _err()
    rc = facade().ernie_flow_schedule_turbo(int(steps), sig.ctypes.data, ts.ctypes.data, e, 512)
    if rc:
        _raise(rc, e.value)
    return sig, ts[:steps]


def rope_frequencies():
    import numpy as np
    out = np.empty(64, np.float32)
    facade().ernie_rope_frequencies(out.ctypes.data)
    return out


def dit_constants(freqs, w, h, valid, text):
    import numpy as np
    freqs = np.ascontiguousarray(freqs, np.float32)
    S = w * h + text
    cos = np.empty((max(S, 1), 128), np.float32)
    sin = np.empty((max(S, 1), 128), np.float32)
    mask = np.empty(max(S, 1), np.float32)
    e = _err()
    rc = facade().ernie_dit_constants(freqs.ctypes.data, w, h, valid, text, cos.ctypes.data, sin.ctypes.data,
                                      mask.ctypes.data, e, 512)
    if rc < 0:
        _raise(rc, e.value)
    return cos, sin, mask, rc


def dit_constants_file(path, w, h, valid, text):
    """Facade dit_constants from the reference's 256-byte frequency file (token limit 6144)."""
    import numpy as np
    S = max(w * h + text, 1)
    cos = np.empty((S, 128), np.float32)
    sin = np.empty((S, 128), np.float32)
    mask = np.empty(S, np.float32)
    e = _err()
    rc = facade().ernie_dit_constants_file(str(path).encode(), w, h, valid, text, cos.ctypes.data, sin.ctypes.data,
                                           mask.ctypes.data, e, 512)
    if rc < 0:
        _raise(rc, e.value)
    return cos, sin, mask, rc


def pad_text(embeddings, bucket):
    """Facade pad_text: [tokens][3072] FP32 embeddings zero-padded to [bucket][3072]."""
    import numpy as np
    emb = np.ascontiguousarray(embeddings, np.float32)
    if emb.ndim != 2 or emb.shape[1] != 3072:
        raise ValueError("embeddings must be [tokens][3072]")
    out = np.empty((max(bucket, 1), 3072), np.float32)
    e = _err()
    rc = facade().ernie_pad_text(emb.ctypes.data, emb.shape[0], bucket, out.ctypes.data, e, 512)
    if rc < 0:
        _raise(rc, e.value)
    return out


def text_constants(freqs, bucket):
    """Facade text_constants: 64 YaRN inverse frequencies -> cos, sin [bucket][128], mask [bucket][bucket]."""
    import numpy as np
    freqs = np.ascontiguousarray(freqs, np.float32)
    if freqs.size != 64:
        raise ValueError("expected 64 inverse frequencies")
    n = max(bucket, 1)
    cos = np.empty((n, 128), np.float32)
    sin = np.empty((n, 128), np.float32)
    mask = np.empty((n, n), np.float32)
    e = _err()
    rc = facade().ernie_text_constants(freqs.ctypes.data, bucket, cos.ctypes.data, sin.ctypes.data, mask.ctypes.data,
                                       e, 512)
    if rc < 0:
        _raise(rc, e.value)
    return cos, sin, mask


def text_embeddings(table_bf16, ids, bucket):
    """Facade text_embeddings over an in-memory BF16 table (uint16 [vocabulary][width])."""
    import numpy as np
    table = np.ascontiguousarray(table_bf16, np.uint16)
    ids = np.ascontiguousarray(ids, np.uint32)
    out = np.empty((max(bucket, 1), table.shape[1]), np.float32)
    e = _err()
    rc = facade().ernie_text_embeddings(table.ctypes.data, table.shape[0], table.shape[1], ids.ctypes.data, ids.size,
                                        bucket, out.ctypes.data, e, 512)
    if rc < 0:
        _raise(rc, e.value)
    return out


def sha256_hex(data):
    """SHA-256 of a bytes-like object through the facade's own implementation."""
    buf = bytes(data)
    out = ctypes.create_string_buffer(65)
    rc = facade().ernie_sha256_hex(buf, len(buf), out)
    if rc:
        _raise(rc, "sha256")
    return out.value.decode()


def _path(p):
    return None if p is None else str(p).encode()


HEAD_INPUT, HEAD_OUTPUT = 1, 2
HEAD_SECTIONS = {HEAD_INPUT: ("conv_1", "conv_1.bias", "gemm_0", "linear_2", "linear_2.bias", "linear_3",
                              "linear_3.bias", "linear_4", "linear_4.bias"),
                 HEAD_OUTPUT: ("linear_2", "linear_2.bias", "gemm_0", "gemm_0.bias")}
TEXT_WEIGHT_LAYERS = ("rmsn_8", "gemm_0", "gemm_1", "gemm_2", "gemm_3", "rmsn_9", "gemm_4", "gemm_5", "gemm_6")


def _sections(info, names):
    return [{"layer": names[i], "dtype": info.section_dtype[i], "begin": info.section_begin[i],
             "data": info.section_data[i], "end": info.section_end[i]} for i in range(info.section_count)]


class HeadFileInfo(ctypes.Structure):
    """ernie_head_file_info (include/ernie.h)."""
    _fields_ = [("part", c_int), ("dim", c_int), ("latent_ch", c_int), ("text_dim", c_int), ("text_tokens", c_int),
                ("image_tokens", c_int), ("tokens", c_int), ("width", c_int), ("height", c_int),
                ("reviewed", c_int), ("contract_sha256", ctypes.c_char * 65), ("bin_bytes", c_size_t),
                ("section_count", c_int), ("section_dtype", c_int * 9), ("section_begin", c_size_t * 9),
                ("section_data", c_size_t * 9), ("section_end", c_size_t * 9)]

    def as_dict(self):
        d = {k: getattr(self, k) for k in ("part", "dim", "latent_ch", "text_dim", "text_tokens", "image_tokens",
                                           "tokens", "width", "height", "bin_bytes")}
        d["reviewed"] = bool(self.reviewed)
        d["contract_sha256"] = self.contract_sha256.decode()
        d["sections"] = _sections(self, HEAD_SECTIONS.get(self.part, ()))
        return d


class TextBlockFileInfo(ctypes.Structure):
    """ernie_text_block_file_info (include/ernie.h)."""
    _fields_ = [("tokens", c_int), ("hidden", c_int), ("heads", c_int), ("kv_heads", c_int), ("ffn", c_int),
                ("reviewed", c_int), ("contract_sha256", ctypes.c_char * 65), ("bin_bytes", c_size_t),
                ("section_count", c_int), ("section_dtype", c_int * 9), ("section_begin", c_size_t * 9),
                ("section_data", c_size_t * 9), ("section_end", c_size_t * 9)]

    def as_dict(self):
        d = {k: getattr(self, k) for k in ("tokens", "hidden", "heads", "kv_heads", "ffn", "bin_bytes")}
        d["reviewed"] = bool(self.reviewed)
        d["contract_sha256"] = self.contract_sha256.decode()
        d["sections"] = _sections(self, TEXT_WEIGHT_LAYERS)
        return d


def head_file_inspect(param_path, bin_path=None, allow_unreviewed=False, expected_bin_sha256=None):
    """Checks a DiT head.ncnn.param (and walks head.ncnn.bin when given) without a device."""
    info = HeadFileInfo()
    e = _err()
    rc = facade().ernie_head_file_inspect(_path(param_path), _path(bin_path), int(bool(allow_unreviewed)),
                                          _path(expected_bin_sha256), ctypes.byref(info), e, 512)
    if rc:
        _raise(rc, e.value)
    return info.as_dict()


def text_block_file_inspect(param_path, bin_path=None, allow_unreviewed=False, expected_bin_sha256=None):
    """Checks a text.ncnn.param (and walks text.ncnn.bin when given) without a device."""
    info = TextBlockFileInfo()
    e = _err()
    rc = facade().ernie_text_block_file_inspect(_path(param_path), _path(bin_path), int(bool(allow_unreviewed)),
                                                _path(expected_bin_sha256), ctypes.byref(info), e, 512)
    if rc:
        _raise(rc, e.value)
    return info.as_dict()


def block_file_inspect(param_path, bin_path=None, allow_unreviewed=False, expected_bin_sha256=None):
    """Checks block.ncnn.param (and walks block.ncnn.bin when given) without a device."""
    info = BlockFileInfo()
    e = _err()
    rc = facade().ernie_block_file_inspect(_path(param_path), _path(bin_path), int(bool(allow_unreviewed)),
                                           _path(expected_bin_sha256), ctypes.byref(info), e, 512)
    if rc:
        _raise(rc, e.value)
    return info.as_dict()


class Context:
    """One ernie_hip context bound to torch's current stream on `device`."""

    def __init__(self, device=0, use_torch_stream=True):
        L = hip()
        p = c_vp()
        rc = L.ernie_hip_create(device, ctypes.byref(p))
        if rc:
            raise ErnieError(rc, f"ernie_hip_create({device}) failed: no usable HIP device")
        self.ctx = p.value
        self.L = L
        if use_torch_stream:
            import torch
            L.ernie_hip_set_stream(self.ctx, c_vp(torch.cuda.current_stream().cuda_stream))

    def close(self):
        if self.ctx:
            self.L.ernie_hip_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def check(self, rc):
        if rc:
            _raise(rc, self.L.ernie_hip_last_error(self.ctx) or b"")
        return rc

    def call(self, name, *args):
        return self.check(getattr(self.L, "ernie_hip_" + name)(self.ctx, *args))

    def synchronize(self):
        self.call("synchronize")

    # ---- ops -------------------------------------------------------------
    def rmsnorm(self, x, x_dtype, gamma, rows, width, out, out_dtype, shift=None, scale=None, eps=1e-6):
        self.call("rmsnorm", ptr(x), x_dtype, ptr(gamma), ptr(shift), ptr(scale), rows, width, eps, ptr(out),
                  out_dtype)

    def layernorm_modulate(self, x, shift, scale, rows, width, out, out_dtype, eps=1e-6):
        self.call("layernorm_modulate", ptr(x), ptr(shift), ptr(scale), rows, width, eps, ptr(out), out_dtype)

    def gelu(self, x, dtype, count):
        self.call("gelu", ptr(x), dtype, count)

    def residual_add(self, a, adt, b, bdt, out, count):
        self.call("residual_add", ptr(a), adt, ptr(b), bdt, ptr(out), count)

    def gemm(self, a, lda, w, ldw, c, ldc, m, n, k, dtype, out_dtype, bias=None):
        self.call("gemm", ptr(a), lda, ptr(w), ldw, ptr(bias), ptr(c), ldc, m, n, k, dtype, out_dtype)

    def sdpa(self, q, k, v, out, dtype, heads, kv_heads, sq, sk, d, strides, mask=None, mask_heads=1, mask_rows=1,
             valid_keys=0, scale=0.0):
        self.call("sdpa", ptr(q), ptr(k), ptr(v), ptr(out), dtype, heads, kv_heads, sq, sk, d, *strides, ptr(mask),
                  mask_heads, mask_rows, valid_keys, scale)

    def qk_norm_rope(self, x, dtype, rows, heads, row_stride, gamma, cos, sin):
        self.call("qk_norm_rope", ptr(x), dtype, rows, heads, row_stride, ptr(gamma), ptr(cos), ptr(sin))

    def euler_step(self, x, v, delta, count, out):
        self.call("euler_step", ptr(x), ptr(v), delta, count, ptr(out))

    def finite(self, x, count):
        f = c_int()
        self.call("finite", ptr(x), count, ctypes.byref(f))
        return bool(f.value)

    def finite_begin(self, x, count, slot):
        self.call("finite_begin", ptr(x), count, slot)

    def finite_end(self, slot):
        f = c_int()
        self.call("finite_end", slot, ctypes.byref(f))
        return bool(f.value)

    def marker(self, index):
        self.call("marker_record", index)

    def marker_elapsed(self, first, last):
        s = c_double()
        self.call("marker_elapsed", first, last, ctypes.byref(s))
        return s.value

    def trim(self):
        return int(self.L.ernie_hip_trim(self.ctx))

    def fill_normal(self, out, dtype, count, seed, offset=0, mean=0.0, std=1.0):
        self.call("fill_normal", ptr(out), dtype, count, seed, offset, mean, std)

    # ---- blocks / heads -----------------------------------------------------
    def block_upload(self, index, weights, dim, ffn, dtype):
        """weights: dict of FP32 numpy arrays keyed like ernie_block_host_weights."""
        import numpy as np
        fields = ("norm1", "wq", "wk", "wv", "norm_q", "norm_k", "wo", "norm2", "w_up", "w_gate", "w_down")
        keep = [np.ascontiguousarray(weights[f], np.float32) for f in fields]
        arr = (c_vp * len(fields))(*[a.ctypes.data for a in keep])
        self.call("block_upload", index, ctypes.cast(arr, c_vp), dim, ffn, dtype)

    def block_upload_tensors(self, index, tensors, dim, ffn, dtype):
        """tensors: dict field -> (numpy array, element dtype); FP16/BF16 arrays hold raw uint16 bits."""
        import numpy as np
        fields = ("norm1", "wq", "wk", "wv", "norm_q", "norm_k", "wo", "norm2", "w_up", "w_gate", "w_down")
        keep = [np.ascontiguousarray(tensors[f][0]) for f in fields]
        arr = (HostTensor * len(fields))(*[HostTensor(a.ctypes.data, tensors[f][1]) for a, f in zip(keep, fields)])
        self.call("block_upload_tensors", index, ctypes.cast(arr, c_vp), dim, ffn, dtype)

    def block_init_random(self, index, dim, ffn, dtype, seed, std=0.02):
        self.call("block_init_random", index, dim, ffn, dtype, seed, std)

    def block_forward(self, index, x, out, mods, cos, sin, S, mask=None, valid_keys=0):
        self.call("block_forward", index, ptr(x), ptr(out), ptr(mods), ptr(cos), ptr(sin), ptr(mask), valid_keys, S)

    def block_sequence(self, blocks, x, out, mods, cos, sin, S, mask=None, valid_keys=0, timing=False):
        import numpy as np
        ids = (c_int * len(blocks))(*blocks)
        secs = np.zeros(len(blocks), np.float64) if timing else None
        self.call("block_sequence", ctypes.cast(ids, c_vp), len(blocks), ptr(x), ptr(out), ptr(mods), ptr(cos),
                  ptr(sin), ptr(mask), valid_keys, S, secs.ctypes.data if timing else None)
        return secs

    # ---- Mistral text blocks --------------------------------------------------
    TEXT_FIELDS = ("norm1", "wq", "wk", "wv", "wo", "norm2", "w_gate", "w_up", "w_down")

    def text_block_upload(self, index, weights, hidden, heads, kv_heads, ffn, dtype):
        """weights: dict of FP32 numpy arrays keyed like TEXT_FIELDS ([out][in] matrices)."""
        import numpy as np
        return self.text_block_upload_tensors(
            index, {f: (np.ascontiguousarray(weights[f], np.float32), FP32) for f in self.TEXT_FIELDS}, hidden,
            heads, kv_heads, ffn, dtype)

    def text_block_upload_tensors(self, index, tensors, hidden, heads, kv_heads, ffn, dtype):
        """tensors: dict field -> (numpy array, element dtype); FP16/BF16 arrays hold raw uint16 bits."""
        import numpy as np
        keep = [np.ascontiguousarray(tensors[f][0]) for f in self.TEXT_FIELDS]
        arr = (HostTensor * len(keep))(*[HostTensor(a.ctypes.data, tensors[f][1])
                                         for a, f in zip(keep, self.TEXT_FIELDS)])
        self.call("text_block_upload_tensors", index, ctypes.cast(arr, c_vp), hidden, heads, kv_heads, ffn, dtype)

    def text_block_init_random(self, index, hidden, heads, kv_heads, ffn, dtype, seed, std=0.02):
        self.call("text_block_init_random", index, hidden, heads, kv_heads, ffn, dtype, seed, std)

    def text_block_forward(self, index, x, out, cos, sin, S, mask=None, causal=False):
        self.call("text_block_forward", index, ptr(x), ptr(out), ptr(cos), ptr(sin), ptr(mask), 1 if causal else 0, S)

    def text_block_sequence(self, blocks, x, out, cos, sin, S, mask=None, causal=False, timing=False):
        import numpy as np
        ids = (c_int * len(blocks))(*blocks)
        secs = np.zeros(len(blocks), np.float64) if timing else None
        self.call("text_block_sequence", ctypes.cast(ids, c_vp), len(blocks), ptr(x), ptr(out), ptr(cos), ptr(sin),
                  ptr(mask), 1 if causal else 0, S, secs.ctypes.data if timing else None)
        return secs

    def sdpa_causal(self, q, k, v, out, dtype, heads, kv_heads, sq, sk, d, strides, scale=0.0):
        self.call("sdpa_causal", ptr(q), ptr(k), ptr(v), ptr(out), dtype, heads, kv_heads, sq, sk, d, *strides, scale)

    def heads_upload(self, weights, dim, latent_ch, text_dim, dtype):
        import numpy as np
        fields = ("x_w", "x_b", "text_w", "t1_w", "t1_b", "t2_w", "t2_b", "mod_w", "mod_b", "out_mod_w",
                  "out_mod_b", "proj_w", "proj_b")
        keep = [np.ascontiguousarray(weights[f], np.float32) for f in fields]
        arr = (c_vp * len(fields))(*[a.ctypes.data for a in keep])
        self.call("heads_upload", ctypes.cast(arr, c_vp), dim, latent_ch, text_dim, dtype)

    HEAD_FIELDS = ("x_w", "x_b", "text_w", "t1_w", "t1_b", "t2_w", "t2_b", "mod_w", "mod_b", "out_mod_w",
                   "out_mod_b", "proj_w", "proj_b")

    def heads_upload_tensors(self, tensors, dim, latent_ch, text_dim, dtype, parts=3):
        """ernie_hip_heads_upload_tensors: tensors maps HEAD_FIELDS names to (numpy array, element dtype) (FP16 /
        BF16 arrays hold raw uint16 bits); the fields of a part not in `parts` may be absent."""
        import numpy as np
        keep = {f: np.ascontiguousarray(tensors[f][0]) for f in self.HEAD_FIELDS if f in tensors}
        arr = (HostTensor * len(self.HEAD_FIELDS))(*[
            HostTensor(keep[f].ctypes.data, tensors[f][1]) if f in keep else HostTensor(None, FP32)
            for f in self.HEAD_FIELDS])
        self.call("heads_upload_tensors", ctypes.cast(arr, c_vp), dim, latent_ch, text_dim, dtype, parts)

    def heads_loaded(self):
        return self.L.ernie_hip_heads_loaded(self.ctx)

    def heads_init_random(self, dim, latent_ch, text_dim, dtype, seed, std=0.02):
        self.call("heads_init_random", dim, latent_ch, text_dim, dtype, seed, std)

    def input_head(self, latent, hw, text, text_tokens, features, x, c, mods):
        self.call("input_head", ptr(latent), hw, ptr(text), text_tokens, ptr(features), ptr(x), ptr(c), ptr(mods))

    def output_head(self, x, S, hw, c, pred):
        self.call("output_head", ptr(x), S, hw, ptr(c), ptr(pred))

    def dit_forward(self, latent, hw, text, text_tokens, features, cos, sin, blocks, pred, mask=None, valid_keys=0):
        ids = (c_int * len(blocks))(*blocks)
        self.call("dit_forward", ptr(latent), hw, ptr(text), text_tokens, ptr(features), ptr(cos), ptr(sin),
                  ptr(mask), valid_keys, ctypes.cast(ids, c_vp), len(blocks), ptr(pred))

    # ---- profiling -----------------------------------------------------------
    def profile(self, enable, classes=None, stride=1):
        """Event timing on/off; `classes` (names from PROFILE_CLASSES) limits which launches are
        bracketed, `stride` brackets only every stride-th launch of each of them."""
        mask = 0xFFFFFFFF if classes is None else sum(1 << PROFILE_CLASSES.index(c) for c in classes)
        self.call("profile_classes", mask)
        self.call("profile_stride", stride)
        self.call("profile_enable", 1 if enable else 0)

    def profile_reset(self):
        self.call("profile_reset")

    def profile_query(self):
        self.call("profile_collect")
        out = {}
        for i, name in enumerate(PROFILE_CLASSES):
            n, ms, fl, by = c_long(), c_double(), c_double(), c_double()
            self.call("profile_query", i, ctypes.byref(n), ctypes.byref(ms), ctypes.byref(fl), ctypes.byref(by))
            out[name] = {"launches": n.value, "ms": ms.value, "flop": fl.value, "bytes": by.value}
        return out

    def mfma_rate(self, iters=4096, launches=10):
        """The device's measured dense FP16 MFMA ceiling (ernie_hip_mfma_rate): FLOP/s over
        `launches` timed launches, their seconds, and the shader clock in Hz."""
        f, hz, s = c_double(), c_double(), c_double()
        self.call("mfma_rate", iters, launches, ctypes.byref(f), ctypes.byref(hz), ctypes.byref(s))
        return {"flop_per_s": f.value, "clock_hz": hz.value, "seconds": s.value}


class Facade:
    """ernie::Device plus the C entry points of the C++ facade."""

    def __init__(self, device=0):
        L = facade()
        p = c_vp()
        rc = L.ernie_device_create(device, ctypes.byref(p))
        if rc:
            raise ErnieError(rc, "ernie_device_create failed: no usable HIP device")
        self.dev = p.value
        self.L = L
        self.hip = Context.__new__(Context)
        self.hip.ctx = L.ernie_device_ctx(self.dev)
        self.hip.L = hip()
        import torch
        hip().ernie_hip_set_stream(self.hip.ctx, c_vp(torch.cuda.current_stream().cuda_stream))

    def close(self):
        if self.dev:
            self.hip.ctx = None
            self.L.ernie_device_destroy(self.dev)
            self.dev = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def run_block_sequence(self, blocks, x, S, dim, mods, cos, sin, out, mask=None, valid_prefix=0, dtype=FP32):
        import numpy as np
        ids = (c_int * len(blocks))(*blocks)
        mp = (c_vp * 6)(*[ptr(m) for m in mods])
        secs = np.zeros(max(len(blocks), 1), np.float64)
        e = _err()
        rc = self.L.ernie_run_block_sequence(self.dev, ctypes.cast(ids, c_vp), len(blocks), ptr(x), S, dim,
                                             ctypes.cast(mp, c_vp), ptr(cos), ptr(sin), ptr(mask), valid_prefix,
                                             dtype, ptr(out), secs.ctypes.data, e, 512)
        if rc:
            _raise(rc, e.value)
        return secs[:len(blocks)]

    def block_load(self, index, param_path, bin_path, dtype, allow_unreviewed=False, expected_bin_sha256=None):
        """Loads block.ncnn.param + block.ncnn.bin into resident block slot `index`."""
        info = BlockFileInfo()
        e = _err()
        rc = self.L.ernie_block_load(self.dev, index, _path(param_path), _path(bin_path), dtype,
                                     int(bool(allow_unreviewed)), _path(expected_bin_sha256), ctypes.byref(info), e,
                                     512)
        if rc:
            _raise(rc, e.value)
        return info.as_dict()

    def head_load(self, param_path, bin_path, dtype, allow_unreviewed=False, expected_bin_sha256=None):
        """Loads a DiT head.ncnn.param + head.ncnn.bin (input or output head, as the graph says)."""
        info = HeadFileInfo()
        e = _err()
        rc = self.L.ernie_head_load(self.dev, _path(param_path), _path(bin_path), dtype, int(bool(allow_unreviewed)),
                                    _path(expected_bin_sha256), ctypes.byref(info), e, 512)
        if rc:
            _raise(rc, e.value)
        return info.as_dict()

    def text_block_load(self, index, param_path, bin_path, dtype, allow_unreviewed=False, expected_bin_sha256=None):
        """Loads text.ncnn.param + text.ncnn.bin into resident text block slot `index`."""
        info = TextBlockFileInfo()
        e = _err()
        rc = self.L.ernie_text_block_load(self.dev, index, _path(param_path), _path(bin_path), dtype,
                                          int(bool(allow_unreviewed)), _path(expected_bin_sha256),
                                          ctypes.byref(info), e, 512)
        if rc:
            _raise(rc, e.value)
        return info.as_dict()

    def run_text_blocks(self, blocks, x, S, width, cos, sin, mask, out, dtype=FP32, causal=False):
        import numpy as np
        ids = (c_int * len(blocks))(*blocks)
        secs = np.zeros(len(blocks), np.float64)
        e = _err()
        rc = self.L.ernie_run_text_blocks(self.dev, ctypes.cast(ids, c_vp), len(blocks), ptr(x), S, width, ptr(cos),
                                          ptr(sin), ptr(mask), 1 if causal else 0, dtype, ptr(out), secs.ctypes.data,
                                          e, 512)
        if rc < 0:
            _raise(rc, e.value)
        return secs

    def op_forward(self, op_type, params, inputs, outputs=(), weights=None):
        """One registered op (ernie_op_forward). inputs / outputs: (tensor, dtype, w, h, c) tuples."""
        import numpy as np
        w = None if weights is None else np.ascontiguousarray(weights, np.float32)
        ins = (OpBlob * max(len(inputs), 1))(*[OpBlob(ptr(t), dt, a, b, c) for t, dt, a, b, c in inputs])
        outs = (OpBlob * max(len(outputs), 1))(*[OpBlob(ptr(t), dt, a, b, c) for t, dt, a, b, c in outputs])
        e = _err()
        rc = self.L.ernie_op_forward(self.dev, op_type.encode(), params.encode(), None if w is None else w.ctypes.data,
                                     0 if w is None else w.size, ins, len(inputs), outs, len(outputs), e, 512)
        if rc:
            _raise(rc, e.value)

    def run_dit(self, blocks, latent, height, width, text, text_tokens, features, dim, cos, sin, prediction,
                mask=None, valid_prefix=0, dtype=FP16, timing=False, observer=None):
        """Facade run_dit; observer(stage, device_ptr, w, h, c) is called per stage."""
        import numpy as np
        ids = (c_int * max(len(blocks), 1))(*blocks)
        secs = np.zeros(max(len(blocks), 1), np.float64) if timing else None
        cb = STAGE_OBSERVER(lambda st, p, w_, h_, c_, u: observer(st.decode(), p, w_, h_, c_)) if observer else \
            ctypes.cast(None, STAGE_OBSERVER)
        e = _err()
        rc = self.L.ernie_run_dit(self.dev, ctypes.cast(ids, c_vp), len(blocks), ptr(latent), height, width, ptr(text),
                                  text_tokens, ptr(features), dim, ptr(cos), ptr(sin), ptr(mask), valid_prefix, dtype,
                                  ptr(prediction), None if secs is None else secs.ctypes.data, cb, None, e, 512)
        if rc:
            _raise(rc, e.value)
        return None if secs is None else secs[:len(blocks)]

    def denoise_observed(self, blocks, latent, height, width, text, text_tokens, cos, sin, mask, valid_prefix, steps,
                         start_step=0, dtype=FP16, collect_details=False, observer=None):
        """Facade denoise with a step observer(step, prediction_ptr, sample_ptr, count)."""
        import numpy as np
        ids = (c_int * max(len(blocks), 1))(*blocks)
        n = max(steps, 1)
        secs = np.zeros(n, np.float64)
        ts = np.zeros(n, np.float32)
        cb = STEP_OBSERVER(lambda i, p, s_, cnt, u: observer(i, p, s_, cnt)) if observer else \
            ctypes.cast(None, STEP_OBSERVER)
        e = _err()
        rc = self.L.ernie_denoise_observed(self.dev, ctypes.cast(ids, c_vp), len(blocks), ptr(latent), height, width,
                                           ptr(text), text_tokens, ptr(cos), ptr(sin), ptr(mask), valid_prefix, steps,
                                           start_step, dtype, int(bool(collect_details)), secs.ctypes.data,
                                           ts.ctypes.data, cb, None, e, 512)
        if rc:
            _raise(rc, e.value)
        return secs[:max(steps - start_step, 0)], ts[:max(steps - start_step, 0)]

    def denoise(self, blocks, latent, height, width, text, text_tokens, cos, sin, mask, valid_prefix, steps,
                start_step=0, dtype=FP16):
        import numpy as np
        ids = (c_int * max(len(blocks), 1))(*blocks)
        n = max(steps, 1)
        secs = np.zeros(n, np.float64)
        ts = np.zeros(n, np.float32)
        e = _err()
        rc = self.L.ernie_denoise(self.dev, ctypes.cast(ids, c_vp), len(blocks), ptr(latent), height, width,
                                  ptr(text), text_tokens, ptr(cos), ptr(sin), ptr(mask), valid_prefix, steps,
                                  start_step, dtype, secs.ctypes.data, ts.ctypes.data, e, 512)
        if rc:
            _raise(rc, e.value)
        return secs[:max(steps - start_step, 0)], ts[:max(steps - start_step, 0)]
