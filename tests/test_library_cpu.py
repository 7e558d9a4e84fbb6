"""CPU checks of the product libraries: they load, export every function the
public headers declare, and the facade's host-side helpers agree with the
oracle bit for bit. No device computation happens here."""
import ctypes
from pathlib import Path

import numpy as np
import pytest

import ernie_amd as E
import oracle as O

GOLDEN = Path(__file__).with_name("golden")


def test_libraries_load_and_export_every_declared_symbol():
    names = E.declared_functions()
    assert len(names) > 40
    hip_lib = ctypes.CDLL(str(E.HIP_LIB))
    facade_lib = ctypes.CDLL(str(E.FACADE_LIB))
    missing = [n for n in names if not hasattr(hip_lib, n) and not hasattr(facade_lib, n)]
    assert not missing, missing


def test_binding_signatures_cover_the_headers():
    E.hip()
    E.facade()
    for n in E.declared_functions():
        lib = E.hip() if n.startswith("ernie_hip_") else E.facade()
        assert getattr(lib, n).argtypes is not None, n


def test_facade_schedule_matches_oracle_bitwise():
    for steps in (1, 2, 3, 8, 9, 50, 1000):
        s1, t1 = E.flow_schedule_turbo(steps)
        s2, t2 = O.flow_schedule_turbo(steps)
        np.testing.assert_array_equal(s1, s2)
        np.testing.assert_array_equal(t1, t2)
    for bad in (0, 1001, -3):
        with pytest.raises(E.ErnieInvalidRequest):
            E.flow_schedule_turbo(bad)


def test_facade_timestep_features_match_oracle_bitwise():
    for t in (0.0, 1.0, 363.63638, 500.0, 999.99, 1000.0):
        np.testing.assert_array_equal(E.timestep_features(t), O.timestep_features(t))
    for bad in (-0.5, 1000.01, float("inf"), float("nan")):
        with pytest.raises(E.ErnieInvalidRequest):
            E.timestep_features(bad)


def test_facade_rope_table_and_constants_match_oracle():
    np.testing.assert_array_equal(E.rope_frequencies(), O.rope_frequencies())
    freqs = np.fromfile(GOLDEN / "rope_inv_freq.f32", dtype="<f4")
    for (w, h, valid, text) in ((64, 64, 40, 64), (32, 32, 32, 32), (86, 48, 1080, 2048), (3, 5, 1, 1)):
        c1, s1, m1, vk = E.dit_constants(freqs, w, h, valid, text)
        c2, s2, m2 = O.dit_constants(freqs, w, h, valid, text)
        np.testing.assert_array_equal(c1, c2)
        np.testing.assert_array_equal(s1, s2)
        np.testing.assert_array_equal(m1, m2)
        assert vk == w * h + valid
    with pytest.raises(E.ErnieInvalidRequest):
        E.dit_constants(freqs, 128, 128, 10, 2048)  # 18432 tokens > 10240
    with pytest.raises(E.ErnieInvalidRequest):
        E.dit_constants(freqs, 4, 4, 0, 8)


def test_context_creation_fails_loudly_without_device():
    import torch
    if torch.cuda.is_available():
        pytest.skip("a device is present")
    with pytest.raises(E.ErnieError):
        E.Context(0, use_torch_stream=False)


def test_dit_constants_from_the_frequency_file(tmp_path):
    # src/conditioning.cpp:10-23: the 256-byte file is size-checked and read; the
    # path overload's token limit is 6144 (src/conditioning.cpp:46-49).
    path = GOLDEN / "rope_inv_freq.f32"
    freqs = np.fromfile(path, dtype="<f4")
    for (w, h, valid, text) in ((64, 64, 40, 64), (3, 5, 1, 1), (48, 86, 1000, 1088)):
        c1, s1, m1, vk = E.dit_constants_file(path, w, h, valid, text)
        c2, s2, m2, vk2 = E.dit_constants(freqs, w, h, valid, text)
        np.testing.assert_array_equal(c1, c2)
        np.testing.assert_array_equal(s1, s2)
        np.testing.assert_array_equal(m1, m2)
        assert vk == vk2 == w * h + valid
    with pytest.raises(E.ErnieInvalidRequest):
        E.dit_constants_file(path, 48, 86, 1080, 2048)  # 6176 tokens > 6144 for this overload
    short = tmp_path / "short.f32"
    short.write_bytes(path.read_bytes()[:252])
    with pytest.raises(E.ErnieInvalidRequest, match="frequency file"):
        E.dit_constants_file(short, 8, 8, 4, 8)
    with pytest.raises(E.ErnieInvalidRequest, match="frequency file"):
        E.dit_constants_file(tmp_path / "missing.f32", 8, 8, 4, 8)
    bad = tmp_path / "bad.f32"
    neg = freqs.copy()
    neg[17] = -1.0
    neg.astype("<f4").tofile(bad)
    with pytest.raises(E.ErnieError, match="Invalid DiT frequency"):
        E.dit_constants_file(bad, 8, 8, 4, 8)
    neg[17] = np.nan
    neg.astype("<f4").tofile(bad)
    with pytest.raises(E.ErnieError, match="Invalid DiT frequency"):
        E.dit_constants_file(bad, 8, 8, 4, 8)


def test_pad_text_zero_pads_to_the_bucket():
    # src/conditioning.cpp:56-67: rows copied, the rest of the bucket zero.
    emb = O.normal((40, 3072), 9)
    out = E.pad_text(emb, 64)
    assert out.shape == (64, 3072)
    np.testing.assert_array_equal(out[:40], emb)
    assert not out[40:].any()
    np.testing.assert_array_equal(E.pad_text(emb, 40), emb)
    for bucket in (39, 2049):
        with pytest.raises(E.ErnieInvalidRequest, match="padding bucket"):
            E.pad_text(emb, bucket)
