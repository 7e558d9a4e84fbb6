"""On-disk block format without a device: SHA-256, the .param graph checks and
the ModelBin section walk (include/ernie.h, host/block_files.cpp).

Fixtures (tests/golden/make_block_fixtures.py): the reference's block-4 graphs
in both reviewed forms and the section table its manifest records for that
block's BF16 weight file.
"""
import hashlib
import json
import struct
from pathlib import Path

import numpy as np
import pytest

import ernie_amd as E

GOLDEN = Path(__file__).resolve().parent / "golden"
COMPONENT = GOLDEN / "block_component_s288.ncnn.param"
RUNTIME = GOLDEN / "block_runtime_s4160.ncnn.param"
SECTIONS = json.loads((GOLDEN / "block04_sections.json").read_text())
# src/shape_graph.cpp:27 (kind "dit"): reviewed hash of the runtime package graph.
RUNTIME_CONTRACT = "51db4065837c28e235784fd0dd196f109ca86822143c025a44ee9372240e4132"

TAGS = {E.FP32: 0, E.BF16: 0x01348B83, E.FP16: 0x01306B47}
FIELDS = ("norm1", "wq", "wk", "wv", "norm_q", "norm_k", "wo", "norm2", "w_up", "w_gate", "w_down")


# ---- writers used by the tests (the layout of tools/pack_block_weights.py:34-69) ----
def half_bits(a, dt):
    """Raw 16-bit patterns of FP32 values that are exact in dt (FP16 or BF16)."""
    a = np.ascontiguousarray(a, np.float32)
    if dt == E.FP16:
        h = a.astype(np.float16)
        assert np.array_equal(h.astype(np.float32), a), "value not exact in FP16"
        return h.view(np.uint16)
    bits = a.view(np.uint32)
    assert not np.any(bits & 0xFFFF), "value not exact in BF16"
    return (bits >> 16).astype(np.uint16)


def write_block_bin(path, weights, storage):
    """weights: dict of FP32 arrays keyed like FIELDS; storage: one dtype or a list of 7 (one per Gemm)."""
    gemm_dts = list(storage) if isinstance(storage, (list, tuple)) else [storage] * 7
    with open(path, "wb") as f:
        gi = 0
        for name in FIELDS:
            a = np.ascontiguousarray(weights[name], np.float32)
            if name.startswith("norm"):
                f.write(a.astype("<f4").tobytes())
                continue
            dt = gemm_dts[gi]
            gi += 1
            f.write(struct.pack("<I", TAGS[dt]))
            if dt == E.FP32:
                f.write(a.astype("<f4").tobytes())
            else:
                raw = half_bits(a, dt).astype("<u2").tobytes()
                f.write(raw + b"\0" * (-len(raw) % 4))


def synthetic_graph(dim, ffn, tokens=40):
    """The reviewed component graph with its widths replaced (an unreviewed topology)."""
    text = COMPONENT.read_text()
    out = []
    for line in text.splitlines():
        f = line.split()
        if len(f) > 1 and f[1].startswith(("gemm_", "rmsn_", "reshape_", "unsqueeze_")):
            rep = {"7=288": f"7={tokens}", "2=288": f"2={tokens}", "1=288": f"1={tokens}",
                   "8=4096": f"8={dim}", "9=4096": f"9={dim}", "8=12288": f"8={ffn}", "9=12288": f"9={ffn}",
                   "0=4096": f"0={dim}", "1=32": f"1={dim // 128}"}
            f = [rep.get(x, x) for x in f]
        out.append(" ".join(f))
    return "\n".join(out) + "\n"


def exact_weights(dim, ffn, seed):
    """Block weights that FP32, BF16 and FP16 all store exactly: k / 4096, |k| <= 127."""
    rng = np.random.default_rng(seed)
    shapes = {"norm1": (dim,), "wq": (dim, dim), "wk": (dim, dim), "wv": (dim, dim), "norm_q": (128,),
              "norm_k": (128,), "wo": (dim, dim), "norm2": (dim,), "w_up": (ffn, dim), "w_gate": (ffn, dim),
              "w_down": (dim, ffn)}
    w = {}
    for name, shape in shapes.items():
        k = rng.integers(-127, 128, size=shape).astype(np.float32) / 4096.0
        w[name] = (1.0 + k).astype(np.float32) if name.startswith("norm") else k
    return w


# ---- SHA-256 -----------------------------------------------------------------------
def test_sha256_fips_examples():
    # FIPS 180-2 appendix B examples.
    assert E.sha256_hex(b"abc") == "ba7816bf8f01cfea414140de5dae2223b00361a396177a9cb410ff61f20015ad"
    assert (E.sha256_hex(b"abcdbcdecdefdefgefghfghighijhijkijkljklmklmnlmnomnopnopq") ==
            "248d6a61d20638b8e5c026930c3e6039a33ce45964ff2167f6ecedd419db06c1")
    assert E.sha256_hex(b"a" * 1000000) == "cdc76e5c9914fb9281a1c7e284d73e67f1809a48a497200e046d39ccc7112cd0"
    assert E.sha256_hex(b"") == "e3b0c44298fc1c149afbf4c8996fb92427ae41e4649b934ca495991b7852b855"


def test_sha256_matches_hashlib_across_block_boundaries():
    rng = np.random.default_rng(0)
    for n in list(range(0, 130)) + [1000, 4096 + 7]:
        data = rng.integers(0, 256, n, dtype=np.uint8).tobytes()
        assert E.sha256_hex(data) == hashlib.sha256(data).hexdigest(), n


# ---- graph --------------------------------------------------------------------------
def test_reference_graphs_match_their_reviewed_contracts():
    c = E.block_file_inspect(COMPONENT)
    assert (c["contract"], c["tokens"], c["dim"], c["ffn"]) == ("component", 288, 4096, 12288)
    assert c["component_sha256"] == SECTIONS["graph_contract_sha256"]
    r = E.block_file_inspect(RUNTIME)
    assert (r["contract"], r["tokens"], r["dim"], r["ffn"]) == ("runtime", 4160, 4096, 12288)
    assert r["runtime_sha256"] == RUNTIME_CONTRACT
    # The two exports differ only in the residual-add layer type and the token count.
    assert r["component_sha256"] != c["component_sha256"]


def edited(text, old, new, count=1):
    assert old in text, old
    return text.replace(old, new, count)


@pytest.mark.parametrize("edit", [
    ("0=2\n", "0=0\n"),                       # a BinaryOp multiply becomes an add
    ("5=1\n", "5=0\n"),                       # SDPA mask flag
    ("-23300=2,64,-233", "-23300=2,32,-233"),  # RoPE halves
])
def test_changed_topology_is_unreviewed(tmp_path, edit):
    p = tmp_path / "block.ncnn.param"
    p.write_text(edited(COMPONENT.read_text(), *edit))
    with pytest.raises(E.ErnieInvalidRequest, match="reviewed"):
        E.block_file_inspect(p)
    assert E.block_file_inspect(p, allow_unreviewed=True)["contract"] == "unreviewed"


@pytest.mark.parametrize("edit, message", [
    (("7767517", "7767518"), "magic"),
    (("74 91", "75 91"), "layers"),
    (("74 91", "74 90"), "blobs"),
    (("rmsn_9 ", "rmsn_8 "), "duplicate layer"),
    (("1=1.000000e-6 2=1", "1=1.000000e-5 2=1"), "eps"),
    (("8=12288 9=4096", "8=12288 9=4095"), "shapes"),
    (("10=-1 2=0 3=1", "10=0 2=0 3=1"), "constant-B"),
    (("Gemm                     gemm_4", "Gemm                     gemm_9"), "expected gemm_4"),
    (("1 1 83 84", "1 1 99 84"), "before it is produced"),
    (("ErnieGELU gelu_7", "Swish gelu_7"), "type outside"),
])
def test_malformed_graphs_are_rejected_even_when_unreviewed_is_allowed(tmp_path, edit, message):
    p = tmp_path / "block.ncnn.param"
    p.write_text(edited(COMPONENT.read_text(), *edit))
    with pytest.raises(E.ErnieInvalidRequest, match=message):
        E.block_file_inspect(p, allow_unreviewed=True)


def test_graph_text_limits(tmp_path):
    p = tmp_path / "nul.param"
    p.write_bytes(COMPONENT.read_bytes().replace(b"74 91", b"74\x0091"))
    with pytest.raises(E.ErnieInvalidRequest, match="NUL"):
        E.block_file_inspect(p)
    p.write_bytes(b"")
    with pytest.raises(E.ErnieInvalidRequest, match="1..1048576"):
        E.block_file_inspect(p)
    with pytest.raises(E.ErnieError):
        E.block_file_inspect(tmp_path / "missing.param")


# ---- ModelBin -------------------------------------------------------------------------
def sparse_bin(path, sections, tag_for):
    """A weight file with zero payloads (sparse) and the Gemm tags at the given section starts."""
    with open(path, "wb") as f:
        for s in sections:
            if s["layer"].startswith("gemm"):
                f.seek(s["begin"])
                f.write(struct.pack("<I", tag_for(s)))
        f.truncate(sections[-1]["end"])


def test_section_walk_reproduces_the_reference_manifest(tmp_path):
    # The reference's BF16 block file of block 4 (the payload is zero here; only the layout matters).
    bin_path = tmp_path / "block.ncnn.bin"
    sparse_bin(bin_path, SECTIONS["sections"], lambda s: TAGS[E.BF16])
    info = E.block_file_inspect(COMPONENT, bin_path)
    assert info["bin_bytes"] == SECTIONS["sections"][-1]["end"]
    assert len(info["sections"]) == 11
    for got, ref in zip(info["sections"], SECTIONS["sections"]):
        assert got["layer"] == ref["layer"]
        assert (got["begin"], got["end"]) == (ref["begin"], ref["end"]), ref["layer"]
        want = E.FP32 if ref["storage"] == "fp32_affine" else E.BF16
        assert got["dtype"] == want
        assert got["data"] == got["begin"] + (0 if want == E.FP32 else 4)


def test_section_walk_errors(tmp_path):
    dim, ffn = 256, 512
    g = tmp_path / "block.ncnn.param"
    g.write_text(synthetic_graph(dim, ffn))
    w = exact_weights(dim, ffn, 1)
    b = tmp_path / "block.ncnn.bin"
    write_block_bin(b, w, [E.FP32, E.BF16, E.FP16, E.BF16, E.FP32, E.FP16, E.BF16])
    data = b.read_bytes()
    info = E.block_file_inspect(g, b, allow_unreviewed=True, expected_bin_sha256=hashlib.sha256(data).hexdigest())
    assert [s["dtype"] for s in info["sections"] if s["layer"].startswith("gemm")] == \
        [E.FP32, E.BF16, E.FP16, E.BF16, E.FP32, E.FP16, E.BF16]
    assert info["bin_bytes"] == len(data)
    with pytest.raises(E.ErnieInvalidRequest, match="checksum"):
        E.block_file_inspect(g, b, allow_unreviewed=True, expected_bin_sha256="0" * 64)
    b.write_bytes(data + b"\0\0\0\0")
    with pytest.raises(E.ErnieInvalidRequest, match="beyond"):
        E.block_file_inspect(g, b, allow_unreviewed=True)
    b.write_bytes(data[:-2])
    with pytest.raises(E.ErnieInvalidRequest, match="truncated"):
        E.block_file_inspect(g, b, allow_unreviewed=True)
    # An int8-quantized section (ncnn tag 0x000D4B38) is not a format of this block.
    first_gemm = info["sections"][1]["begin"]
    b.write_bytes(data[:first_gemm] + struct.pack("<I", 0x000D4B38) + data[first_gemm + 4:])
    with pytest.raises(E.ErnieInvalidRequest, match="tag 0x000d4b38"):
        E.block_file_inspect(g, b, allow_unreviewed=True)
    b.write_bytes(b"")
    with pytest.raises(E.ErnieInvalidRequest, match="empty"):
        E.block_file_inspect(g, b, allow_unreviewed=True)
