"""DiT head and text block files (heads/{input,output}/head.ncnn.{param,bin},
text.ncnn.{param,bin}) read without ncnn, on the CPU.

The graphs are the reference's own (tests/golden, written by make_block_fixtures.py);
their SHA-256 is the one each reference directory's model.json records, and their
normalised forms must hash to the reviewed runtime contracts of src/shape_graph.cpp:31.
Weight files are written here in the ModelBin layout: tagged weights (FP32 0, BF16
0x01348B83, FP16 0x01306B47), raw FP32 biases and RMSNorm gammas. The text block's
section order, shapes and storage are checked against the table the reference
recorded for text block 4.
"""
import json
import struct
from pathlib import Path

import numpy as np
import pytest

import ernie_amd as E
from test_block_files import TAGS, half_bits

GOLDEN = Path(__file__).with_name("golden")
HEAD_HASHES = json.loads((GOLDEN / "heads.json").read_text())
TEXT_SECTIONS = json.loads((GOLDEN / "text_block04_sections.json").read_text())
# src/shape_graph.cpp:31: reviewed hashes of the normalised "input", "output" and "text" graphs.
CONTRACT = {"input": "3710a502802138e8605ca54a9132fb9a9a1888841586c1d7067f7043769bbecb",
            "output": "98bf1afc154dd05cf419aafad4aa383af311e44658e644d0c322ffb50431533c",
            "text": "dda8db13b6e20a00c1133485c3be2ef37db56b1db058e42a405b51d24fc64b0e"}
TEXT_S64 = GOLDEN / "text_s64.ncnn.param"


# ---- graph and weight writers shared with the GPU tests -----------------------------------
def _rewrite(template, per_layer):
    out = []
    for line in template.read_text().splitlines():
        f = line.split()
        if len(f) > 1 and f[1] in per_layer:
            f = [per_layer[f[1]].get(x, x) for x in f]
        out.append(" ".join(f))
    return "\n".join(out) + "\n"


def head_graph(kind, dim, latent, text_dim, width, height, text_tokens):
    """The reference's component head graph (4x4 grid, 272 text slots) with other widths."""
    hw = width * height
    if kind == "input":
        return _rewrite(GOLDEN / "head_input_s288.ncnn.param", {
            "conv_1": {"0=4096": f"0={dim}", "6=524288": f"6={dim * latent}"},
            "reshape_7": {"0=16": f"0={hw}", "1=4096": f"1={dim}"},
            "gemm_0": {"7=272": f"7={text_tokens}", "8=4096": f"8={dim}", "9=3072": f"9={text_dim}"},
            "linear_2": {"0=4096": f"0={dim}", "2=16777216": f"2={dim * dim}"},
            "linear_3": {"0=4096": f"0={dim}", "2=16777216": f"2={dim * dim}"},
            "linear_4": {"0=24576": f"0={6 * dim}", "2=100663296": f"2={6 * dim * dim}"},
            "reshape_8": {"0=4096": f"0={dim}"}})
    return _rewrite(GOLDEN / "head_output_s288.ncnn.param", {
        "linear_2": {"0=8192": f"0={2 * dim}", "2=33554432": f"2={2 * dim * dim}"},
        "ln_1": {"0=4096": f"0={dim}"},
        "reshape_3": {"0=4096": f"0={dim}"}, "reshape_4": {"0=4096": f"0={dim}"},
        "gemm_0": {"7=288": f"7={hw + text_tokens}", "8=128": f"8={latent}", "9=4096": f"9={dim}"},
        "slice_0": {"-23310=1,16": f"-23310=1,{hw}"},
        "reshape_5": {"0=4": f"0={width}", "1=4": f"1={height}", "2=128": f"2={latent}"}})


def text_graph(hidden, heads, kv_heads, ffn, tokens):
    """The reference's 64-token text block graph with other widths and token count."""
    q, kv = heads * 128, kv_heads * 128
    t = str(tokens)
    return _rewrite(TEXT_S64, {
        "rmsn_8": {"0=3072": f"0={hidden}"}, "rmsn_9": {"0=3072": f"0={hidden}"},
        "gemm_0": {"7=64": f"7={t}", "8=4096": f"8={q}", "9=3072": f"9={hidden}"},
        "gemm_1": {"7=64": f"7={t}", "8=1024": f"8={kv}", "9=3072": f"9={hidden}"},
        "gemm_2": {"7=64": f"7={t}", "8=1024": f"8={kv}", "9=3072": f"9={hidden}"},
        "gemm_3": {"7=64": f"7={t}", "8=3072": f"8={hidden}", "9=4096": f"9={q}"},
        "gemm_4": {"7=64": f"7={t}", "8=9216": f"8={ffn}", "9=3072": f"9={hidden}"},
        "gemm_5": {"7=64": f"7={t}", "8=9216": f"8={ffn}", "9=3072": f"9={hidden}"},
        "gemm_6": {"7=64": f"7={t}", "8=3072": f"8={hidden}", "9=9216": f"9={ffn}"},
        "reshape_10": {"1=32": f"1={heads}", "2=64": f"2={t}"},
        "reshape_11": {"1=8": f"1={kv_heads}", "2=64": f"2={t}"},
        "reshape_12": {"1=8": f"1={kv_heads}", "2=64": f"2={t}"},
        "reshape_13": {"0=4096": f"0={q}", "1=64": f"1={t}"},
        "unsqueeze_18": {"1=64": f"1={t}"}, "unsqueeze_19": {"1=64": f"1={t}"}})


HEAD_LAYOUT = {  # (field, tagged) in .bin order
    "input": (("x_w", True), ("x_b", False), ("text_w", True), ("t1_w", True), ("t1_b", False), ("t2_w", True),
              ("t2_b", False), ("mod_w", True), ("mod_b", False)),
    "output": (("out_mod_w", True), ("out_mod_b", False), ("proj_w", True), ("proj_b", False)),
}
TEXT_FIELDS = ("norm1", "wq", "wk", "wv", "wo", "norm2", "w_gate", "w_up", "w_down")


def _write_section(f, a, tagged, dt):
    a = np.ascontiguousarray(a, np.float32)
    if not tagged:
        f.write(a.astype("<f4").tobytes())
        return
    f.write(struct.pack("<I", TAGS[dt]))
    if dt == E.FP32:
        f.write(a.astype("<f4").tobytes())
    else:
        raw = half_bits(a, dt).astype("<u2").tobytes()
        f.write(raw + b"\0" * (-len(raw) % 4))


def write_head_bin(path, kind, weights, storage):
    with open(path, "wb") as f:
        for field, tagged in HEAD_LAYOUT[kind]:
            _write_section(f, weights[field], tagged, storage)


def write_text_bin(path, weights, storage):
    with open(path, "wb") as f:
        for field in TEXT_FIELDS:
            _write_section(f, weights[field], not field.startswith("norm"), storage)


def exact_head_weights(dim, latent, text_dim, seed):
    """Head weights exact in FP32, BF16 and FP16 (k / 4096, |k| <= 127; biases k / 64)."""
    rng = np.random.default_rng(seed)
    shapes = {"x_w": (dim, latent), "x_b": (dim,), "text_w": (dim, text_dim), "t1_w": (dim, dim), "t1_b": (dim,),
              "t2_w": (dim, dim), "t2_b": (dim,), "mod_w": (6 * dim, dim), "mod_b": (6 * dim,),
              "out_mod_w": (2 * dim, dim), "out_mod_b": (2 * dim,), "proj_w": (latent, dim), "proj_b": (latent,)}
    draw = lambda s: rng.integers(-127, 128, size=s, dtype=np.int8).astype(np.float32)
    return {n: draw(s) / (64.0 if len(s) == 1 else 4096.0) for n, s in shapes.items()}


def exact_text_weights(hidden, heads, kv_heads, ffn, seed):
    rng = np.random.default_rng(seed)
    q, kv = heads * 128, kv_heads * 128
    shapes = {"norm1": (hidden,), "wq": (q, hidden), "wk": (kv, hidden), "wv": (kv, hidden), "wo": (hidden, q),
              "norm2": (hidden,), "w_gate": (ffn, hidden), "w_up": (ffn, hidden), "w_down": (hidden, ffn)}
    w = {}
    for n, s in shapes.items():
        k = rng.integers(-127, 128, size=s).astype(np.float32) / 4096.0
        w[n] = (1.0 + k).astype(np.float32) if n.startswith("norm") else k
    return w


def _sparse(path, size, tags=()):
    """A zero-filled (sparse) file of `size` bytes with 4-byte tags written at offsets."""
    with open(path, "wb") as f:
        f.truncate(size)
        for off, tag in tags:
            f.seek(off)
            f.write(struct.pack("<I", tag))


# ---- the reference's graphs ------------------------------------------------------------
@pytest.mark.parametrize("name", sorted(HEAD_HASHES))
def test_head_fixtures_are_the_recorded_graphs(name):
    assert E.sha256_hex((GOLDEN / name).read_bytes()) == HEAD_HASHES[name]


@pytest.mark.parametrize("name,expect", [
    ("head_input_s288.ncnn.param", dict(part=1, dim=4096, latent_ch=128, text_dim=3072, text_tokens=272,
                                        image_tokens=16, tokens=288, width=0, height=0)),
    ("head_input_s4160.ncnn.param", dict(part=1, dim=4096, latent_ch=128, text_dim=3072, text_tokens=64,
                                         image_tokens=4096, tokens=4160, width=0, height=0)),
    ("head_output_s288.ncnn.param", dict(part=2, dim=4096, latent_ch=128, text_dim=0, text_tokens=272,
                                         image_tokens=16, tokens=288, width=4, height=4)),
    ("head_output_s4160.ncnn.param", dict(part=2, dim=4096, latent_ch=128, text_dim=0, text_tokens=64,
                                          image_tokens=4096, tokens=4160, width=64, height=64)),
])
def test_reference_head_graphs_meet_the_runtime_contract(name, expect):
    info = E.head_file_inspect(GOLDEN / name)
    assert {k: info[k] for k in expect} == expect
    assert info["reviewed"] and info["contract_sha256"] == CONTRACT["input" if expect["part"] == 1 else "output"]
    assert info["sections"] == [] and info["bin_bytes"] == 0


@pytest.mark.parametrize("kind,shape", [("input", (4096, 128, 3072, 4, 4, 272)), ("input", (4096, 128, 3072, 64, 64, 64)),
                                        ("output", (4096, 128, 3072, 4, 4, 272)),
                                        ("output", (4096, 128, 3072, 64, 64, 64))])
def test_head_graph_writer_reproduces_the_reference_graphs(kind, shape):
    # The test writer, given the reference's shapes, yields the reference's graphs (up to
    # column alignment), so graphs it writes at other widths differ from them only there.
    tag = "s288" if shape[3] == 4 else "s4160"
    ref = (GOLDEN / f"head_{kind}_{tag}.ncnn.param").read_text()
    norm = lambda t: [" ".join(l.split()) for l in t.splitlines()]
    assert norm(head_graph(kind, *shape)) == norm(ref)


def test_text_graph_writer_reproduces_the_reference_graph():
    norm = lambda t: [" ".join(l.split()) for l in t.splitlines()]
    assert norm(text_graph(3072, 32, 8, 9216, 64)) == norm(TEXT_S64.read_text())


def _input_head_size(dim, latent, text_dim, half=False):
    e = 2 if half else 4
    tagged = lambda n: 4 + (n * e + 3) // 4 * 4
    return (tagged(dim * latent) + 4 * dim + tagged(dim * text_dim) + 2 * (tagged(dim * dim) + 4 * dim) +
            tagged(6 * dim * dim) + 4 * 6 * dim)


def test_full_size_input_head_sections(tmp_path):
    # The reference's input head at full width: an FP32 file (as pnnx writes it, fp16=0)
    # is all tags 0 and raw floats, so a zero-filled file of the exact size is well formed.
    dim, latent, text_dim = 4096, 128, 3072
    size = _input_head_size(dim, latent, text_dim)
    b = tmp_path / "head.ncnn.bin"
    _sparse(b, size)
    info = E.head_file_inspect(GOLDEN / "head_input_s4160.ncnn.param", b)
    counts = [dim * latent, dim, dim * text_dim, dim * dim, dim, dim * dim, dim, 6 * dim * dim, 6 * dim]
    assert [s["layer"] for s in info["sections"]] == list(E.HEAD_SECTIONS[E.HEAD_INPUT])
    assert all(s["dtype"] == E.FP32 for s in info["sections"])
    off = 0
    for s, n, (_, tagged) in zip(info["sections"], counts, HEAD_LAYOUT["input"]):
        assert s["begin"] == off and s["data"] == off + (4 if tagged else 0) and s["end"] == s["data"] + 4 * n
        off = s["end"]
    assert off == size == info["bin_bytes"]
    for bad_size in (size - 4, size + 4):
        _sparse(b, bad_size)
        with pytest.raises(E.ErnieInvalidRequest):
            E.head_file_inspect(GOLDEN / "head_input_s4160.ncnn.param", b)


def test_full_size_output_head_bf16_sections(tmp_path):
    dim, latent = 4096, 128
    # linear_2 [8192][4096] BF16 + bias 8192, gemm_0 [128][4096] BF16 + bias 128.
    s0 = 4 + 2 * 2 * dim * dim
    s1 = s0 + 4 * 2 * dim
    s2 = s1 + 4 + 2 * latent * dim
    size = s2 + 4 * latent
    b = tmp_path / "head.ncnn.bin"
    _sparse(b, size, [(0, TAGS[E.BF16]), (s1, TAGS[E.BF16])])
    info = E.head_file_inspect(GOLDEN / "head_output_s288.ncnn.param", b)
    assert [(s["layer"], s["dtype"], s["end"]) for s in info["sections"]] == [
        ("linear_2", E.BF16, s0), ("linear_2.bias", E.FP32, s1), ("gemm_0", E.BF16, s2), ("gemm_0.bias", E.FP32, size)]
    # An unknown tag (a quantized section) is refused.
    _sparse(b, size, [(0, 0x000D4B38), (s1, TAGS[E.BF16])])
    with pytest.raises(E.ErnieInvalidRequest, match="tag"):
        E.head_file_inspect(GOLDEN / "head_output_s288.ncnn.param", b)


def test_head_checksum_and_unreviewed_widths(tmp_path):
    dim, latent, text_dim = 256, 32, 64
    w = exact_head_weights(dim, latent, text_dim, seed=1)
    g = tmp_path / "head.ncnn.param"
    g.write_text(head_graph("input", dim, latent, text_dim, 4, 2, 8))
    b = tmp_path / "head.ncnn.bin"
    write_head_bin(b, "input", w, E.FP16)
    with pytest.raises(E.ErnieInvalidRequest, match="reviewed"):
        E.head_file_inspect(g, b)
    info = E.head_file_inspect(g, b, allow_unreviewed=True, expected_bin_sha256=E.sha256_hex(b.read_bytes()).upper())
    assert (info["part"], info["dim"], info["latent_ch"], info["text_dim"], info["image_tokens"],
            info["text_tokens"], info["reviewed"]) == (1, dim, latent, text_dim, 8, 8, False)
    assert info["bin_bytes"] == _input_head_size(dim, latent, text_dim, half=True)
    with pytest.raises(E.ErnieInvalidRequest, match="checksum"):
        E.head_file_inspect(g, b, allow_unreviewed=True, expected_bin_sha256="0" * 64)
    # Shape inconsistencies are refused even when unreviewed topologies are allowed.
    bad = head_graph("input", dim, latent, text_dim, 4, 2, 8).replace(f"2={6 * dim * dim}", f"2={6 * dim * dim + 1}")
    g.write_text(bad)
    with pytest.raises(E.ErnieInvalidRequest):
        E.head_file_inspect(g, allow_unreviewed=True)
    out = head_graph("output", dim, latent, text_dim, 4, 2, 8).replace("-23310=1,8", "-23310=1,9")
    g.write_text(out)
    with pytest.raises(E.ErnieInvalidRequest):
        E.head_file_inspect(g, allow_unreviewed=True)


# ---- text blocks -------------------------------------------------------------------------
@pytest.mark.parametrize("name", ["text_s64.ncnn.param"])
def test_reference_text_graph_meets_the_runtime_contract(name):
    info = E.text_block_file_inspect(GOLDEN / name)
    assert (info["tokens"], info["hidden"], info["heads"], info["kv_heads"], info["ffn"]) == (64, 3072, 32, 8, 9216)
    assert info["reviewed"] and info["contract_sha256"] == CONTRACT["text"]


def test_text_sections_match_the_recorded_table(tmp_path):
    # The BF16 file tools/build_text_weights.py writes: raw FP32 gammas, tagged BF16 Gemms,
    # in the order, shapes and storage recorded for text block 4.
    tags, off = [], 0
    expect = []
    for sec in TEXT_SECTIONS["sections"]:
        n = int(np.prod(sec["shape"]))
        if sec["storage"] == "fp32":
            expect.append((sec["layer"], E.FP32, off, off, off + 4 * n))
            off += 4 * n
        else:
            assert sec["storage"] == "bf16"
            tags.append((off, TAGS[E.BF16]))
            end = off + 4 + (2 * n + 3) // 4 * 4
            expect.append((sec["layer"], E.BF16, off, off + 4, end))
            off = end
    b = tmp_path / "text.ncnn.bin"
    _sparse(b, off, tags)
    info = E.text_block_file_inspect(TEXT_S64, b)
    assert [(s["layer"], s["dtype"], s["begin"], s["data"], s["end"]) for s in info["sections"]] == expect
    assert info["bin_bytes"] == off
    _sparse(b, off + 2, tags)
    with pytest.raises(E.ErnieInvalidRequest, match="beyond"):
        E.text_block_file_inspect(TEXT_S64, b)


def test_text_graph_checks(tmp_path):
    g = tmp_path / "text.ncnn.param"
    g.write_text(text_graph(512, 4, 2, 1024, 16))
    with pytest.raises(E.ErnieInvalidRequest, match="reviewed"):
        E.text_block_file_inspect(g)
    info = E.text_block_file_inspect(g, allow_unreviewed=True)
    assert (info["tokens"], info["hidden"], info["heads"], info["kv_heads"], info["ffn"]) == (16, 512, 4, 2, 1024)
    # The 64-token graph at 32 tokens in one Gemm only: token counts disagree.
    g.write_text(TEXT_S64.read_text().replace("7=64 8=1024 9=3072", "7=32 8=1024 9=3072", 1))
    with pytest.raises(E.ErnieInvalidRequest, match="token"):
        E.text_block_file_inspect(g, allow_unreviewed=True)
    # An RMSNorm with the DiT's eps is not the text block's.
    g.write_text(TEXT_S64.read_text().replace("1=1.000000e-5", "1=1.000000e-6", 1))
    with pytest.raises(E.ErnieInvalidRequest, match="eps"):
        E.text_block_file_inspect(g, allow_unreviewed=True)
    # A DiT block graph is not a text block.
    with pytest.raises(E.ErnieInvalidRequest):
        E.text_block_file_inspect(GOLDEN / "block_component_s288.ncnn.param", allow_unreviewed=True)
