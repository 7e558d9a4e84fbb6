"""CPU checks of the Mistral text path: the oracle's text block against a PyTorch
FP64 restatement of tools/export_text_block.py:56-67, its SiLU and text constants
against closed forms, the causal GQA probe's FP64 oracle against the oracle's
attention, and the facade's host helpers (text_constants, text_embeddings)
against the oracle and numpy bit for bit. No device computation."""
import math

import numpy as np
import pytest

import ernie_amd as E
import kat
import oracle as O

HIDDEN, HEADS, KV_HEADS, FFN = 256, 4, 2, 512


def small_text_block(seed=30, hidden=HIDDEN, heads=HEADS, kv_heads=KV_HEADS, ffn=FFN, std=0.05):
    shapes = {"norm1": (hidden,), "wq": (heads * 128, hidden), "wk": (kv_heads * 128, hidden),
              "wv": (kv_heads * 128, hidden), "wo": (hidden, heads * 128), "norm2": (hidden,),
              "w_gate": (ffn, hidden), "w_up": (ffn, hidden), "w_down": (hidden, ffn)}
    return {n: O.normal(shapes[n], seed, offset=i << 40, mean=1.0 if n.startswith("norm") else 0.0, std=std)
            for i, n in enumerate(O.TEXT_FIELDS)}


def yarn_like_frequencies():
    """64 positive inverse frequencies in the shape of the converter's table."""
    return (1.0 / (1e6 ** (np.arange(0, 128, 2) / 128.0))).astype(np.float32)


def torch_text_block_fp64(w, x, cos, sin, mask, heads, kv_heads):
    """tools/export_text_block.py:56-67 (TextBlock.forward) with torch.nn.functional in FP64."""
    import torch
    F = torch.nn.functional
    T = {k: torch.from_numpy(np.asarray(v)).double() for k, v in w.items()}
    x = torch.from_numpy(x).double()
    hidden = x.shape[1]
    c, s = torch.from_numpy(cos).double()[None], torch.from_numpy(sin).double()[None]

    def rotary(t):  # export_dit_block.ExportBlock.rotary: halves of 64
        a, b = t[..., :64], t[..., 64:]
        return torch.cat((a * c[..., :64] - b * s[..., :64], b * c[..., 64:] + a * s[..., 64:]), dim=-1)

    norm = F.rms_norm(x, (hidden,), T["norm1"], 1e-5)
    q = F.linear(norm, T["wq"]).reshape(-1, heads, 128).transpose(0, 1)
    k = F.linear(norm, T["wk"]).reshape(-1, kv_heads, 128).transpose(0, 1)
    v = F.linear(norm, T["wv"]).reshape(-1, kv_heads, 128).transpose(0, 1)
    q, k = rotary(q), rotary(k)
    m = torch.from_numpy(mask).double()
    a = F.scaled_dot_product_attention(q[None], k[None], v[None], m, enable_gqa=True)[0]
    x = x + F.linear(a.transpose(0, 1).reshape(-1, heads * 128), T["wo"])
    h2 = F.rms_norm(x, (hidden,), T["norm2"], 1e-5)
    return (x + F.linear(F.silu(F.linear(h2, T["w_gate"])) * F.linear(h2, T["w_up"]), T["w_down"])).numpy()


def test_silu_matches_fp64_closed_form():
    x = np.linspace(-30, 30, 4001, dtype=np.float32)
    ref = x.astype(np.float64) / (1.0 + np.exp(-x.astype(np.float64)))
    assert np.max(np.abs(O.silu(x) - ref)) <= 4e-6
    np.testing.assert_array_equal(O.silu(np.zeros(3, np.float32)), np.zeros(3, np.float32))


def test_text_constants_closed_form_and_mask_structure():
    f = yarn_like_frequencies()
    cos, sin, mask = O.text_constants(f, 37)
    t = np.arange(37)[:, None].astype(np.float64)
    phase = (np.arange(37)[:, None].astype(np.float32) * f[None, :]).astype(np.float64)
    np.testing.assert_allclose(cos[:, :64], np.cos(phase), atol=2e-7)
    np.testing.assert_allclose(sin[:, :64], np.sin(phase), atol=2e-7)
    np.testing.assert_array_equal(cos[:, 64:], cos[:, :64])  # c[j] = c[j + 64]
    np.testing.assert_array_equal(sin[:, 64:], sin[:, :64])
    np.testing.assert_array_equal(cos[0], np.ones(128, np.float32))  # position 0: angle 0
    expected = np.where(np.arange(37)[None, :] > t, -np.finfo(np.float32).max, 0.0).astype(np.float32)
    np.testing.assert_array_equal(mask, expected)
    for bad in (0, 2049):
        with pytest.raises(ValueError):
            O.text_constants(f, bad)
    with pytest.raises(ValueError):
        O.text_constants(np.r_[f[:-1], -1.0].astype(np.float32), 8)


def test_text_block_oracle_matches_torch_fp64():
    w = small_text_block()
    S = 24
    cos, sin, mask = O.text_constants(yarn_like_frequencies(), S)
    x = O.normal((S, HIDDEN), 31, std=0.2)
    out = O.text_block_forward(w, x, cos, sin, mask, HEADS, KV_HEADS)
    ref = torch_text_block_fp64(w, x, cos, sin, mask, HEADS, KV_HEADS)
    m = kat.fp32_block_rule(out, ref)
    assert m["passed"] and m["nrmse"] < 2e-6, m


def test_text_block_causality_and_zero_branches():
    """Causal mask: token t never depends on later tokens. Zero o_proj and down_proj
    make the block the identity (both residual branches vanish)."""
    w = small_text_block()
    S = 16
    cos, sin, mask = O.text_constants(yarn_like_frequencies(), S)
    x = O.normal((S, HIDDEN), 32, std=0.2)
    out = O.text_block_forward(w, x, cos, sin, mask, HEADS, KV_HEADS)
    x2 = x.copy()
    x2[10:] = O.normal((S - 10, HIDDEN), 33, std=0.2)
    out2 = O.text_block_forward(w, x2, cos, sin, mask, HEADS, KV_HEADS)
    np.testing.assert_array_equal(out[:10], out2[:10])
    z = dict(w, wo=np.zeros_like(w["wo"]), w_down=np.zeros_like(w["w_down"]))
    np.testing.assert_array_equal(O.text_block_forward(z, x, cos, sin, mask, HEADS, KV_HEADS), x)


def test_gqa_probe_oracle_matches_oracle_attention():
    """probes/attention_probe.cpp's visible-key FP64 oracle against the oracle's SDPA
    with the dense causal mask (precise accumulation)."""
    for length, seed in ((32, 11), (17, 83)):
        q, k, v, mask = kat.gqa_causal_case(length, seed)
        ref = kat.gqa_causal_expected(q, k, v)
        got = O.sdpa(q, k, v, mask=mask)
        assert np.max(np.abs(got - ref)) <= 2e-6


def test_facade_text_constants_match_oracle_bitwise():
    f = yarn_like_frequencies()
    for bucket in (1, 32, 64, 300):
        for a, b in zip(E.text_constants(f, bucket), O.text_constants(f, bucket)):
            np.testing.assert_array_equal(a, b)
    for bad in (0, 2049):
        with pytest.raises(E.ErnieInvalidRequest):
            E.text_constants(f, bad)


def test_facade_text_embeddings_widen_bf16_rows():
    rng = np.random.default_rng(5)
    vocab, width = 97, 48
    table = rng.integers(0, 65536, size=(vocab, width), dtype=np.uint16)
    table[(table & 0x7F80) == 0x7F80] = 0  # no Inf/NaN patterns
    ids = np.array([3, 96, 0, 3], np.uint32)
    out = E.text_embeddings(table, ids, 8)
    expected = np.zeros((8, width), np.float32)
    expected[:4] = (table[ids].astype(np.uint32) << 16).view(np.float32)
    np.testing.assert_array_equal(out, expected)
    with pytest.raises(E.ErnieInvalidRequest):
        E.text_embeddings(table, np.array([97], np.uint32), 8)  # outside the vocabulary
    with pytest.raises(E.ErnieInvalidRequest):
        E.text_embeddings(table, np.arange(9, dtype=np.uint32), 8)  # more ids than the bucket
    with pytest.raises(E.ErnieInvalidRequest):
        E.text_embeddings(table, np.array([], np.uint32), 8)
