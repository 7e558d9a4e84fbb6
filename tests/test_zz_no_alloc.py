"""The text block entry point that allocates nothing (its workspace is the library's
fixed device scratch) against the allocating entry point it varies: bitwise equal
outputs on two calls in a row, the second with fewer tokens, and no device memory
taken by either call."""
import numpy as np
import pytest

import ernie_amd as E
import oracle as O
from gpu_util import NAMES, dev, empty, host
from test_text_cpu import small_text_block, yarn_like_frequencies

pytestmark = pytest.mark.gpu

HIDDEN, HEADS, KV_HEADS, FFN = 3072, 32, 8, 9216  # the reference's Mistral text block


def text_inputs(S, seed):
    cos, sin, mask = O.text_constants(yarn_like_frequencies(), S)
    return O.normal((S, HIDDEN), seed, std=0.2), cos, sin, mask


def forward(c, name, index, x, out, cos, sin, mask, causal, S):
    c.call(name, index, E.ptr(x), E.ptr(out), E.ptr(cos), E.ptr(sin), E.ptr(mask), 1 if causal else 0, S)
    return host(out)


@pytest.mark.parametrize("dt", [E.FP16, E.BF16, E.FP32], ids=lambda d: NAMES[d])
def test_no_alloc_text_block_matches_the_allocating_entry(dt):
    import torch
    c = E.Context(0)
    try:
        w = small_text_block(seed=61, hidden=HIDDEN, heads=HEADS, kv_heads=KV_HEADS, ffn=FFN, std=0.02)
        c.text_block_upload(0, w, HIDDEN, HEADS, KV_HEADS, FFN, dt)
        # Two calls in a row, the second with fewer tokens (and the dense mask instead of
        # the causal rule); every device buffer exists before the calls.
        cases = []
        for S, causal in ((64, True), (33, False)):
            x, cos, sin, mask = text_inputs(S, seed=62 + S)
            cases.append((S, causal, dev(x), dev(cos), dev(sin), None if causal else dev(mask), empty((S, HIDDEN))))
        # The first launch of each kernel loads its code object into device memory (the
        # runtime's lazy loading, not an allocation of the library): one untimed call
        # first, then the two calls whose device memory use is measured.
        S, causal, xd, cd, sd, md, out = cases[0]
        c.call("text_block_forward_noalloc", 0, E.ptr(xd), E.ptr(out), E.ptr(cd), E.ptr(sd), E.ptr(md), 1, S)
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info()[0]
        results = {}
        for S, causal, xd, cd, sd, md, out in cases:
            c.call("text_block_forward_noalloc", 0, E.ptr(xd), E.ptr(out), E.ptr(cd), E.ptr(sd), E.ptr(md),
                   1 if causal else 0, S)
        torch.cuda.synchronize()
        taken = free_before - torch.cuda.mem_get_info()[0]
        assert taken < (1 << 20), f"the no-allocation calls took {taken} bytes of device memory"
        for S, causal, xd, cd, sd, md, out in cases:
            results[S] = host(out)
        # The allocating entry point on the same inputs, after the no-allocation calls.
        for S, causal, xd, cd, sd, md, _ in cases:
            ref = forward(c, "text_block_forward", 0, xd, empty((S, HIDDEN)), cd, sd, md, causal, S)
            assert np.isfinite(ref).all()
            np.testing.assert_array_equal(results[S], ref)
        # Beyond the fixed scratch's token limit the call is refused before any work.
        S = 65
        x, cos, sin, _ = text_inputs(S, seed=7)
        with pytest.raises(E.ErnieError, match="at most 64 tokens"):
            forward(c, "text_block_forward_noalloc", 0, dev(x), empty((S, HIDDEN)), dev(cos), dev(sin), None, True, S)
    finally:
        torch.cuda.synchronize()
        c.close()


def test_no_alloc_text_block_under_graph_capture():
    # The callers the entry point is for: one call recorded into a HIP graph on the
    # context's stream, then replayed on new inputs copied into the same buffers. Each
    # replay (with this program's own eager work and a synchronisation between replays)
    # must equal the allocating entry point on the same inputs, bitwise.
    import torch
    dt, S = E.FP16, 48
    c = E.Context(0)
    stream = torch.cuda.Stream()
    try:
        w = small_text_block(seed=71, hidden=HIDDEN, heads=HEADS, kv_heads=KV_HEADS, ffn=FFN, std=0.02)
        c.text_block_upload(0, w, HIDDEN, HEADS, KV_HEADS, FFN, dt)
        x, cos, sin, _ = text_inputs(S, seed=72)
        xd, cd, sd, out = dev(x), dev(cos), dev(sin), empty((S, HIDDEN))
        args = (0, E.ptr(xd), E.ptr(out), E.ptr(cd), E.ptr(sd), None, 1, S)
        torch.cuda.synchronize()
        c.call("set_stream", E.c_vp(stream.cuda_stream))
        c.call("text_block_forward_noalloc", *args)  # code objects loaded outside the capture
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream, capture_error_mode="relaxed"):
            c.call("text_block_forward_noalloc", *args)
        for seed in (73, 74, 75):
            xn, _, _, _ = text_inputs(S, seed=seed)
            xd.copy_(torch.from_numpy(xn).cuda())
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got = host(out)
            ref = forward(c, "text_block_forward", 0, xd, empty((S, HIDDEN)), cd, sd, None, True, S)
            assert np.isfinite(ref).all()
            np.testing.assert_array_equal(got, ref, err_msg=f"replay with input seed {seed}")
    finally:
        torch.cuda.synchronize()
        c.close()
