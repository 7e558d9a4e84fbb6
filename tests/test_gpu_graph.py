"""The DiT block path recorded into a HIP graph and replayed. Once a context's
workspace exists for a token count, a block sequence makes no allocation, host
synchronisation or memset, so a serving loop can capture it on the context's
stream and replay it on new inputs copied into the same buffers."""
import numpy as np
import pytest

import ernie_amd as E
import oracle as O
from gpu_util import dev, empty, host
from test_oracle import small_block, small_inputs

pytestmark = pytest.mark.gpu


def test_block_sequence_replayed_from_a_hip_graph():
    # Two FP16 blocks of width 1024 (8 heads), FFN 2048, S = 4136 = 16 x 256 + 40 (64 x 64
    # image tokens, 40 text, 30 valid): the captured launches include the rotary pair
    # packing, light tail tiles in the Q/K/V and up/gate GEMMs, the K-split output and
    # down GEMMs with their reductions, and the attention's key-split tail with its merge.
    # Every replay (with this program's own eager work and a synchronisation between
    # replays) must equal the eager sequence on the same inputs, bitwise.
    import torch
    dim, ffn, S, dt = 1024, 2048, 4136, E.FP16
    c = E.Context(0)
    stream = torch.cuda.Stream()
    try:
        for b in range(2):
            c.block_upload(b, small_block(dim=dim, ffn=ffn, seed=91, block=b), dim, ffn, dt)
        x, mods, cos, sin, mask = small_inputs(S=S, dim=dim, image=(64, 64), valid=30, seed=92)
        valid = int(np.sum(mask == 0))
        xd, out, md, cd, sd = dev(x), empty((S, dim)), dev(mods), dev(cos), dev(sin)
        torch.cuda.synchronize()
        c.call("set_stream", E.c_vp(stream.cuda_stream))
        # Workspace, rotary pair buffer and code objects come into being outside the capture.
        c.block_sequence([0, 1], xd, out, md, cd, sd, S, valid_keys=valid)
        stream.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph, stream=stream, capture_error_mode="relaxed"):
            c.block_sequence([0, 1], xd, out, md, cd, sd, S, valid_keys=valid)
        ref_out = empty((S, dim))
        for seed in (93, 94, 95):
            xd.copy_(torch.from_numpy(O.normal((S, dim), seed)).cuda())
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            got = host(out)
            c.block_sequence([0, 1], xd, ref_out, md, cd, sd, S, valid_keys=valid)
            stream.synchronize()
            ref = host(ref_out)
            assert np.isfinite(ref).all()
            assert float(np.abs(ref - host(xd)).max()) > 0  # the blocks changed the stream
            np.testing.assert_array_equal(got, ref, err_msg=f"replay with input seed {seed}")
    finally:
        torch.cuda.synchronize()
        c.close()
