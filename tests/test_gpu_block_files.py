"""Blocks loaded from block.ncnn.param + block.ncnn.bin compute exactly what
the same weights uploaded from FP32 host arrays compute.

The weights are chosen exact in FP32, BF16 and FP16, so every ModelBin storage
tag describes the same values; the device outputs must then agree bitwise.
"""
import numpy as np
import pytest

import ernie_amd as E
from gpu_util import NAMES, ALL_DT, dev, empty, host
from test_block_files import COMPONENT, exact_weights, synthetic_graph, write_block_bin
from test_oracle import small_inputs

pytestmark = pytest.mark.gpu


def forward(ctx, index, x, mods, cos, sin, mask):
    S, dim = x.shape
    out = empty((S, dim))
    valid = int(np.sum(mask == 0))
    ctx.block_forward(index, dev(x), out, dev(mods), dev(cos), dev(sin), S, mask=dev(mask), valid_keys=valid)
    return host(out)


@pytest.mark.parametrize("dt", ALL_DT, ids=lambda d: NAMES[d])
def test_loaded_block_matches_uploaded_block(tmp_path, dt):
    dim, ffn = 256, 512
    fac = E.Facade(0)
    try:
        w = exact_weights(dim, ffn, seed=3)
        graph = tmp_path / "block.ncnn.param"
        graph.write_text(synthetic_graph(dim, ffn))
        layouts = {"fp32": E.FP32, "bf16": E.BF16, "fp16": E.FP16,
                   "mixed": [E.BF16, E.FP32, E.FP16, E.BF16, E.FP16, E.FP32, E.BF16]}
        x, mods, cos, sin, mask = small_inputs(S=40, dim=dim)
        fac.hip.block_upload(0, w, dim, ffn, dt)
        ref = forward(fac.hip, 0, x, mods, cos, sin, mask)
        assert np.isfinite(ref).all()
        for i, (name, storage) in enumerate(layouts.items(), start=1):
            b = tmp_path / f"{name}.bin"
            write_block_bin(b, w, storage)
            info = fac.block_load(i, graph, b, dt, allow_unreviewed=True)
            assert (info["dim"], info["ffn"], info["contract"]) == (dim, ffn, "unreviewed")
            np.testing.assert_array_equal(forward(fac.hip, i, x, mods, cos, sin, mask), ref, err_msg=name)
        # An unreviewed graph is refused unless the caller opts in; the slot keeps its weights.
        with pytest.raises(E.ErnieInvalidRequest):
            fac.block_load(1, graph, tmp_path / "bf16.bin", dt)
        np.testing.assert_array_equal(forward(fac.hip, 1, x, mods, cos, sin, mask), ref)
    finally:
        fac.close()


def test_full_size_bf16_file_in_the_reviewed_graph(tmp_path):
    # A 4096-wide block stored the way the reference ships it: BF16 Gemm sections in
    # the reviewed component graph, loaded at BF16 and at FP16 storage.
    dim, ffn = 4096, 12288
    fac = E.Facade(0)
    try:
        w = exact_weights(dim, ffn, seed=4)
        b = tmp_path / "block.ncnn.bin"
        write_block_bin(b, w, E.BF16)
        x, mods, cos, sin, mask = small_inputs(S=288, dim=dim, image=(16, 16), valid=20, seed=5)
        for dt in (E.BF16, E.FP16):
            info = fac.block_load(10, COMPONENT, b, dt)
            assert (info["contract"], info["tokens"], info["bin_bytes"]) == ("component", 288, b.stat().st_size)
            fac.hip.block_upload(11, w, dim, ffn, dt)
            got = forward(fac.hip, 10, x, mods, cos, sin, mask)
            np.testing.assert_array_equal(got, forward(fac.hip, 11, x, mods, cos, sin, mask), err_msg=NAMES[dt])
            assert np.isfinite(got).all()
        for i in (10, 11):
            fac.hip.call("block_release", i)
    finally:
        fac.close()
