"""Writes rope_inv_freq.f32: the 64-entry DiT RoPE frequency table evaluated with
PyTorch's FP32 CPU kernels, i.e. the expression of tools/prepare_pipeline.py:63
(cat over dims 32, 48, 48 of 1 / 256 ** (arange(0, dim, 2) / dim)). This is a
library evaluation of a published formula; the reference is not imported.
"""
from pathlib import Path

import torch

table = torch.cat([1. / (256 ** (torch.arange(0, dim, 2, dtype=torch.float32) / dim)) for dim in (32, 48, 48)])
assert table.dtype == torch.float32 and table.numel() == 64
out = Path(__file__).with_name("rope_inv_freq.f32")
table.numpy().astype("<f4").tofile(out)
print(out, table[:4].tolist())
