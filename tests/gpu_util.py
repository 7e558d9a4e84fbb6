"""Device-buffer plumbing for the GPU tests (torch allocates, ernie_hip computes)."""
import numpy as np

import ernie_amd as E

TORCH_DT = {}


def torch_dtype(dt):
    import torch
    return {E.FP32: torch.float32, E.FP16: torch.float16, E.BF16: torch.bfloat16}[dt]


def dev(a, dt=E.FP32):
    """numpy FP32 -> device tensor in storage dtype (RNE conversion)."""
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()
    return t.to(torch_dtype(dt)).contiguous()


def empty(shape, dt=E.FP32):
    import torch
    return torch.empty(shape, dtype=torch_dtype(dt), device="cuda")


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.float().cpu().numpy()


def stored(a, dt):
    """The FP32 value of `a` after rounding to storage dtype dt."""
    return host(dev(a, dt))


NAMES = {E.FP32: "fp32", E.FP16: "fp16", E.BF16: "bf16"}
ALL_DT = [E.FP32, E.FP16, E.BF16]
