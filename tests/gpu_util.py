"""Helpers for the GPU tests: numpy <-> device tensors (torch is only the
allocator and stream here; every computation goes through libtbq)."""
import numpy as np


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to("cuda")


def empty(n, dtype):
    import torch
    return torch.empty(n, dtype=dtype, device="cuda")


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()
