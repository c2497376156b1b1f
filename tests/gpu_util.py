"""Helpers of the GPU parity tests: device copies through torch (the allocator), tolerance checks."""
import ctypes
import sys

import numpy as np


def dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def zeros(shape, dtype):
    import torch
    return torch.zeros(shape, dtype=dtype, device="cuda")


def host(t):
    import torch
    torch.cuda.synchronize()
    return t.cpu().numpy()


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def announce(*parts):
    """Name the case before a GPU step (flushed, so a crash still shows what ran)."""
    print("[gpu case]", *parts, flush=True)
    sys.stdout.flush()


def cvoid(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())
