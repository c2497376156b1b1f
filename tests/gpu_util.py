"""Helpers of the GPU parity tests: device copies through torch (the allocator), tolerance checks."""
import ctypes
import sys

import numpy as np


# Device tensors handed to asynchronous launches stay referenced until the next host() synchronises, so the
# caching allocator cannot hand their memory to a later allocation while a kernel may still read it.
_live = []


def dev(a):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(a)).cuda()
    _live.append(t)
    return t


def zeros(shape, dtype):
    import torch
    t = torch.zeros(shape, dtype=dtype, device="cuda")
    _live.append(t)
    return t


def host(t):
    import torch
    torch.cuda.synchronize()
    out = t.cpu().numpy()
    _live.clear()
    return out


def rel_l2(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30))


def announce(*parts):
    """Name the case before a GPU step (flushed, so a crash still shows what ran)."""
    print("[gpu case]", *parts, flush=True)
    sys.stdout.flush()


def cvoid(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())
