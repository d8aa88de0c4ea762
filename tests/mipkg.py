"""Test-side access to the product package (its directory name is not an identifier) and
small torch helpers for device buffers. torch is only plumbing here: device memory and the
current stream handed to the C ABI."""
import importlib

import numpy as np

mi = importlib.import_module("intel-arc-inference-server_amd")


def torch():
    import torch as T
    return T


def dev(a):
    """numpy array -> torch device tensor with the same bytes."""
    if a is None:
        return None
    T = torch()
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        t = T.from_numpy(a.view(np.int16))
    elif a.dtype == np.uint32:
        t = T.from_numpy(a.view(np.int32))
    else:
        t = T.from_numpy(a)
    return t.to("cuda")


def host(t, dtype):
    """torch device tensor -> numpy array viewed as `dtype`."""
    return t.detach().cpu().numpy().view(dtype)


def empty(shape, dtype):
    T = torch()
    tmap = {np.uint16: T.int16, np.uint32: T.int32, np.float32: T.float32, np.int8: T.int8,
            np.float64: T.float64, np.int32: T.int32}
    return T.empty(shape, dtype=tmap[dtype], device="cuda")


def ptr(t):
    return t.data_ptr() if t is not None else None


def stream():
    return torch().cuda.current_stream().cuda_stream


def sync():
    torch().cuda.synchronize()
