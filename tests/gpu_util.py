"""Helpers shared by the GPU parity tests (device buffers via torch)."""
import numpy as np
import torch

_NP2T = {
    np.dtype(np.int32): torch.int32,
    np.dtype(np.uint32): torch.uint32,
    np.dtype(np.float32): torch.float32,
    np.dtype(np.int64): torch.int64,
    np.dtype(np.uint64): torch.uint64,
    np.dtype(np.float64): torch.float64,
}


def to_dev(a: np.ndarray, pad: int = 0):
    """Copy a host array to cuda:0.  pad > 0 returns a view starting `pad`
    elements into a larger buffer (a pointer that is not 16-byte aligned)."""
    t = torch.empty(a.size + pad, dtype=_NP2T[a.dtype], device="cuda")
    view = t[pad:]
    view.copy_(torch.from_numpy(np.ascontiguousarray(a)))
    return view


def empty(n: int, dtype, pad: int = 0):
    t = torch.empty(n + pad, dtype=_NP2T[np.dtype(dtype)], device="cuda")
    return t[pad:]


def to_host(t) -> np.ndarray:
    torch.cuda.synchronize()
    return t.cpu().numpy()


def temp(nbytes: int):
    """Temp storage (torch's allocator returns >= 512-byte aligned blocks)."""
    return torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda") if nbytes else None


def random_array(dtype, n: int, seed: int = 0) -> np.ndarray:
    rng = np.random.default_rng(seed)
    dt = np.dtype(dtype)
    if dt.kind == "f":
        a = (rng.standard_normal(n) * 100).astype(dt)
        if n > 10:
            a[::37] = 0.0
            a[::41] = -0.0
        return a
    info = np.iinfo(dt)
    return rng.integers(info.min, info.max, size=n, dtype=dt, endpoint=True)
