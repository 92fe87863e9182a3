"""Device helpers for the GPU parity tests: numpy <-> torch device tensors on the current HIP stream."""
import numpy as np

_torch = None


def torch():
    """torch, with a dedicated (non-null, default-priority) stream made current: the reference's entry points
    reject the null stream (mmvq:2323-2325) and so do ours."""
    global _torch
    if _torch is None:
        import torch as t
        t.cuda.set_stream(t.cuda.Stream(device=0))
        _torch = t
    return _torch


def dev(a, dtype=None):
    """Copy a numpy array to cuda:0 (uint8 / float32 / int32 / uint16 keep their dtype)."""
    t = torch()
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        a = a.view(np.int16)
    return t.from_numpy(a.copy()).to("cuda:0")


def empty(n, dtype="float32"):
    t = torch()
    return t.empty(n, dtype=getattr(t, dtype), device="cuda:0")


def host(t):
    torch().cuda.synchronize()
    a = t.detach().cpu().numpy()
    if a.dtype == np.int16:
        a = a.view(np.uint16)
    return a


def assert_close_rel(actual, ref, rtol=1e-3, atol_frac=1e-5, what=""):
    """|actual - ref| <= rtol * |ref| + atol_frac * max|ref|, elementwise."""
    actual = np.asarray(actual, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    scale = max(float(np.abs(ref).max()), 1e-30)
    err = np.abs(actual - ref)
    bound = rtol * np.abs(ref) + atol_frac * scale
    bad = np.nonzero(err > bound)[0]
    assert bad.size == 0, (f"{what}: {bad.size} of {ref.size} outside tolerance; worst idx {bad[np.argmax(err[bad])]} "
                           f"err {err[bad].max():.3e} ref scale {scale:.3e}")
