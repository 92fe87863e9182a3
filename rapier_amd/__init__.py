"""rapier_amd - MI355X-native exact-verify MTP hot path for the qwen35 hybrid (Rapier's engine, gfx950).

The compute lives in ``librapier_mi.so`` (hand-written HIP, C ABI declared in ``include/rapier_mi.h``).  This module
is the host-side mirror of the reference's ``strata::kernels`` launch surface: the same function names, argument
meaning and error behaviour (``ValueError`` where the reference throws ``std::invalid_argument``, ``RuntimeError``
for ``std::runtime_error``).  Device memory and streams come from PyTorch (``torch.Tensor`` arguments); nothing
here computes on the CPU.  A missing library is an ``ImportError``-style failure, never a fallback.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "librapier_mi.so")
CSRC = os.path.join(_HERE, "csrc")

RMI_OK, RMI_ERR_SHAPE, RMI_ERR_POINTER, RMI_ERR_STREAM, RMI_ERR_LAUNCH, RMI_ERR_UNSUPPORTED, RMI_ERR_STATE = range(7)
GGML_Q8_0, GGML_Q6_K = 8, 14
Q6K_BYTES, Q8_0_BYTES, Q8_1_BYTES = 210, 34, 36

_lib = None
_vp, _i, _f, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes); every int-returning entry is a status code checked by _call
SIGNATURES = {
    "rmi_last_error": (ctypes.c_char_p, []),
    "rmi_version": (ctypes.c_char_p, []),
    "rmi_native_q8_1_bytes": (_sz, [_i, _i]),
    "rmi_native_quantize_q8_1": (_i, [_vp, _vp, _i, _i, _vp]),
    "rmi_native_q6_k_mmvq": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_native_q6_k_mmvq_res": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _vp]),
    "rmi_native_q6_k_mmvq_res_n": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_q6_k_block_dots": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
}


class RapierError(RuntimeError):
    pass


def build(force: bool = False, jobs: int = 8) -> str:
    """Compile librapier_mi.so for gfx950 with hipcc (cross-compiles without a GPU)."""
    cmd = ["make", f"-j{jobs}"] + (["-B"] if force else [])
    subprocess.run(cmd, cwd=CSRC, check=True)
    return LIB_PATH


def lib():
    """The loaded HIP library.  Raises if it has not been built: there is no CPU fallback."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"rapier_amd: {LIB_PATH} is missing; run __graft_entry__.build() first")
        # One HIP runtime per process: torch bundles its own libamdhip64 (soname libamdhip64.so.7).  Loading torch
        # first makes our NEEDED libamdhip64.so.7 bind to that copy, so device pointers and streams are shared;
        # loading ours first would start a second runtime that does not see torch's allocations.
        try:
            import torch  # noqa: F401
        except ImportError:
            pass
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def last_error() -> str:
    return lib().rmi_last_error().decode()


def _call(name, *args):
    rc = getattr(lib(), name)(*args)
    if rc != RMI_OK:
        msg = last_error()
        if rc in (RMI_ERR_SHAPE, RMI_ERR_POINTER, RMI_ERR_STREAM, RMI_ERR_UNSUPPORTED):
            raise ValueError(msg)
        raise RapierError(msg)


def _p(t):
    """Device pointer of a torch tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(stream):
    if stream is None:
        import torch
        return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    if isinstance(stream, int):
        return ctypes.c_void_p(stream)
    return ctypes.c_void_p(stream.cuda_stream)


# ---- strata::kernels mirror -----------------------------------------------------------------------------------------

def native_q8_1_bytes(n_in: int, ncols: int) -> int:
    n = lib().rmi_native_q8_1_bytes(n_in, ncols)
    if n == 0:
        raise ValueError(last_error())
    return n


def native_quantize_q8_1(x, x_q8_1, n_in: int, ncols: int, stream=None):
    _call("rmi_native_quantize_q8_1", _p(x), _p(x_q8_1), n_in, ncols, _stream(stream))


def native_q6_k_mmvq(w, x_q8_1, y, n_in: int, n_out: int, ncols: int, stream=None):
    _call("rmi_native_q6_k_mmvq", _p(w), _p(x_q8_1), _p(y), n_in, n_out, ncols, _stream(stream))


def native_q6_k_mmvq_res(w, x_q8_1, y, res, partials, n_in: int, n_out: int, stream=None):
    _call("rmi_native_q6_k_mmvq_res", _p(w), _p(x_q8_1), _p(y), _p(res), _p(partials), n_in, n_out, _stream(stream))


def native_q6_k_mmvq_res_n(w, x_q8_1, y, res, partials, n_in: int, n_out: int, ncols: int, stream=None):
    _call("rmi_native_q6_k_mmvq_res_n", _p(w), _p(x_q8_1), _p(y), _p(res), _p(partials), n_in, n_out, ncols,
          _stream(stream))


def q6_k_block_dots(w, x_q8_1, out, n_in: int, n_out: int, stream=None):
    _call("rmi_q6_k_block_dots", _p(w), _p(x_q8_1), _p(out), n_in, n_out, _stream(stream))
