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
    "rmi_native_q4_k_mmvq": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_native_q5_k_mmvq": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_native_q4_k_mmvq_res_n": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_native_q5_k_mmvq_res_n": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_native_q4_k_mmvq_res": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _vp]),
    "rmi_native_q5_k_mmvq_res": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _vp]),
    "rmi_q6_k_packed_bytes": (_sz, [_i, _i]),
    "rmi_q6_k_pack": (_i, [_vp, _vp, _i, _i, _vp]),
    "rmi_native_q6_k_pack_copy": (_i, [_vp, _i, _i]),
    "rmi_native_q6_k_unpack": (_i, [_vp]),
    "rmi_native_q6_k_packed_copies": (_i, []),
    "rmi_q6_k_pack_swiglu": (_i, [_vp, _vp, _i, _i, _vp]),
    "rmi_native_q6_k_swiglu_packed": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_rms_quant_apply_self": (_i, [_vp, _vp, _vp, _i, _f, _i, _vp]),
    "rmi_native_q6_k_mmvq_packed": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_native_q6_k_mmvq_packed_res_n": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_q6_k_block_dots": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "rmi_native_q6_k_mmvq_packed_norm": (_i, [_vp, _vp, _vp, _vp, _f, _vp, _i, _i, _i, _vp]),
    "rmi_native_q6_k_swiglu_packed_norm": (_i, [_vp, _vp, _vp, _vp, _f, _vp, _i, _i, _i, _vp]),
    "rmi_q6_k_packed_norm_preferred": (_i, [_i, _i, _i]),
    "rmi_gen_q6_k": (_i, [_vp, _sz, ctypes.c_uint64, _f, _vp]),
    "rmi_gen_q8_0": (_i, [_vp, _sz, ctypes.c_uint64, _f, _vp]),
    "rmi_gen_normal": (_i, [_vp, _sz, ctypes.c_uint64, _f, _f, _vp]),
    "rmi_gen_normal_f16": (_i, [_vp, _sz, ctypes.c_uint64, _f, _f, _vp]),
    "rmi_stream_read": (_i, [_vp, _sz, _i, _vp, _vp]),
    "rmi_gdn_exchange_timeouts": (ctypes.c_uint, []),
    "rmi_gdn_exchange_test": (_i, [ctypes.c_uint, _i]),
    "rmi_gdn_exchange_bytes": (_sz, [_i]),
    "rmi_gdn_layer_tokens_x": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _vp, _vp, _vp, _f, _vp, _i, _vp,
                                    _i, _i, _i, _i, _vp, _vp]),
    "rmi_rms_quant_apply": (_i, [_vp, _vp, _vp, _vp, _i, _f, _i, _vp]),
    "rmi_rms_quant_apply_pair": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _f, _i, _vp]),
    "rmi_rms_norm_out": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _f, _i, _vp]),
    "rmi_rms_norm_out_strided": (_i, [_vp, _vp, _vp, _vp, _i, _vp, _i, _f, _i, _vp]),
    "rmi_row_sum_partials": (_i, [_vp, _vp, _i, _i, _vp]),
    "rmi_add_partials": (_i, [_vp, _vp, _vp, _i, _i, _vp]),
    "rmi_swiglu_quant": (_i, [_vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_swiglu_quant_interleaved": (_i, [_vp, _vp, _i, _i, _i, _vp]),
    "rmi_sig_mul_quant": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "rmi_beta_gate": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_argmax_workspace_bytes": (_sz, [_i]),
    "rmi_argmax": (_i, [_vp, _i, _i, _i, _vp, _vp, _vp]),
    "rmi_topk_workspace_bytes": (_sz, [_i]),
    "rmi_topk": (_i, [_vp, _i, _i, _vp, _vp, _vp, _vp]),
    "rmi_embed_q6_k": (_i, [_vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_embed": (_i, [_i, _vp, _vp, _vp, _vp, _i, _i, _i, _vp]),
    "rmi_embed_quant_apply_pair": (_i, [_i, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _f, _i, _vp]),
    "rmi_fused_gdn_conv_l2": (_i, [_vp, _vp, _vp, _vp, _i, _i, _f, _vp]),
    "rmi_fused_gdn_step_norm_silu_q8": (_i, [_vp] * 8 + [_f, _vp, _vp, _i, _i, _vp]),
    "rmi_gdn_layer_tokens": (_i, [_vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _vp, _vp, _vp, _f, _vp, _i, _vp,
                                  _i, _i, _i, _i, _vp]),
    "rmi_attn_prep": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _f, _f, _i, _i, _vp]),
    "rmi_attn_prep_rope": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _i, _i, _i, _vp, _f, _i, _i, _vp]),
    "rmi_gqa_flash_decode_prep": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _vp,
                                       _f, _i, _i, _i, _f, _vp]),
    "rmi_gqa_rope_table_bytes": (ctypes.c_size_t, [_i]),
    "rmi_gqa_flash_decode_prep_rt": (_i, [_vp, _i, _vp, _vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i,
                                          _vp, _f, _i, _i, _i, _f, _vp, _i, _vp]),
    "rmi_rms_norm_weighted": (_i, [_vp, _vp, _i, _i, _f, _vp]),
    "rmi_native_rope_apply": (_i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    "rmi_add_inplace": (_i, [_vp, _vp, _i, _vp]),
    "rmi_scale_inplace": (_i, [_vp, _i, _f, _vp]),
    "rmi_silu_inplace": (_i, [_vp, _i, _vp]),
    "rmi_gqa_workspace_bytes": (_sz, [_i, _i, _i]),
    "rmi_gqa_noalloc_scratch_bytes": (_sz, [_i, _i, _i, _i]),
    "rmi_gqa_noalloc_scratch_max": (_sz, []),
    "rmi_gqa_flash_decode_noalloc": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _i, _f,
                                          _vp]),
    "rmi_gqa_flash_decode": (_i, [_vp, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _i, _vp, _i, _i, _i, _i, _i, _i, _f,
                                  _vp]),
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


def _check(rc):
    if rc != RMI_OK:
        msg = last_error()
        if rc in (RMI_ERR_SHAPE, RMI_ERR_POINTER, RMI_ERR_STREAM, RMI_ERR_UNSUPPORTED):
            raise ValueError(msg)
        raise RapierError(msg)


def _call(name, *args):
    _check(getattr(lib(), name)(*args))


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


def native_kquant_mmvq(ggml_type, w, x_q8_1, y, n_in: int, n_out: int, ncols: int = 1, stream=None):
    """Q4_K (12) / Q5_K (13) x Q8_1 GEMV"""
    name = {12: "rmi_native_q4_k_mmvq", 13: "rmi_native_q5_k_mmvq"}[ggml_type]
    _call(name, _p(w), _p(x_q8_1), _p(y), n_in, n_out, ncols, _stream(stream))


def native_kquant_mmvq_res_n(ggml_type, w, x_q8_1, y, res, partials, n_in: int, n_out: int, ncols: int = 1,
                             stream=None):
    name = {12: "rmi_native_q4_k_mmvq_res_n", 13: "rmi_native_q5_k_mmvq_res_n"}[ggml_type]
    _call(name, _p(w), _p(x_q8_1), _p(y), _p(res), _p(partials), n_in, n_out, ncols, _stream(stream))


def q6_k_packed_bytes(n_in: int, n_out: int) -> int:
    n = lib().rmi_q6_k_packed_bytes(n_in, n_out)
    if n == 0:
        raise ValueError(last_error())
    return n


def q6_k_pack(w, w_packed, n_in: int, n_out: int, stream=None):
    _call("rmi_q6_k_pack", _p(w), _p(w_packed), n_in, n_out, _stream(stream))


def native_q6_k_pack(w, n_in: int, n_out: int) -> bool:
    """native_q6_k_pack (mmvq:2930-2960): a library-owned packed copy of the GGUF-layout matrix ``w`` that
    native_q6_k_mmvq / _res / _res_n then run on (the same bits); False where the packed layout does not take the
    shape, as the reference returns false."""
    rc = lib().rmi_native_q6_k_pack_copy(_p(w), n_in, n_out)
    if rc == RMI_ERR_UNSUPPORTED:
        return False
    _check(rc)
    return True


def native_q6_k_unpack(w):
    _call("rmi_native_q6_k_unpack", _p(w))


def native_q6_k_packed_copies() -> int:
    return int(lib().rmi_native_q6_k_packed_copies())


def q6_k_pack_swiglu(w, w_packed, n_in: int, n_ff: int, stream=None):
    """pack an up||gate Q6_K matrix ([up n_ff rows | gate n_ff rows]) in the SwiGLU row order"""
    _call("rmi_q6_k_pack_swiglu", _p(w), _p(w_packed), n_in, n_ff, _stream(stream))


def native_q6_k_swiglu_packed(w_packed, x_q8_1, y_q8_1, n_in: int, n_ff: int, ncols: int, stream=None):
    """Q8_1 of silu(gate) * up from an up||gate matrix packed by q6_k_pack_swiglu (one launch)"""
    _call("rmi_native_q6_k_swiglu_packed", _p(w_packed), _p(x_q8_1), _p(y_q8_1), n_in, n_ff, ncols, _stream(stream))


def native_q6_k_mmvq_packed(w_packed, x_q8_1, y, n_in: int, n_out: int, ncols: int, stream=None):
    _call("rmi_native_q6_k_mmvq_packed", _p(w_packed), _p(x_q8_1), _p(y), n_in, n_out, ncols, _stream(stream))


def native_q6_k_mmvq_packed_norm(w_packed, x, w_norm, partials, eps, y, n_in: int, n_out: int, ncols: int,
                                 stream=None):
    """rms_quant_apply + packed GEMV in one launch (the norm quantized in the GEMV's stage); same bits as the pair"""
    _call("rmi_native_q6_k_mmvq_packed_norm", _p(w_packed), _p(x), _p(w_norm), _p(partials), eps, _p(y), n_in, n_out,
          ncols, _stream(stream))


def native_q6_k_swiglu_packed_norm(w_packed, x, w_norm, partials, eps, y_q8_1, n_in: int, n_ff: int, ncols: int,
                                   stream=None):
    """rms_quant_apply + the fused up||gate SwiGLU GEMV in one launch; same bits as the pair"""
    _call("rmi_native_q6_k_swiglu_packed_norm", _p(w_packed), _p(x), _p(w_norm), _p(partials), eps, _p(y_q8_1), n_in,
          n_ff, ncols, _stream(stream))


def native_q6_k_mmvq_packed_res_n(w_packed, x_q8_1, y, res, partials, n_in: int, n_out: int, ncols: int,
                                  stream=None):
    _call("rmi_native_q6_k_mmvq_packed_res_n", _p(w_packed), _p(x_q8_1), _p(y), _p(res), _p(partials), n_in, n_out,
          ncols, _stream(stream))


def q6_k_block_dots(w, x_q8_1, out, n_in: int, n_out: int, stream=None):
    _call("rmi_q6_k_block_dots", _p(w), _p(x_q8_1), _p(out), n_in, n_out, _stream(stream))


# ---- seeded synthetic tensors in HBM (random-init stand-in for a GGUF file) -----------------------------------------

def gen_q6_k(w, nblocks: int, seed: int, d_std: float = 1e-3, stream=None):
    """Fill ``nblocks`` Q6_K blocks: codes U{0..63}, sub-scales U[-32,31], d = fp16(|N(0, d_std)|)."""
    _call("rmi_gen_q6_k", _p(w), nblocks, seed, d_std, _stream(stream))


def gen_q8_0(w, nblocks: int, seed: int, d_std: float = 1e-2, stream=None):
    _call("rmi_gen_q8_0", _p(w), nblocks, seed, d_std, _stream(stream))


def gen_normal(out, n: int, seed: int, mean: float = 0.0, std: float = 1.0, stream=None):
    _call("rmi_gen_normal", _p(out), n, seed, mean, std, _stream(stream))


def gen_normal_f16(out, n: int, seed: int, mean: float = 0.0, std: float = 1.0, stream=None):
    _call("rmi_gen_normal_f16", _p(out), n, seed, mean, std, _stream(stream))


def stream_read(buf, nbytes: int, grid: int, out, stream=None):
    """the single-launch read-bandwidth reference: streams nbytes of buf with grid x 256 lanes and discards them"""
    _call("rmi_stream_read", _p(buf), nbytes, grid, _p(out), _stream(stream))


# ---- norm / activation epilogues (qw:602-715) ----------------------------------------------------------------------

def rms_quant_apply(x, w, partials, y_q8_1, cols, eps, ncols=1, stream=None):
    _call("rmi_rms_quant_apply", _p(x), _p(w), _p(partials), _p(y_q8_1), cols, eps, ncols, _stream(stream))


def rms_quant_apply_self(x, w, y_q8_1, cols, eps, ncols=1, stream=None):
    """row_sum_partials(x) + rms_quant_apply in one launch (same bytes)"""
    _call("rmi_rms_quant_apply_self", _p(x), _p(w), _p(y_q8_1), cols, eps, ncols, _stream(stream))


def rms_quant_apply_pair(x0, w0, partials0, x1, w1, partials1, y_q8_1, cols, eps, ncols=1, stream=None):
    _call("rmi_rms_quant_apply_pair", _p(x0), _p(w0), _p(partials0), _p(x1), _p(w1), _p(partials1), _p(y_q8_1), cols,
          eps, ncols, _stream(stream))


def rms_norm_out(x, w, partials, out, out_partials, cols, eps, ncols=1, stream=None):
    _call("rmi_rms_norm_out", _p(x), _p(w), _p(partials), _p(out), _p(out_partials), cols, eps, ncols,
          _stream(stream))


def rms_norm_out_strided(x, w, partials, out, out_stride, out_partials, cols, eps, ncols=1, stream=None):
    _call("rmi_rms_norm_out_strided", _p(x), _p(w), _p(partials), _p(out), out_stride, _p(out_partials), cols, eps,
          ncols, _stream(stream))


def row_sum_partials(x, partials, n, ncols=1, stream=None):
    _call("rmi_row_sum_partials", _p(x), _p(partials), n, ncols, _stream(stream))


def add_partials(x, o, partials, n, ncols=1, stream=None):
    _call("rmi_add_partials", _p(x), _p(o), _p(partials), n, ncols, _stream(stream))


def swiglu_quant(up, gate, y_q8_1, n, ncols=1, col_stride=None, stream=None):
    _call("rmi_swiglu_quant", _p(up), _p(gate), _p(y_q8_1), n, ncols, n if col_stride is None else col_stride,
          _stream(stream))


def swiglu_quant_interleaved(up_gate, y_q8_1, n, ncols=1, col_stride=None, stream=None):
    _call("rmi_swiglu_quant_interleaved", _p(up_gate), _p(y_q8_1), n, ncols, 2 * n if col_stride is None else col_stride,
          _stream(stream))


def sig_mul_quant(o, g, y_q8_1, n, ncols=1, o_stride=None, g_stride=None, stream=None):
    _call("rmi_sig_mul_quant", _p(o), _p(g), _p(y_q8_1), n, ncols, n if o_stride is None else o_stride,
          n if g_stride is None else g_stride, _stream(stream))


def beta_gate(beta_alpha, dt, ssm_a, ggate, n, ncols=1, ab_stride=None, stream=None):
    _call("rmi_beta_gate", _p(beta_alpha), _p(dt), _p(ssm_a), _p(ggate), n, ncols,
          2 * n if ab_stride is None else ab_stride, _stream(stream))


def argmax_workspace_bytes(ncols):
    return lib().rmi_argmax_workspace_bytes(ncols)


def argmax(logits, n, out_idx, workspace, ncols=1, col_stride=None, stream=None):
    _call("rmi_argmax", _p(logits), n, ncols, n if col_stride is None else col_stride, _p(out_idx), _p(workspace),
          _stream(stream))


def topk_workspace_bytes(n):
    return lib().rmi_topk_workspace_bytes(n)


def topk(logits, n, k, out_idx, out_val, workspace, stream=None):
    """the k largest of n logits: out_idx (int32) and out_val (fp32), logit descending, lower id first on ties"""
    _call("rmi_topk", _p(logits), n, k, _p(out_idx), _p(out_val), _p(workspace), _stream(stream))


def embed_q6_k(emb, tokens, x, partials, n_embd, n_vocab, ncols=1, stream=None):
    _call("rmi_embed_q6_k", _p(emb), _p(tokens), _p(x), _p(partials), n_embd, n_vocab, ncols, _stream(stream))


def embed(ggml_type, emb, tokens, x, partials, n_embd, n_vocab, ncols=1, stream=None):
    """token rows of a GGUF type 14 (Q6_K) / 13 (Q5_K) / 12 (Q4_K) table, dequantized on the device"""
    _call("rmi_embed", ggml_type, _p(emb), _p(tokens), _p(x), _p(partials), n_embd, n_vocab, ncols, _stream(stream))


def embed_quant_apply_pair(ggml_type, emb, tokens, w0, x1, w1, partials1, y_q8_1, cols, n_vocab, eps, ncols=1,
                           stream=None):
    """embed + rms_quant_apply_pair(embedding rows, w0, .., x1, w1, partials1) in one launch (same bytes)"""
    _call("rmi_embed_quant_apply_pair", ggml_type, _p(emb), _p(tokens), _p(w0), _p(x1), _p(w1), _p(partials1),
          _p(y_q8_1), cols, n_vocab, eps, ncols, _stream(stream))


# ---- Gated DeltaNet (fgdn:40-133) ----------------------------------------------------------------------------------

def fused_gdn_conv_l2(history, qkv, conv_w, h, channels, qk_heads, eps, stream=None):
    _call("rmi_fused_gdn_conv_l2", _p(history), _p(qkv), _p(conv_w), _p(h), channels, qk_heads, eps, _stream(stream))


def fused_gdn_step_norm_silu_q8(state, q, k, v, gate, beta, z, gamma, eps, y, q8, h_k, h_v, stream=None):
    _call("rmi_fused_gdn_step_norm_silu_q8", _p(state), _p(q), _p(k), _p(v), _p(gate), _p(beta), _p(z), _p(gamma),
          eps, _p(y), _p(q8), h_k, h_v, _stream(stream))


def gdn_exchange_timeouts() -> int:
    """bounded waits of the split GDN kernel that ran out (0 in every correct run)"""
    return lib().rmi_gdn_exchange_timeouts()


def gdn_exchange_test(spin_limit: int = 0, force_miss: bool = False) -> None:
    """test hook: the split GDN kernel's wait bound (0 = default) and a switch that makes every wait time out"""
    _call("rmi_gdn_exchange_test", spin_limit, 1 if force_miss else 0)


def gdn_exchange_bytes(h_v: int) -> int:
    return lib().rmi_gdn_exchange_bytes(h_v)


def gdn_layer_tokens_x(state_a, state_b, hist_a, hist_b, sel, qkvz, qkvz_stride, ab, ab_stride, conv_w, dt, ssm_a,
                       gamma, eps, y, y_stride, q8, q8_stride, h_k, h_v, ntok, xch, stream=None):
    """gdn_layer_tokens with 1 / 2-token launches on four workgroups per value head (xch: zeroed exchange buffer)"""
    _call("rmi_gdn_layer_tokens_x", _p(state_a), _p(state_b), _p(hist_a), _p(hist_b), _p(sel), _p(qkvz), qkvz_stride,
          _p(ab), ab_stride, _p(conv_w), _p(dt), _p(ssm_a), _p(gamma), eps, _p(y), y_stride, _p(q8), q8_stride, h_k,
          h_v, ntok, _p(xch), _stream(stream))


def gdn_layer_tokens(state_a, state_b, hist_a, hist_b, sel, qkvz, qkvz_stride, ab, ab_stride, conv_w, dt, ssm_a,
                     gamma, eps, y, y_stride, q8, q8_stride, h_k, h_v, ntok, stream=None):
    _call("rmi_gdn_layer_tokens", _p(state_a), _p(state_b), _p(hist_a), _p(hist_b), _p(sel), _p(qkvz), qkvz_stride,
          _p(ab), ab_stride, _p(conv_w), _p(dt), _p(ssm_a), _p(gamma), eps, _p(y), y_stride, _p(q8), q8_stride, h_k,
          h_v, ntok, _stream(stream))


# ---- attention --------------------------------------------------------------------------------------------------------

def attn_prep(q3, q3_stride, qn, kn, kcache, vcache, pos, qout, n_head, n_kv, head_dim, n_rot, theta, eps, ntok,
              max_ctx, stream=None):
    _call("rmi_attn_prep", _p(q3), q3_stride, _p(qn), _p(kn), _p(kcache), _p(vcache), _p(pos), _p(qout), n_head,
          n_kv, head_dim, n_rot, theta, eps, ntok, max_ctx, _stream(stream))


class RopeParams(ctypes.Structure):
    """rmi_rope_params: YaRN as the reference configures it (qw:1991-1999)"""
    _fields_ = [(n, ctypes.c_float) for n in ("freq_base", "factor", "orig_ctx", "ext_factor", "attn_factor",
                                              "beta_fast", "beta_slow")]


def attn_prep_rope(q3, q3_stride, qn, kn, kcache, vcache, pos, qout, n_head, n_kv, head_dim, n_rot, freq_base, factor,
                   orig_ctx, eps, ntok, max_ctx, ext_factor=1.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0,
                   stream=None):
    rope = RopeParams(freq_base, factor, orig_ctx, ext_factor, attn_factor, beta_fast, beta_slow)
    _call("rmi_attn_prep_rope", _p(q3), q3_stride, _p(qn), _p(kn), _p(kcache), _p(vcache), _p(pos), _p(qout), n_head,
          n_kv, head_dim, n_rot, ctypes.byref(rope), eps, ntok, max_ctx, _stream(stream))


def gqa_flash_decode_prep(q3, q3_stride, qn, kn, kcache, vcache, pos, y, y_stride, q8, q8_stride, workspace, n_head,
                          n_kv, head_dim, n_rot, freq_base, factor, orig_ctx, eps, ntok, max_ctx, nsub, scale,
                          ext_factor=1.0, attn_factor=1.0, beta_fast=32.0, beta_slow=1.0, stream=None):
    """attn_prep folded into the split-K decode attention (one slot group: decode and verify)"""
    rope = RopeParams(freq_base, factor, orig_ctx, ext_factor, attn_factor, beta_fast, beta_slow)
    _call("rmi_gqa_flash_decode_prep", _p(q3), q3_stride, _p(qn), _p(kn), _p(kcache), _p(vcache), _p(pos), _p(y),
          y_stride, _p(q8), q8_stride, _p(workspace), n_head, n_kv, head_dim, n_rot, ctypes.byref(rope), eps, ntok,
          max_ctx, nsub, scale, _stream(stream))


def gqa_rope_table_bytes(n_rot: int) -> int:
    return lib().rmi_gqa_rope_table_bytes(n_rot)


def gqa_flash_decode_prep_rt(q3, q3_stride, qn, kn, kcache, vcache, pos, y, y_stride, q8, q8_stride, workspace,
                             n_head, n_kv, head_dim, n_rot, freq_base, factor, orig_ctx, eps, ntok, max_ctx, nsub,
                             scale, rope_table, table_mode, ext_factor=1.0, attn_factor=1.0, beta_fast=32.0,
                             beta_slow=1.0, stream=None):
    """gqa_flash_decode_prep with the forward pass's RoPE table (table_mode 0 compute, 1 compute and store, 2 load)"""
    rope = RopeParams(freq_base, factor, orig_ctx, ext_factor, attn_factor, beta_fast, beta_slow)
    _call("rmi_gqa_flash_decode_prep_rt", _p(q3), q3_stride, _p(qn), _p(kn), _p(kcache), _p(vcache), _p(pos), _p(y),
          y_stride, _p(q8), q8_stride, _p(workspace), n_head, n_kv, head_dim, n_rot, ctypes.byref(rope), eps, ntok,
          max_ctx, nsub, scale, _p(rope_table), table_mode, _stream(stream))


def rms_norm_weighted(x, w, rows, cols, eps, stream=None):
    """per-row RMSNorm in place (strata::kernels::rms_norm_weighted, qw:971-975)"""
    _call("rmi_rms_norm_weighted", _p(x), _p(w), rows, cols, eps, _stream(stream))


def native_rope_apply(x, y, heads, head_dim, n_rot, pos, freq_base, factor=1.0, orig_ctx=0.0, ext_factor=1.0,
                      attn_factor=1.0, beta_fast=32.0, beta_slow=1.0, stream=None):
    """NEOX / YaRN RoPE of each head at its device position pos[h] (strata::kernels::native_rope_apply)"""
    rope = RopeParams(freq_base, factor, orig_ctx, ext_factor, attn_factor, beta_fast, beta_slow)
    _call("rmi_native_rope_apply", _p(x), _p(y), heads, head_dim, n_rot, ctypes.byref(rope), _p(pos), _stream(stream))


def add_inplace(x, y, n, stream=None):
    _call("rmi_add_inplace", _p(x), _p(y), n, _stream(stream))


def scale_inplace(x, n, s, stream=None):
    _call("rmi_scale_inplace", _p(x), n, s, _stream(stream))


def silu_inplace(x, n, stream=None):
    _call("rmi_silu_inplace", _p(x), n, _stream(stream))


def gqa_workspace_bytes(max_ctx, n_kv, nsub):
    return lib().rmi_gqa_workspace_bytes(max_ctx, n_kv, nsub)


def gqa_flash_decode(q, kcache, vcache, pos, gate_src, gate_stride, y, y_stride, q8, q8_stride, workspace, n_head,
                     n_kv, head_dim, ntok, max_ctx, nsub, scale, stream=None):
    _call("rmi_gqa_flash_decode", _p(q), _p(kcache), _p(vcache), _p(pos), _p(gate_src), gate_stride, _p(y), y_stride,
          _p(q8), q8_stride, _p(workspace), n_head, n_kv, head_dim, ntok, max_ctx, nsub, scale, _stream(stream))


def gqa_flash_decode_noalloc(q, kcache, vcache, pos, gate_src, gate_stride, y, y_stride, q8, q8_stride, n_head, n_kv,
                             head_dim, ntok, max_ctx, nsub, scale, stream=None):
    """rmi_gqa_flash_decode without a workspace argument: the split-K records live in the library's own per-GPU
    scratch array (rmi_gqa_noalloc_scratch_max() bytes); no allocation.  Calls that overlap on one GPU race."""
    _call("rmi_gqa_flash_decode_noalloc", _p(q), _p(kcache), _p(vcache), _p(pos), _p(gate_src), gate_stride, _p(y),
          y_stride, _p(q8), q8_stride, n_head, n_kv, head_dim, ntok, max_ctx, nsub, scale, _stream(stream))
