"""CPU oracle for the exact-verify MTP hot path: numpy front end over ``liboracle.so``.

TEST INFRASTRUCTURE ONLY.  Imported by ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` as the checker; the product package ``rapier_amd`` never imports it.  Each wrapper names the C
function (and through it the reference file:line) it calls.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

Q6K_BYTES = 210
Q4K_BYTES = 144
Q5K_BYTES = 176
Q8_0_BYTES = 34
Q8_1_BYTES = 36

_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")
_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_c = ctypes
_SIGS = {
    "orc_rand_u64": (_c.c_uint64, [_c.c_uint64, _c.c_uint64]),
    "orc_rand_normal": (_c.c_double, [_c.c_uint64, _c.c_uint64]),
    "orc_fill_normal": (None, [_f32p, _c.c_size_t, _c.c_uint64, _c.c_double, _c.c_double]),
    "orc_gen_q6k": (None, [_u8p, _c.c_size_t, _c.c_uint64, _c.c_double]),
    "orc_gen_q8_0": (None, [_u8p, _c.c_size_t, _c.c_uint64, _c.c_double]),
    "orc_f32_to_f16": (_c.c_uint16, [_c.c_float]),
    "orc_f16_to_f32": (_c.c_float, [_c.c_uint16]),
    "orc_f16_sat": (_c.c_uint16, [_c.c_float]),
    "orc_quantize_q8_1": (None, [_f32p, _u8p, _c.c_int, _c.c_int]),
    "orc_dequantize_q8_1": (None, [_u8p, _f32p, _c.c_int]),
    "orc_q6k_code": (_c.c_int, [_u8p, _c.c_int]),
    "orc_q6k_dequant_row": (None, [_u8p, _f32p, _c.c_int]),
    "orc_q4k_dequant_row": (None, [_u8p, _f32p, _c.c_int]),
    "orc_q5k_dequant_row": (None, [_u8p, _f32p, _c.c_int]),
    "orc_q6k_block_dots": (None, [_u8p, _u8p, _i32p, _c.c_int, _c.c_int]),
    "orc_q6k_block_dots_lanes": (None, [_u8p, _u8p, _i32p, _c.c_int, _c.c_int]),
    "orc_q8_0_block_dots": (None, [_u8p, _u8p, _i32p, _c.c_int, _c.c_int]),
    "orc_q6k_gemv": (None, [_u8p, _u8p, _c.c_void_p, _f64p, _c.c_void_p, _c.c_int, _c.c_int, _c.c_int]),
    "orc_q8_0_gemv": (None, [_u8p, _u8p, _c.c_void_p, _f64p, _c.c_void_p, _c.c_int, _c.c_int, _c.c_int]),
    "orc_q4k_gemv": (None, [_u8p, _u8p, _c.c_void_p, _f64p, _c.c_void_p, _c.c_int, _c.c_int, _c.c_int]),
    "orc_q5k_gemv": (None, [_u8p, _u8p, _c.c_void_p, _f64p, _c.c_void_p, _c.c_int, _c.c_int, _c.c_int]),
    "orc_q6k_gemv_f32_omp": (None, [_u8p, _u8p, _c.c_void_p, _f32p, _c.c_void_p, _c.c_int, _c.c_int, _c.c_int,
                                     _c.c_int]),
    "orc_row_sum_partials": (None, [_f32p, _f64p, _c.c_int]),
    "orc_rms_inv": (_c.c_double, [_f64p, _c.c_int, _c.c_int, _c.c_double]),
    "orc_rms_norm_out": (None, [_f32p, _f32p, _c.c_double, _f64p, _c.c_int]),
    "orc_swiglu": (None, [_f32p, _f32p, _f64p, _c.c_int]),
    "orc_sig_mul": (None, [_f32p, _f32p, _f64p, _c.c_int]),
    "orc_beta_gate": (None, [_f32p, _f32p, _f32p, _f32p, _f64p, _f64p, _c.c_int]),
    "orc_gdn_conv_l2": (None, [_f32p, _f32p, _f32p, _f64p, _c.c_int, _c.c_int, _c.c_double]),
    "orc_gdn_step_norm": (None, [_f64p, _f64p, _f64p, _f64p, _f64p, _f64p, _f32p, _f32p, _c.c_double, _f64p,
                                 _c.c_int, _c.c_int]),
    "orc_gqa_decode": (None, [_f32p, _u16p, _u16p, _f64p, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_double]),
    "orc_rms_norm_heads": (None, [_f32p, _f32p, _f64p, _c.c_int, _c.c_int, _c.c_double]),
    "orc_rope_neox": (None, [_f64p, _f64p, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_double]),
    "orc_rope_yarn": (None, [_f64p, _f64p, _c.c_int, _c.c_int, _c.c_int, _c.c_int] + [_c.c_double] * 7),
    "orc_argmax": (_c.c_int, [_f32p, _c.c_int]),
    "orc_topk": (_c.c_int, [_f32p, _c.c_int, _c.c_int, _i32p, _f32p]),
}


def build(force: bool = False) -> str:
    """Compile liboracle.so with the Makefile beside this file (gcc, a few seconds)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-s", "-B" if force else "liboracle.so"], cwd=_HERE, check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        for name, (res, args) in _SIGS.items():
            fn = getattr(_lib, name)
            fn.restype = res
            fn.argtypes = args
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


# ---- generators --------------------------------------------------------------------------------------------------

def normal(n: int, seed: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_fill_normal(out, n, seed, mean, std)
    return out


def gen_q6k(n_out: int, n_in: int, seed: int, d_std: float = 1e-3) -> np.ndarray:
    """Q6_K matrix with codes U{0..63}, sub-scales U[-32,31], d = fp16(|N(0, d_std)|); row-major bytes."""
    nb = n_out * (n_in // 256)
    w = np.empty(nb * Q6K_BYTES, dtype=np.uint8)
    lib().orc_gen_q6k(w, nb, seed, d_std)
    return w


def gen_q8_0(n_out: int, n_in: int, seed: int, d_std: float = 1e-2) -> np.ndarray:
    nb = n_out * (n_in // 32)
    w = np.empty(nb * Q8_0_BYTES, dtype=np.uint8)
    lib().orc_gen_q8_0(w, nb, seed, d_std)
    return w


# ---- fp16 / Q8_1 -------------------------------------------------------------------------------------------------

def f16_to_f32(h: np.ndarray) -> np.ndarray:
    return np.asarray(h, dtype=np.uint16).view(np.float16).astype(np.float32)


def quantize_q8_1(x: np.ndarray, n_in: int, ncols: int = 1) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32).reshape(-1)
    assert x.size == n_in * ncols
    y = np.empty(ncols * (n_in // 32) * Q8_1_BYTES, dtype=np.uint8)
    lib().orc_quantize_q8_1(x, y, n_in, ncols)
    return y


def dequantize_q8_1(y: np.ndarray, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().orc_dequantize_q8_1(np.ascontiguousarray(y, dtype=np.uint8), out, n)
    return out


def q8_1_fields(y: np.ndarray):
    """Split Q8_1 bytes into (d fp16 bits, sum fp16 bits, int8 codes[nb, 32])."""
    blk = np.asarray(y, dtype=np.uint8).reshape(-1, Q8_1_BYTES)
    ds = blk[:, :4].copy().view(np.uint16)
    return ds[:, 0].copy(), ds[:, 1].copy(), blk[:, 4:].copy().view(np.int8)


# ---- Q6_K / Q8_0 --------------------------------------------------------------------------------------------------

def q6k_dequant(w: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    out = np.empty((n_out, n_in), dtype=np.float32)
    row = n_in // 256 * Q6K_BYTES
    for r in range(n_out):
        lib().orc_q6k_dequant_row(np.ascontiguousarray(w[r * row:(r + 1) * row]), out[r], n_in)
    return out


def q4k_dequant(w: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    """ggml dequantize_row_q4_K (token_embd of Q5_K_M files, qw:109-115) -> float32 [n_out * n_in]"""
    y = np.empty(n_out * n_in, np.float32)
    lib().orc_q4k_dequant_row(np.ascontiguousarray(w, np.uint8), y, n_out * n_in)
    return y


def q5k_dequant(w: np.ndarray, n_out: int, n_in: int) -> np.ndarray:
    """ggml dequantize_row_q5_K -> float32 [n_out * n_in]"""
    y = np.empty(n_out * n_in, np.float32)
    lib().orc_q5k_dequant_row(np.ascontiguousarray(w, np.uint8), y, n_out * n_in)
    return y


def q6k_block_dots(w, xq, n_in, n_out, lanes=False):
    out = np.empty((n_out, n_in // 32), dtype=np.int32)
    fn = lib().orc_q6k_block_dots_lanes if lanes else lib().orc_q6k_block_dots
    fn(np.ascontiguousarray(w), np.ascontiguousarray(xq), out, n_in, n_out)
    return out


def q8_0_block_dots(w, xq, n_in, n_out):
    out = np.empty((n_out, n_in // 32), dtype=np.int32)
    lib().orc_q8_0_block_dots(np.ascontiguousarray(w), np.ascontiguousarray(xq), out, n_in, n_out)
    return out


def _gemv(fn, w, xq, n_in, n_out, ncols, res, want_partials):
    y = np.empty(ncols * n_out, dtype=np.float64)
    np_ = (n_out + 3) // 4
    part = np.empty(ncols * np_, dtype=np.float64) if want_partials else None
    res_a = None if res is None else np.ascontiguousarray(res, dtype=np.float32).reshape(-1)
    fn(np.ascontiguousarray(w), np.ascontiguousarray(xq), _ptr(res_a), y, _ptr(part), n_in, n_out, ncols)
    return (y, part) if want_partials else y


def q6k_gemv(w, xq, n_in, n_out, ncols=1, res=None, partials=False):
    """fp64 y = W x (+ res), per column; partials = sum of squares of each 4-row group."""
    return _gemv(lib().orc_q6k_gemv, w, xq, n_in, n_out, ncols, res, partials)


def q4k_gemv(w, xq, n_in, n_out, ncols=1, res=None, partials=False):
    """Q4_K x Q8_1 GEMV (mmvq:562-640) in exact integers + fp64"""
    return _gemv(lib().orc_q4k_gemv, w, xq, n_in, n_out, ncols, res, partials)


def q5k_gemv(w, xq, n_in, n_out, ncols=1, res=None, partials=False):
    """Q5_K x Q8_1 GEMV (mmvq:185-300) in exact integers + fp64"""
    return _gemv(lib().orc_q5k_gemv, w, xq, n_in, n_out, ncols, res, partials)


def q8_0_gemv(w, xq, n_in, n_out, ncols=1, res=None, partials=False):
    return _gemv(lib().orc_q8_0_gemv, w, xq, n_in, n_out, ncols, res, partials)


def q6k_gemv_f32(w, xq, n_in, n_out, ncols=1, res=None, threads=1):
    y = np.empty(ncols * n_out, dtype=np.float32)
    part = np.empty(ncols * ((n_out + 3) // 4), dtype=np.float32)
    res_a = None if res is None else np.ascontiguousarray(res, dtype=np.float32).reshape(-1)
    lib().orc_q6k_gemv_f32_omp(w, xq, _ptr(res_a), y, _ptr(part), n_in, n_out, ncols, threads)
    return y, part


# ---- epilogues, GDN, attention -----------------------------------------------------------------------------------

def row_sum_partials(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty((x.size + 3) // 4, dtype=np.float64)
    lib().orc_row_sum_partials(x, out, x.size)
    return out


def rms_inv(partials, cols, eps):
    p = np.ascontiguousarray(partials, dtype=np.float64)
    return lib().orc_rms_inv(p, p.size, cols, eps)


def rms_norm_out(x, w, inv):
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.size, dtype=np.float64)
    lib().orc_rms_norm_out(x, np.ascontiguousarray(w, dtype=np.float32), inv, out, x.size)
    return out


def swiglu(up, gate):
    up = np.ascontiguousarray(up, dtype=np.float32)
    out = np.empty(up.size, dtype=np.float64)
    lib().orc_swiglu(up, np.ascontiguousarray(gate, dtype=np.float32), out, up.size)
    return out


def sig_mul(o, g):
    o = np.ascontiguousarray(o, dtype=np.float32)
    out = np.empty(o.size, dtype=np.float64)
    lib().orc_sig_mul(o, np.ascontiguousarray(g, dtype=np.float32), out, o.size)
    return out


def beta_gate(beta_in, alpha, dt, ssm_a):
    n = len(beta_in)
    b = np.empty(n, dtype=np.float64)
    g = np.empty(n, dtype=np.float64)
    f = lambda a: np.ascontiguousarray(a, dtype=np.float32)  # noqa: E731
    lib().orc_beta_gate(f(beta_in), f(alpha), f(dt), f(ssm_a), b, g, n)
    return b, g


def gdn_conv_l2(hist, x, w, qk_heads, eps):
    """Returns (h fp64, updated history); ``hist`` is not modified."""
    hist = np.array(hist, dtype=np.float32, copy=True).reshape(-1)
    x = np.ascontiguousarray(x, dtype=np.float32)
    h = np.empty(x.size, dtype=np.float64)
    lib().orc_gdn_conv_l2(hist, x, np.ascontiguousarray(w, dtype=np.float32), h, x.size, qk_heads, eps)
    return h, hist


def gdn_step_norm(state, q, k, v, gate, beta, z, gamma, eps, h_k, h_v):
    """Returns (y fp64, new state fp64); ``state`` is [128][h_v][128]."""
    st = np.array(state, dtype=np.float64, copy=True).reshape(-1)
    d = lambda a: np.ascontiguousarray(a, dtype=np.float64).reshape(-1)  # noqa: E731
    f = lambda a: np.ascontiguousarray(a, dtype=np.float32).reshape(-1)  # noqa: E731
    y = np.empty(h_v * 128, dtype=np.float64)
    lib().orc_gdn_step_norm(st, d(q), d(k), d(v), d(gate), d(beta), f(z), f(gamma), eps, y, h_k, h_v)
    return y, st


def gqa_decode(q, kc, vc, n_head, n_kv, hd, n_tok, scale):
    o = np.empty(n_head * hd, dtype=np.float64)
    lib().orc_gqa_decode(np.ascontiguousarray(q, dtype=np.float32).reshape(-1),
                         np.ascontiguousarray(kc, dtype=np.uint16).reshape(-1),
                         np.ascontiguousarray(vc, dtype=np.uint16).reshape(-1), o, n_head, n_kv, hd, n_tok, scale)
    return o


def rms_norm_heads(x, w, rows, cols, eps):
    out = np.empty(rows * cols, dtype=np.float64)
    lib().orc_rms_norm_heads(np.ascontiguousarray(x, dtype=np.float32).reshape(-1),
                             np.ascontiguousarray(w, dtype=np.float32), out, rows, cols, eps)
    return out


def rope_neox(x, heads, hd, n_rot, pos, theta):
    x = np.ascontiguousarray(x, dtype=np.float64).reshape(-1)
    out = np.empty_like(x)
    lib().orc_rope_neox(x, out, heads, hd, n_rot, pos, theta)
    return out


def rope_yarn(x, heads, hd, n_rot, pos, base, factor, orig_ctx, ext_factor=1.0, attn_factor=1.0, beta_fast=32.0,
              beta_slow=1.0):
    """YaRN NEOX RoPE with the reference's parameters (qw:1991-1999) -> float64"""
    out = np.empty(heads * hd, np.float64)
    lib().orc_rope_yarn(np.ascontiguousarray(x, np.float64), out, heads, hd, n_rot, pos, base, factor, orig_ctx,
                        ext_factor, attn_factor, beta_fast, beta_slow)
    return out


def argmax(l):
    l = np.ascontiguousarray(l, dtype=np.float32)
    return lib().orc_argmax(l, l.size)


def topk(l, k):
    """topk_out (qw:2513-2531) restated in C: [(id, logit)] of the k largest logits, descending"""
    l = np.ascontiguousarray(l, dtype=np.float32)
    ids = np.zeros(k, np.int32)
    vals = np.zeros(k, np.float32)
    m = lib().orc_topk(l, l.size, k, ids, vals)
    return list(zip(ids[:m].tolist(), vals[:m].tolist()))


def topk_sorted(l, k):
    """the same list by a full sort: logit descending, then id ascending (-0 equal to +0)"""
    l = np.asarray(l, dtype=np.float32)
    order = np.lexsort((np.arange(l.size), -(l.astype(np.float64) + 0.0)))[:k]
    return [(int(i), float(l[i])) for i in order]


# ---- the CPU baseline's SIMD timing build (cpu_round.c) --------------------------------------------------------------
_CPR_PATH = os.path.join(_HERE, "libcpu_round.so")
_cpr = None
_CPR_SIGS = {
    "cpr_simd_level": (_c.c_int, []),
    "cpr_q6k_gemv": (None, [_u8p, _u8p, _c.c_void_p, _f32p, _c.c_void_p, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                            _c.c_int]),
    "cpr_gdn_layer": (None, [_f32p, _c.c_int, _f32p, _f32p, _f32p, _f32p, _f32p, _c.c_float, _f32p, _f32p, _f32p,
                             _c.c_int, _c.c_int, _c.c_int, _c.c_int]),
    "cpr_gqa_decode": (None, [_f32p, _u16p, _u16p, _f32p, _c.c_int, _c.c_int, _c.c_int, _c.c_int, _c.c_int,
                              _c.c_float, _c.c_int]),
}


def cpr():
    """the timing build (libcpu_round.so): the reported CPU baseline's kernels, checked against the oracle"""
    global _cpr
    if _cpr is None:
        if not os.path.exists(_CPR_PATH):
            subprocess.run(["make", "-s", "libcpu_round.so"], cwd=_HERE, check=True)
        _cpr = ctypes.CDLL(_CPR_PATH)
        for name, (res, args) in _CPR_SIGS.items():
            fn = getattr(_cpr, name)
            fn.restype = res
            fn.argtypes = args
    return _cpr


def cpr_q6k_gemv(w, xq, n_in, n_out, ncols=1, res=None, partials=False, threads=1, simd=2):
    """timing-build Q6_K x Q8_1 GEMV (fp32): y, and the 4-row partials when res and partials"""
    y = np.empty(ncols * n_out, np.float32)
    part = np.empty(ncols * ((n_out + 3) // 4), np.float32) if (partials and res is not None) else None
    res_a = None if res is None else np.ascontiguousarray(res, dtype=np.float32).reshape(-1)
    cpr().cpr_q6k_gemv(w, xq, _ptr(res_a), y, _ptr(part), n_in, n_out, ncols, threads, simd)
    return (y, part) if part is not None else y


def cpr_gdn_layer(qkvz, stride, ab, conv_w, dt, ssm_a, gamma, eps, hist, state, h_k, h_v, ntok, threads=1):
    """timing-build GDN layer for ntok tokens: returns (y, new history, new state); inputs are not modified"""
    f = lambda a: np.ascontiguousarray(a, dtype=np.float32).reshape(-1)  # noqa: E731
    hist, state = f(hist).copy(), f(state).copy()
    y = np.empty(ntok * h_v * 128, np.float32)
    cpr().cpr_gdn_layer(f(qkvz), stride, f(ab), f(conv_w), f(dt), f(ssm_a), f(gamma), eps, hist, state, y, h_k, h_v,
                        ntok, threads)
    return y, hist, state


def cpr_gqa_decode(q, kc, vc, n_head, n_kv, hd, pos0, ntok, scale, threads=1):
    o = np.empty(ntok * n_head * hd, np.float32)
    cpr().cpr_gqa_decode(np.ascontiguousarray(q, np.float32).reshape(-1), np.ascontiguousarray(kc, np.uint16),
                         np.ascontiguousarray(vc, np.uint16), o, n_head, n_kv, hd, pos0, ntok, scale, threads)
    return o
