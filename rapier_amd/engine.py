"""Host mirror of the decode engine (include/rapier_mi_engine.h): the reference's qwythos Engine with its
forward_token / draft_predict / launch_token_verify loop, driven through the C ABI.

Greedy decoding and the exact-verify MTP rounds both run as one hipGraph launch per token / round; this module only
moves token ids in and out.
"""
from __future__ import annotations

import ctypes

from . import _call, _stream, last_error, lib

GREEDY, MTP, MTP_FORCED = 0, 1, 2
BUF_GDN_STATE, BUF_GDN_HIST, BUF_K_CACHE, BUF_V_CACHE, BUF_HIDDEN = 0, 1, 2, 3, 4


class ModelConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_embd", "n_ff", "n_vocab", "n_layer", "ssm_h_k", "ssm_h_v", "n_head",
                                            "n_kv", "head_dim", "n_rot")] + \
               [("rope_theta", ctypes.c_float), ("eps", ctypes.c_float)]


class EngineInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in ("trunk_weight_bytes", "lm_head_bytes", "draft_block_bytes",
                                               "round_weight_bytes", "token_weight_bytes", "kv_bytes_per_pos")] + \
               [(n, ctypes.c_int) for n in ("gdn_layers", "attn_layers", "max_ctx", "attn_chunk")]


class GenRequest(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int), ("n_gen", ctypes.c_int), ("use_graph", ctypes.c_int),
                ("ref_tokens", ctypes.POINTER(ctypes.c_int)), ("ref_base", ctypes.c_int), ("ref_len", ctypes.c_int),
                ("pattern", ctypes.POINTER(ctypes.c_uint8)), ("pattern_len", ctypes.c_int)]


class GenStats(ctypes.Structure):
    _fields_ = [("tokens", ctypes.c_int), ("emitted", ctypes.c_int), ("rounds", ctypes.c_int),
                ("accepted", ctypes.c_int), ("gpu_ms", ctypes.c_float)]

    def as_dict(self):
        return {k: getattr(self, k) for k, _ in self._fields_}


_bound = False


def _bind():
    global _bound
    if _bound:
        return
    L = lib()
    P = ctypes.POINTER
    sig = {
        "rmi_qwen35_9b_config": (ModelConfig, []),
        "rmi_engine_create": (ctypes.c_int, [P(ModelConfig), ctypes.c_uint64, ctypes.c_int, ctypes.c_void_p,
                                             P(ctypes.c_void_p)]),
        "rmi_engine_destroy": (ctypes.c_int, [ctypes.c_void_p]),
        "rmi_engine_info": (ctypes.c_int, [ctypes.c_void_p, P(EngineInfo)]),
        "rmi_engine_prefill": (ctypes.c_int, [ctypes.c_void_p, P(ctypes.c_int), ctypes.c_int, P(ctypes.c_int)]),
        "rmi_engine_prefill_batch": (ctypes.c_int, [ctypes.c_void_p, P(ctypes.c_int), ctypes.c_int, ctypes.c_int,
                                                    P(ctypes.c_int)]),
        "rmi_engine_read": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_size_t,
                                           ctypes.c_void_p, ctypes.c_size_t]),
        "rmi_engine_synth_context": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_int,
                                                    P(ctypes.c_int)]),
        "rmi_engine_save_state": (ctypes.c_int, [ctypes.c_void_p]),
        "rmi_engine_restore_state": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]),
        "rmi_engine_state": (ctypes.c_int, [ctypes.c_void_p, P(ctypes.c_int), P(ctypes.c_int)]),
        "rmi_engine_generate": (ctypes.c_int, [ctypes.c_void_p, P(GenRequest), P(ctypes.c_int), P(GenStats)]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _bound = True


def qwen35_9b_config() -> ModelConfig:
    _bind()
    return lib().rmi_qwen35_9b_config()


def small_config(**kw) -> ModelConfig:
    """A small member of the same hybrid family (3 GDN + 1 attention layers) for tests."""
    c = ModelConfig(n_embd=2048, n_ff=4096, n_vocab=5000, n_layer=4, ssm_h_k=4, ssm_h_v=8, n_head=8, n_kv=2,
                    head_dim=256, n_rot=64, rope_theta=1e7, eps=1e-6)
    for k, v in kw.items():
        setattr(c, k, v)
    return c


class Engine:
    def __init__(self, cfg: ModelConfig, seed: int = 1234, max_ctx: int = 4096, stream=None):
        _bind()
        self.cfg = cfg
        h = ctypes.c_void_p()
        _call("rmi_engine_create", ctypes.byref(cfg), seed, max_ctx, _stream(stream), ctypes.byref(h))
        self._h = h

    def close(self):
        if self._h:
            lib().rmi_engine_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def info(self) -> dict:
        i = EngineInfo()
        _call("rmi_engine_info", self._h, ctypes.byref(i))
        return {k: getattr(i, k) for k, _ in i._fields_}

    def prefill(self, tokens, batch: int = 16) -> int:
        """Ingest the prompt from position 0; batch 1 is the token-by-token path, 2..16 the chunked one."""
        arr = (ctypes.c_int * len(tokens))(*tokens)
        first = ctypes.c_int()
        _call("rmi_engine_prefill_batch", self._h, arr, len(tokens), batch, ctypes.byref(first))
        return first.value

    def read(self, which: int, layer: int, nbytes: int, offset: int = 0):
        """bytes [offset, offset + nbytes) of an engine buffer (BUF_*) as a uint8 numpy array"""
        import numpy as np
        out = np.empty(nbytes, np.uint8)
        _call("rmi_engine_read", self._h, which, layer, offset, out.ctypes.data_as(ctypes.c_void_p), nbytes)
        return out

    def synth_context(self, n_ctx: int, seed: int, last_token: int) -> int:
        first = ctypes.c_int()
        _call("rmi_engine_synth_context", self._h, n_ctx, seed, last_token, ctypes.byref(first))
        return first.value

    def save_state(self):
        _call("rmi_engine_save_state", self._h)

    def restore_state(self, pos: int, cur: int):
        _call("rmi_engine_restore_state", self._h, pos, cur)

    def state(self):
        p, t = ctypes.c_int(), ctypes.c_int()
        _call("rmi_engine_state", self._h, ctypes.byref(p), ctypes.byref(t))
        return p.value, t.value

    def generate(self, n_gen: int, mode: int = GREEDY, ref_tokens=None, ref_base: int = 0, pattern=None,
                 use_graph: bool = True):
        req = GenRequest(mode=mode, n_gen=n_gen, use_graph=1 if use_graph else 0)
        keep = []
        if ref_tokens is not None:
            ra = (ctypes.c_int * len(ref_tokens))(*ref_tokens)
            keep.append(ra)
            req.ref_tokens = ra
            req.ref_base = ref_base
            req.ref_len = len(ref_tokens)
        if pattern is not None:
            pa = (ctypes.c_uint8 * len(pattern))(*pattern)
            keep.append(pa)
            req.pattern = pa
            req.pattern_len = len(pattern)
        out = (ctypes.c_int * n_gen)()
        st = GenStats()
        _call("rmi_engine_generate", self._h, ctypes.byref(req), out, ctypes.byref(st))
        return list(out), st.as_dict()


__all__ = ["Engine", "ModelConfig", "qwen35_9b_config", "small_config", "GREEDY", "MTP", "MTP_FORCED", "last_error"]
