"""Host mirror of the decode engine (include/rapier_mi_engine.h): the reference's qwythos Engine with its
forward_token / draft_predict / launch_token_verify loop, driven through the C ABI.

Greedy decoding and the exact-verify MTP rounds both run as one hipGraph launch per token / round; this module only
moves token ids in and out.
"""
from __future__ import annotations

import ctypes
import os

from . import _call, _stream, last_error, lib

GREEDY, MTP, MTP_FORCED = 0, 1, 2
BUF_GDN_STATE, BUF_GDN_HIST, BUF_K_CACHE, BUF_V_CACHE, BUF_HIDDEN, BUF_LOGITS, BUF_ROUND = 0, 1, 2, 3, 4, 5, 6


class ModelConfig(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in ("n_embd", "n_ff", "n_vocab", "n_layer", "ssm_h_k", "ssm_h_v", "n_head",
                                            "n_kv", "head_dim", "n_rot")] + \
               [("rope_theta", ctypes.c_float), ("eps", ctypes.c_float), ("rope_factor", ctypes.c_float),
                ("rope_orig_ctx", ctypes.c_float)]


class EngineInfo(ctypes.Structure):
    _fields_ = [(n, ctypes.c_size_t) for n in ("trunk_weight_bytes", "lm_head_bytes", "draft_block_bytes",
                                               "round_weight_bytes", "token_weight_bytes", "kv_bytes_per_pos")] + \
               [(n, ctypes.c_int) for n in ("gdn_layers", "attn_layers", "max_ctx", "attn_chunk")]


class GenRequest(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int), ("n_gen", ctypes.c_int), ("use_graph", ctypes.c_int),
                ("ref_tokens", ctypes.POINTER(ctypes.c_int)), ("ref_base", ctypes.c_int), ("ref_len", ctypes.c_int),
                ("pattern", ctypes.POINTER(ctypes.c_uint8)), ("pattern_len", ctypes.c_int)]


class ServeOptions(ctypes.Structure):
    _fields_ = [("eos", ctypes.c_int), ("batch", ctypes.c_int), ("topk", ctypes.c_int)]


_CB = ctypes.CFUNCTYPE
SERVE_RESET = _CB(ctypes.c_int, ctypes.c_void_p)
SERVE_INGEST = _CB(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int), ctypes.c_int, ctypes.c_int,
                   ctypes.POINTER(ctypes.c_int))
SERVE_TOPK = _CB(ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(ctypes.c_int),
                 ctypes.POINTER(ctypes.c_float))
SERVE_GEN_BEGIN = _CB(ctypes.c_int, ctypes.c_void_p, ctypes.c_int)
SERVE_GEN_STEP = _CB(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int))
SERVE_POSITION = _CB(ctypes.c_int, ctypes.c_void_p, ctypes.POINTER(ctypes.c_int))
SERVE_ERROR = _CB(ctypes.c_void_p, ctypes.c_void_p)   # returns a char* the backend keeps alive


class ServeBackend(ctypes.Structure):
    _fields_ = [("user", ctypes.c_void_p), ("max_ctx", ctypes.c_int), ("reset", SERVE_RESET),
                ("ingest", SERVE_INGEST), ("topk", SERVE_TOPK), ("gen_begin", SERVE_GEN_BEGIN),
                ("gen_step", SERVE_GEN_STEP), ("position", SERVE_POSITION), ("error", SERVE_ERROR)]


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
        "rmi_engine_create_gguf": (ctypes.c_int, [ctypes.c_char_p, ctypes.c_int, ctypes.c_void_p, P(ctypes.c_void_p)]),
        "rmi_engine_config": (ctypes.c_int, [ctypes.c_void_p, P(ModelConfig)]),
        "rmi_gguf_open": (ctypes.c_int, [ctypes.c_char_p, P(ctypes.c_void_p)]),
        "rmi_gguf_close": (None, [ctypes.c_void_p]),
        "rmi_gguf_tensor_count": (ctypes.c_int64, [ctypes.c_void_p]),
        "rmi_gguf_find": (ctypes.c_int64, [ctypes.c_void_p, ctypes.c_char_p]),
        "rmi_gguf_tensor_info": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int64, P(ctypes.c_char_p), P(ctypes.c_int),
                                                P(ctypes.c_int), P(ctypes.c_int64), P(ctypes.c_size_t),
                                                P(ctypes.c_void_p)]),
        "rmi_gguf_get_num": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, P(ctypes.c_double)]),
        "rmi_gguf_get_str": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, P(ctypes.c_char_p)]),
        "rmi_gguf_array_len": (ctypes.c_int64, [ctypes.c_void_p, ctypes.c_char_p]),
        "rmi_gguf_array_str": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int64, P(ctypes.c_char_p)]),
        "rmi_gguf_array_num": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int64, P(ctypes.c_double)]),
        "rmi_engine_synth_context": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_uint64, ctypes.c_int,
                                                    P(ctypes.c_int)]),
        "rmi_engine_save_state": (ctypes.c_int, [ctypes.c_void_p]),
        "rmi_engine_restore_state": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int]),
        "rmi_engine_state": (ctypes.c_int, [ctypes.c_void_p, P(ctypes.c_int), P(ctypes.c_int)]),
        "rmi_engine_generate": (ctypes.c_int, [ctypes.c_void_p, P(GenRequest), P(ctypes.c_int), P(GenStats)]),
        "rmi_engine_reset": (ctypes.c_int, [ctypes.c_void_p]),
        "rmi_engine_ingest": (ctypes.c_int, [ctypes.c_void_p, P(ctypes.c_int), ctypes.c_int, ctypes.c_int,
                                             P(ctypes.c_int)]),
        "rmi_engine_gen_begin": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int]),
        "rmi_engine_gen_step": (ctypes.c_int, [ctypes.c_void_p, P(ctypes.c_int), P(ctypes.c_int)]),
        "rmi_engine_topk": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, P(ctypes.c_int),
                                           P(ctypes.c_float)]),
        "rmi_serve_default_options": (ServeOptions, []),
        "rmi_serve_fd": (ctypes.c_int, [P(ServeBackend), P(ServeOptions), ctypes.c_int, ctypes.c_int]),
        "rmi_serve_engine": (ctypes.c_int, [ctypes.c_void_p, P(ServeOptions), ctypes.c_int, ctypes.c_int]),
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


class GgufFile:
    """A memory-mapped GGUF file (the engine's reader, rmi_gguf_*): metadata and tensor table."""

    def __init__(self, path: str):
        _bind()
        h = ctypes.c_void_p()
        _call("rmi_gguf_open", os.fsencode(path), ctypes.byref(h))
        self._h = h

    def close(self):
        if self._h:
            lib().rmi_gguf_close(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self):
        return lib().rmi_gguf_tensor_count(self._h)

    def find(self, name: str) -> int:
        return lib().rmi_gguf_find(self._h, name.encode())

    def tensor(self, i: int):
        """(name, ggml type, dims tuple, data bytes as a uint8 array or None)"""
        import numpy as np
        name, t, nd = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
        dims, nbytes, data = (ctypes.c_int64 * 4)(), ctypes.c_size_t(), ctypes.c_void_p()
        _call("rmi_gguf_tensor_info", self._h, i, ctypes.byref(name), ctypes.byref(t), ctypes.byref(nd), dims,
              ctypes.byref(nbytes), ctypes.byref(data))
        arr = None
        if data.value:
            arr = np.ctypeslib.as_array((ctypes.c_uint8 * nbytes.value).from_address(data.value)).copy()
        return name.value.decode(), t.value, tuple(dims[:nd.value]), arr

    def num(self, key: str):
        v = ctypes.c_double()
        return v.value if lib().rmi_gguf_get_num(self._h, key.encode(), ctypes.byref(v)) == 0 else None

    def str(self, key: str):
        v = ctypes.c_char_p()
        return v.value.decode() if lib().rmi_gguf_get_str(self._h, key.encode(), ctypes.byref(v)) == 0 else None

    def array(self, key: str):
        n = lib().rmi_gguf_array_len(self._h, key.encode())
        if n < 0:
            return None
        out = []
        for i in range(n):
            sv, dv = ctypes.c_char_p(), ctypes.c_double()
            if lib().rmi_gguf_array_str(self._h, key.encode(), i, ctypes.byref(sv)) == 0:
                out.append(sv.value.decode())
            else:
                _call("rmi_gguf_array_num", self._h, key.encode(), i, ctypes.byref(dv))
                out.append(dv.value)
        return out


class Engine:
    def __init__(self, cfg: ModelConfig, seed: int = 1234, max_ctx: int = 4096, stream=None, _handle=None):
        _bind()
        if _handle is not None:
            self._h = _handle
            c = ModelConfig()
            _call("rmi_engine_config", self._h, ctypes.byref(c))
            self.cfg = c
            return
        self.cfg = cfg
        h = ctypes.c_void_p()
        _call("rmi_engine_create", ctypes.byref(cfg), seed, max_ctx, _stream(stream), ctypes.byref(h))
        self._h = h

    @classmethod
    def from_gguf(cls, path: str, max_ctx: int = 4096, stream=None) -> "Engine":
        """a qwen35 GGUF (load_model, qw:1978-2134)"""
        _bind()
        h = ctypes.c_void_p()
        _call("rmi_engine_create_gguf", os.fsencode(path), max_ctx, _stream(stream), ctypes.byref(h))
        return cls(None, _handle=h)

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

    def reset(self):
        """empty context at position 0"""
        _call("rmi_engine_reset", self._h)

    def ingest(self, tokens, batch: int = 16) -> int:
        """feed tokens at the current position; returns the greedy token after them"""
        arr = (ctypes.c_int * len(tokens))(*tokens)
        first = ctypes.c_int()
        _call("rmi_engine_ingest", self._h, arr, len(tokens), batch, ctypes.byref(first))
        return first.value

    def gen_begin(self, mode: int = GREEDY):
        _call("rmi_engine_gen_begin", self._h, mode)

    def gen_step(self):
        """one greedy forward ([next]) or one verify round ([c0] or [c0, c1])"""
        out = (ctypes.c_int * 2)()
        n = ctypes.c_int()
        _call("rmi_engine_gen_step", self._h, out, ctypes.byref(n))
        return list(out)[:n.value]

    def topk(self, k: int = 40, col: int = 0):
        """[(id, logit)] of the k largest logits of the last head pass, logit descending, lower id first on ties"""
        ids = (ctypes.c_int * k)()
        vals = (ctypes.c_float * k)()
        _call("rmi_engine_topk", self._h, col, k, ids, vals)
        return list(zip(list(ids), list(vals)))

    def serve_fd(self, in_fd: int, out_fd: int, eos: int = 248046, batch: int = 16, topk: int = 40):
        """the --serve protocol over two file descriptors (rmi_serve_engine), until end of input"""
        o = ServeOptions(eos=eos, batch=batch, topk=topk)
        _call("rmi_serve_engine", self._h, ctypes.byref(o), in_fd, out_fd)

    def read(self, which: int, layer: int, nbytes: int, offset: int = 0):
        """bytes [offset, offset + nbytes) of an engine buffer (BUF_*) as a uint8 numpy array"""
        import numpy as np
        out = np.empty(nbytes, np.uint8)
        _call("rmi_engine_read", self._h, which, layer, offset, out.ctypes.data_as(ctypes.c_void_p), nbytes)
        return out

    def round_slots(self) -> dict:
        """the round's token slots (BUF_ROUND): position, current token, candidate, verify / draft argmaxes, accept"""
        v = self.read(BUF_ROUND, 0, 32).view("<i4")
        keys = ("pos", "cur", "cand", "v0", "v1", "c0", "c1", "accept")
        return {k: int(x) for k, x in zip(keys, v)}

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


def serve_fd(backend: ServeBackend, in_fd: int, out_fd: int, eos: int = 248046, batch: int = 16, topk: int = 40):
    """the --serve protocol loop over any backend (rmi_serve_fd); returns its status code"""
    _bind()
    o = ServeOptions(eos=eos, batch=batch, topk=topk)
    return lib().rmi_serve_fd(ctypes.byref(backend), ctypes.byref(o), in_fd, out_fd)


__all__ = ["Engine", "ModelConfig", "qwen35_9b_config", "small_config", "GREEDY", "MTP", "MTP_FORCED", "last_error"]
