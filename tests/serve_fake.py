"""A deterministic stand-in for the engine behind the serve protocol, for CPU tests of rmi_serve_fd against the
oracle's restated serve loop (oracle/serve.py).  Test data only.

The "model": the greedy token after a context is a hash of it (the end-of-sequence id every few positions), its
logits a seeded vector with many equal values and the greedy token on top; a verify round accepts the draft by a
hash of the position.  Both the C loop (through rmi_serve_backend callbacks) and the oracle loop drive one instance
each, so their lines must agree exactly.
"""
from __future__ import annotations

import ctypes

import numpy as np

import oracle

RMI_OK, RMI_ERR_LAUNCH, RMI_ERR_STATE = 0, 4, 6


class FakeModel:
    def __init__(self, vocab: int = 300, max_ctx: int = 400, eos: int = 7, seed: int = 0, fail_at=None):
        self.V, self.max_ctx, self.eos, self.seed = vocab, max_ctx, eos, seed
        self.ctx: list = []
        self.cur = 0
        self.mode = -1
        self.err = b""
        self.fail_at = fail_at          # (call name, n-th call) that reports a device failure
        self.calls: dict = {}

    # ---- the model ----
    def _h(self, ctx) -> int:
        h = 1469598103934665603 ^ self.seed
        for t in ctx:
            h = ((h ^ (t & 0xffffffff)) * 1099511628211) & 0xffffffffffffffff
        return h

    def next_token(self, ctx) -> int:
        if len(ctx) % 9 == 5:
            return self.eos
        return int(self._h(ctx) % self.V)

    def logits(self, ctx):
        rng = np.random.default_rng(self._h(ctx) & 0xffffffff)
        l = (rng.integers(-40, 40, self.V) / 8.0).astype(np.float32)
        l[self.next_token(ctx)] = np.float32(6.0)
        return l

    def accepts(self) -> bool:
        return (self._h([len(self.ctx), 99]) >> 7) % 2 == 0

    # ---- the oracle's engine interface ----
    def reset(self):
        self.ctx, self.cur = [], 0

    def position(self) -> int:
        return len(self.ctx)

    def ingest(self, tokens) -> int:
        self.ctx += list(tokens)
        self.cur = self.next_token(self.ctx)
        return self.cur

    def top(self, k):
        return oracle.topk(self.logits(self.ctx), k)

    def greedy_step(self) -> int:
        self.ctx.append(self.cur)
        self.cur = self.next_token(self.ctx)
        return self.cur

    def mtp_begin(self):
        pass

    def mtp_round(self):
        c0 = self.next_token(self.ctx + [self.cur])
        if self.accepts():                        # the candidate was c0: both columns stand
            self.ctx += [self.cur, c0]
            c1 = self.next_token(self.ctx)
            self.cur = c1
            return c0, c1, True
        self.ctx.append(self.cur)                 # rejected: column 0 stands
        self.cur = c0
        return c0, (c0 + 1) % self.V, False

    # ---- rmi_serve_backend callbacks ----
    def _tick(self, name) -> bool:
        self.calls[name] = self.calls.get(name, 0) + 1
        if self.fail_at and self.fail_at == (name, self.calls[name]):
            self.err = b"fake device failure"
            return True
        return False

    def backend(self):
        from rapier_amd import engine as E
        m = self

        def reset(_u):
            if m._tick("reset"):
                return RMI_ERR_LAUNCH
            m.reset()
            m.mode = -1
            return RMI_OK

        def ingest(_u, toks, n, batch, first):
            if m._tick("ingest"):
                return RMI_ERR_LAUNCH
            t = [toks[i] for i in range(n)]
            if any(x < 0 or x >= m.V for x in t):
                m.err = b"rmi_engine_ingest: bad token id"
                return RMI_ERR_STATE
            first[0] = m.ingest(t)
            m.mode = -1
            return RMI_OK

        def topk(_u, k, ids, vals):
            if m._tick("topk"):
                return RMI_ERR_LAUNCH
            for i, (a, b) in enumerate(m.top(k)):
                ids[i], vals[i] = a, b
            return RMI_OK

        def gen_begin(_u, mode):
            if m._tick("gen_begin"):
                return RMI_ERR_LAUNCH
            m.mode = mode
            return RMI_OK

        def gen_step(_u, out, n):
            if m._tick("gen_step"):
                return RMI_ERR_LAUNCH
            if m.mode == 0:
                out[0], n[0] = m.greedy_step(), 1
            elif m.mode == 1:
                c0, c1, acc = m.mtp_round()
                out[0], n[0] = c0, 1
                if acc:
                    out[1], n[0] = c1, 2
            else:
                m.err = b"gen_step before gen_begin"
                return RMI_ERR_STATE
            return RMI_OK

        def position(_u, p):
            p[0] = m.position()
            return RMI_OK

        def error(_u):
            m._errbuf = ctypes.create_string_buffer(m.err)      # kept alive until the next failure
            return ctypes.addressof(m._errbuf)

        cbs = [E.SERVE_RESET(reset), E.SERVE_INGEST(ingest), E.SERVE_TOPK(topk), E.SERVE_GEN_BEGIN(gen_begin),
               E.SERVE_GEN_STEP(gen_step), E.SERVE_POSITION(position), E.SERVE_ERROR(error)]
        b = E.ServeBackend(None, m.max_ctx, *cbs)
        b._keep = cbs                             # the callbacks must outlive the call
        return b


def run_c_loop(model: FakeModel, lines, eos: int, topk: int = 40, batch: int = 16, tmp_path=None):
    """the C loop over model: request lines in, (status, response lines) out"""
    import os
    import tempfile

    from rapier_amd import engine as E
    d = tmp_path or tempfile.mkdtemp()
    src, dst = os.path.join(d, "req.jsonl"), os.path.join(d, "resp.jsonl")
    with open(src, "w") as f:
        f.write("".join(ln + "\n" for ln in lines))
    fi, fo = os.open(src, os.O_RDONLY), os.open(dst, os.O_WRONLY | os.O_CREAT | os.O_TRUNC)
    try:
        rc = E.serve_fd(model.backend(), fi, fo, eos=eos, batch=batch, topk=topk)
    finally:
        os.close(fi)
        os.close(fo)
    with open(dst) as f:
        return rc, f.read().splitlines()

