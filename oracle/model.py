"""CPU oracle of the qwen35 engine: the reference's forward_token (src/qwythos.cpp:1773-1824) and draft_predict
(qw:1316-1406) composed from the oracle's pinned pieces, on the tensors of a qwen35 GGUF.

TEST INFRASTRUCTURE ONLY (the checker for rmi_engine_create_gguf and the engine's composition).  Every matrix is
applied separately (no concatenation), activations are quantized to Q8_1 where the reference quantizes them, and
every value the engine stores as fp32 (or fp16 in the KV cache) is rounded to it here, so the two differ only by
fp32-vs-fp64 arithmetic inside the ops.

Per trunk layer (qw:1438-1588 per column):
  GDN:        Q8_1(rms(x) * attn_norm) -> qkv, z, beta, alpha GEMVs -> beta_gate -> conv + SiLU + L2 -> delta-rule step
              + RMSNorm * SiLU(z) -> Q8_1 -> ssm_out GEMV + x
  attention:  Q8_1(rms(x) * attn_norm) -> q|gate, k, v GEMVs -> per-head RMSNorm (q_norm, k_norm), NEOX / YaRN RoPE ->
              fp16 K/V at pos -> softmax(q k^T / 16) v over 0..pos -> * sigmoid(gate) -> Q8_1 -> attn_output GEMV + x
  FFN:        Q8_1(rms(x) * post_attention_norm) -> up, gate GEMVs -> SiLU(gate) * up -> Q8_1 -> down GEMV + x
Head: Q8_1(rms(x) * output_norm) -> output GEMV (logits); hidden = rms(x) * output_norm (the draft's input).
Draft at position pos for token t with the previous hidden h: [enorm(emb t) | hnorm(h)] -> Q8_1 -> eh_proj -> one
attention layer + FFN (blk.<n_layer>) -> Q8_1(rms * shared_head_norm) -> output GEMV.
"""
from __future__ import annotations

import numpy as np

import oracle as orc

S = 128


def f32(a):
    return np.asarray(a, dtype=np.float64).astype(np.float32)


class Qwen35:
    """tensors: name -> (ggml type, dims, uint8 bytes or float32 array) as in the GGUF; config from the shapes."""

    def __init__(self, tensors: dict, n_layer: int, eps: float = 1e-6, rope_base: float = 1e7, n_rot: int = 64,
                 rope_factor: float = 1.0, rope_orig_ctx: float = 262144.0, max_ctx: int = 512):
        self.t = tensors
        self.n_layer = n_layer
        self.eps, self.base, self.n_rot = eps, rope_base, n_rot
        self.factor, self.orig = rope_factor, rope_orig_ctx
        emb = tensors["token_embd.weight"]
        self.emb_type, (self.n_embd, self.n_vocab) = emb[0], emb[1]
        self.attn = [f"blk.{il}.attn_q.weight" in tensors for il in range(n_layer)]
        a = next(il for il in range(n_layer + 1) if f"blk.{il}.attn_q.weight" in tensors)
        self.hd = tensors[f"blk.{a}.attn_q_norm.weight"][1][0]
        self.n_head = tensors[f"blk.{a}.attn_q.weight"][1][1] // (2 * self.hd)
        self.n_kv = tensors[f"blk.{a}.attn_k.weight"][1][1] // self.hd
        g = next((il for il in range(n_layer) if not self.attn[il]), None)
        if g is not None:
            self.h_v = tensors[f"blk.{g}.ssm_a"][1][0]
            self.h_k = (tensors[f"blk.{g}.attn_qkv.weight"][1][1] - S * self.h_v) // (2 * S)
        self.max_ctx = max_ctx
        self.reset()

    def reset(self):
        self.state = {il: np.zeros(S * self.h_v * S) for il in range(self.n_layer) if not self.attn[il]}
        ch = (2 * self.h_k + self.h_v) * S if self.state else 0
        self.hist = {il: np.zeros(3 * ch, np.float32) for il in self.state}
        kv = self.max_ctx * self.n_kv * self.hd
        self.kc = {il: np.zeros(kv, np.uint16) for il in list(range(self.n_layer)) + [self.n_layer]
                   if il == self.n_layer or self.attn[il]}
        self.vc = {il: np.zeros(kv, np.uint16) for il in self.kc}

    # ---- pieces ----
    def w(self, name):
        return self.t[name]

    def gemv(self, name, xq, res=None):
        tp, dims, data = self.t[name]
        fn = {14: orc.q6k_gemv, 13: orc.q5k_gemv, 12: orc.q4k_gemv, 8: orc.q8_0_gemv}[tp]
        y = fn(data, xq, dims[0], dims[1])
        return f32(y if res is None else y + res)

    def embed(self, tok):
        tp, dims, data = self.t["token_embd.weight"]
        row = {14: orc.Q6K_BYTES, 13: orc.Q5K_BYTES, 12: orc.Q4K_BYTES}[tp] * (dims[0] // 256)
        r = data[tok * row:(tok + 1) * row]
        if tp == 14:
            return orc.q6k_dequant(r, 1, dims[0]).reshape(-1)
        return (orc.q5k_dequant if tp == 13 else orc.q4k_dequant)(r, 1, dims[0])

    def rms_q8(self, x, wname):
        """rms_quant_apply (qw:627-655): Q8_1 of x * w * rsqrt(mean(x^2) + eps), partials of 4 in order"""
        inv = orc.rms_inv(orc.row_sum_partials(x), x.size, self.eps)
        return orc.quantize_q8_1(f32(orc.rms_norm_out(x, self.t[wname][2], inv)), x.size)

    def rope(self, x, heads, pos):
        if self.factor > 1.0:
            return orc.rope_yarn(x, heads, self.hd, self.n_rot, pos, self.base, self.factor, self.orig)
        return orc.rope_neox(x, heads, self.hd, self.n_rot, pos, self.base)

    def attention(self, il, x, pos):
        p = f"blk.{il}."
        xq = self.rms_q8(x, p + "attn_norm.weight")
        qg, k, v = self.gemv(p + "attn_q.weight", xq), self.gemv(p + "attn_k.weight", xq), self.gemv(p + "attn_v.weight", xq)
        hd, nh, nkv = self.hd, self.n_head, self.n_kv
        qg = qg.reshape(nh, 2, hd)
        q = f32(self.rope(orc.rms_norm_heads(qg[:, 0].reshape(-1), self.t[p + "attn_q_norm.weight"][2], nh, hd, self.eps),
                          nh, pos))
        kr = self.rope(orc.rms_norm_heads(k, self.t[p + "attn_k_norm.weight"][2], nkv, hd, self.eps), nkv, pos)
        row = slice(pos * nkv * hd, (pos + 1) * nkv * hd)
        self.kc[il][row] = kr.astype(np.float32).astype(np.float16).view(np.uint16)
        self.vc[il][row] = v.astype(np.float16).view(np.uint16)
        o = orc.gqa_decode(q, self.kc[il], self.vc[il], nh, nkv, hd, pos + 1, 1.0 / np.sqrt(hd))
        y = f32(orc.sig_mul(f32(o), qg[:, 1].reshape(-1)))
        return self.gemv(p + "attn_output.weight", orc.quantize_q8_1(y, y.size), res=x)

    def gdn(self, il, x):
        p = f"blk.{il}."
        xq = self.rms_q8(x, p + "attn_norm.weight")
        qkv, z = self.gemv(p + "attn_qkv.weight", xq), self.gemv(p + "attn_gate.weight", xq)
        b, a = self.gemv(p + "ssm_beta.weight", xq), self.gemv(p + "ssm_alpha.weight", xq)
        beta, gate = orc.beta_gate(b, a, self.t[p + "ssm_dt.bias"][2], self.t[p + "ssm_a"][2])
        h, self.hist[il] = orc.gdn_conv_l2(self.hist[il], qkv, self.t[p + "ssm_conv1d.weight"][2], 2 * self.h_k,
                                           self.eps)
        hk = self.h_k * S
        y, self.state[il] = orc.gdn_step_norm(self.state[il], h[:hk], h[hk:2 * hk], h[2 * hk:], gate, beta, z,
                                              self.t[p + "ssm_norm.weight"][2], self.eps, self.h_k, self.h_v)
        y = f32(y)
        return self.gemv(p + "ssm_out.weight", orc.quantize_q8_1(y, y.size), res=x)

    def ffn(self, il, x):
        p = f"blk.{il}."
        xq = self.rms_q8(x, p + "post_attention_norm.weight")
        up, gt = self.gemv(p + "ffn_up.weight", xq), self.gemv(p + "ffn_gate.weight", xq)
        s = f32(orc.swiglu(up, gt))
        return self.gemv(p + "ffn_down.weight", orc.quantize_q8_1(s, s.size), res=x)

    def hidden(self, x, wname):
        """rms_norm_out (qw:616-672): x * w * rsqrt(mean(x^2) + eps) in fp32, and its partials"""
        inv = orc.rms_inv(orc.row_sum_partials(x), x.size, self.eps)
        h = f32(orc.rms_norm_out(x, self.t[wname][2], inv))
        return h, orc.row_sum_partials(h)

    # ---- the reference's passes ----
    def forward(self, tok, pos):
        """forward_token (qw:1773-1824): logits (fp32) of the token at pos, and the final-normed hidden"""
        x = self.embed(tok)
        for il in range(self.n_layer):
            x = self.attention(il, x, pos) if self.attn[il] else self.gdn(il, x)
            x = self.ffn(il, x)
        logits = self.gemv("output.weight", self.rms_q8(x, "output_norm.weight"))
        return logits, self.hidden(x, "output_norm.weight")[0]

    def draft(self, tok, pos, h_prev, with_head=True):
        """draft_predict (qw:1316-1406): [enorm(emb) | hnorm(h_prev)] -> eh_proj -> blk.<n_layer> -> head"""
        d = self.n_layer
        e = self.embed(tok)
        en, _ = self.hidden(e, f"blk.{d}.nextn.enorm.weight")
        hn, _ = self.hidden(h_prev, f"blk.{d}.nextn.hnorm.weight")
        eh = np.concatenate([en, hn])
        x = self.gemv(f"blk.{d}.nextn.eh_proj.weight", orc.quantize_q8_1(eh, eh.size))
        x = self.ffn(d, self.attention(d, x, pos))
        if not with_head:
            return None
        return self.gemv("output.weight", self.rms_q8(x, f"blk.{d}.nextn.shared_head_norm.weight"))

    def prefill(self, tokens):
        """the engine's prefill: draft KV row i from (token i, hidden i - 1; zero at 0), then the trunk token"""
        h = np.zeros(self.n_embd, np.float32)
        logits = None
        for i, t in enumerate(tokens):
            self.draft(t, i, h, with_head=False)
            logits, h = self.forward(t, i)
        return logits, h
