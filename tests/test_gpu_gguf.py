"""A qwen35 GGUF through rmi_engine_create_gguf (load_model, qw:1978-2134) against the CPU oracle of the whole model
(oracle/model.py: forward_token qw:1773-1824 and draft_predict qw:1316-1406 composed from the pinned oracle pieces,
every matrix applied on its own, no concatenation).

The files are small members of the family (the nextn draft block always present) written with the reference's tensor
names and metadata keys.  Without Q8_1 rounding differences the engine and the oracle agree to ~1e-7 (fp32 against
fp64 inside the ops; observed on one-layer models).  But a ~1e-7 difference ahead of a Q8_1 quantization rounds an
activation to the neighbouring code now and then (~1e-5 per element here), which moves every output of the next GEMV
by about (amax / 127) / (sqrt(n) rms), ~1e-3 of their scale, and later tokens and layers carry it.  So the bars
(written here) admit such flips and still catch any systematic error, which would touch every row:
- K/V cache rows (trunk attention layers and the draft block): with one trunk layer at least 80% within fp16 rounding
  of the oracle's row (2e-3 of its max|.|) and every row within 3e-2; with four layers every row within 6e-2 (a flip
  perturbs the GDN state, and every later position carries it);
- logits and the final-normed hidden within 1e-2 (one layer) or 5e-2 (four layers) of max|.|, correlation > 0.9999 /
  0.999; GDN states within the same bound;
- the first greedy token equal to the oracle's argmax wherever the oracle's top-2 margin exceeds twice the bound; along
  a greedy stream (the oracle fed the engine's tokens) every token whose oracle margin exceeds 3e-2 of max|logit|
  (3x the observed error) equal to the oracle's argmax; MTP after a GGUF load bit-identical to greedy."""
import os

import numpy as np
import pytest

from tests.gguf_writer import STR, U32, F32 as GF32, write_gguf

pytestmark = pytest.mark.gpu

N_EMBD, N_FF, N_VOCAB, N_LAYER = 2048, 4096, 5000, 4
H_K, H_V, N_HEAD, N_KV, HD = 4, 8, 8, 2, 256


@pytest.fixture(scope="module")
def E():
    import rapier_amd.engine as eng
    from tests.gpu_util import torch
    torch()
    return eng


# a Q5_K_M-like type plan: matrix name suffix -> GGML type (others Q6_K).  qkv | gate | beta | alpha and q | k | v mix
# types (the per-part fallback), up | gate share Q5_K (one concatenated K-quant GEMV), ssm_out / attn_output / down
# are K-quant and Q8_0 residual GEMVs
MIXED = {"attn_qkv.weight": 13, "ssm_beta.weight": 8, "ssm_alpha.weight": 8, "ssm_out.weight": 12,
         "attn_q.weight": 13, "attn_k.weight": 13, "attn_output.weight": 12, "ffn_up.weight": 13,
         "ffn_gate.weight": 13, "ffn_down.weight": 8, "nextn.eh_proj.weight": 12}


def build_model(orc, seed=1, emb_type="Q6_K", rope_factor=None, pattern=(0, 0, 0, 1), mixed=False):
    """tensors name -> (ggml type, dims, data) with the reference's names (qw:2003-2127); pattern[il] = 1 for an
    attention layer; mixed: the MIXED type plan"""
    from tests.kquant import k_blocks
    rng = np.random.default_rng(seed)
    t = {}
    cnt = [0]

    def q6(name, n_in, n_out):
        cnt[0] += 1
        tp = next((v for k, v in MIXED.items() if name.endswith(k)), 14) if mixed else 14
        if tp == 14:
            data = orc.gen_q6k(n_out, n_in, seed=seed * 1000 + cnt[0])
        elif tp == 8:
            data = orc.gen_q8_0(n_out, n_in, seed=seed * 1000 + cnt[0], d_std=3e-3)
        else:
            data, _ = k_blocks(np.random.default_rng(seed * 1000 + cnt[0]), n_out * n_in // 256, tp == 13, d_std=2e-3)
        t[name] = (tp, (n_in, n_out), data)

    def vec(name, n, mean=1.0, std=0.1):
        t[name] = (0, (n,), (mean + std * rng.standard_normal(n)).astype(np.float32))

    if emb_type == "Q6_K":
        q6("token_embd.weight", N_EMBD, N_VOCAB)
    else:
        five = emb_type == "Q5_K"
        data, _ = k_blocks(rng, N_VOCAB * N_EMBD // 256, five)
        t["token_embd.weight"] = (13 if five else 12, (N_EMBD, N_VOCAB), data)
    q6("output.weight", N_EMBD, N_VOCAB)
    vec("output_norm.weight", N_EMBD)

    def attn(il):
        p = f"blk.{il}."
        vec(p + "attn_norm.weight", N_EMBD)
        vec(p + "post_attention_norm.weight", N_EMBD)
        q6(p + "attn_q.weight", N_EMBD, 2 * N_HEAD * HD)
        q6(p + "attn_k.weight", N_EMBD, N_KV * HD)
        q6(p + "attn_v.weight", N_EMBD, N_KV * HD)
        q6(p + "attn_output.weight", N_HEAD * HD, N_EMBD)
        vec(p + "attn_q_norm.weight", HD)
        vec(p + "attn_k_norm.weight", HD)

    def ffn(il):
        p = f"blk.{il}."
        q6(p + "ffn_up.weight", N_EMBD, N_FF)
        q6(p + "ffn_gate.weight", N_EMBD, N_FF)
        q6(p + "ffn_down.weight", N_FF, N_EMBD)

    ch = (2 * H_K + H_V) * 128
    n_layer = len(pattern)
    for il in range(n_layer):
        p = f"blk.{il}."
        if pattern[il]:
            attn(il)
        else:
            vec(p + "attn_norm.weight", N_EMBD)
            vec(p + "post_attention_norm.weight", N_EMBD)
            q6(p + "attn_qkv.weight", N_EMBD, ch)
            q6(p + "attn_gate.weight", N_EMBD, H_V * 128)
            q6(p + "ssm_beta.weight", N_EMBD, H_V)
            q6(p + "ssm_alpha.weight", N_EMBD, H_V)
            q6(p + "ssm_out.weight", H_V * 128, N_EMBD)
            t[p + "ssm_conv1d.weight"] = (0, (4, ch), (0.5 * rng.standard_normal(4 * ch)).astype(np.float32))
            vec(p + "ssm_dt.bias", H_V, 0.0, 0.3)
            t[p + "ssm_a"] = (0, (H_V,), (-np.exp(0.5 * rng.standard_normal(H_V))).astype(np.float32))
            vec(p + "ssm_norm.weight", 128)
        ffn(il)
    d = n_layer
    attn(d)
    ffn(d)
    q6(f"blk.{d}.nextn.eh_proj.weight", 2 * N_EMBD, N_EMBD)
    for w in ("enorm", "hnorm", "shared_head_norm"):
        vec(f"blk.{d}.nextn.{w}.weight", N_EMBD)
    meta = [("general.architecture", STR, "qwen35"), ("qwen35.block_count", U32, n_layer + 1),
            ("qwen35.nextn_predict_layers", U32, 1), ("qwen35.attention.layer_norm_rms_epsilon", GF32, 1e-6),
            ("qwen35.rope.freq_base", GF32, 1e7), ("qwen35.rope.dimension_count", U32, 64),
            ("qwen35.embedding_length", U32, N_EMBD)]
    if rope_factor:
        meta += [("qwen35.rope.scaling.factor", GF32, rope_factor),
                 ("qwen35.rope.scaling.original_context_length", U32, 4096)]
    return t, meta


def write(t, meta, path):
    names = {0: "F32", 14: "Q6_K", 13: "Q5_K", 12: "Q4_K", 8: "Q8_0"}
    return write_gguf(str(path), meta, [(n, names[tp], dims, data) for n, (tp, dims, data) in t.items()])


def close(a, b, frac, what):
    a, b = np.asarray(a, np.float64), np.asarray(b, np.float64)
    err, scale = np.abs(a - b).max(), np.abs(b).max()
    assert err <= frac * scale, f"{what}: max err {err:.3e} vs {frac} x {scale:.3e}"
    return err


def oracle_model(orc, t, n_layer, **kw):
    import oracle.model as om
    return om.Qwen35(t, n_layer, **kw)


def check_rows(got, ref, row, exact_frac, bound, what):
    """K/V rows: a fraction exact_frac within fp16 rounding (2e-3), every one within bound (relative to max|row|)"""
    got, ref = got.reshape(-1, row), ref.reshape(-1, row)
    rel = np.abs(got - ref).max(1) / np.maximum(np.abs(ref).max(1), 1e-30)
    assert rel.max() <= bound, f"{what}: row errors {np.round(rel, 5)}"
    assert (rel <= 2e-3).mean() >= exact_frac, f"{what}: row errors {np.round(rel, 5)}"


@pytest.mark.parametrize("pattern,emb_type,rope_factor,mixed", [
    ((0,), "Q6_K", None, False), ((1,), "Q5_K", 4.0, False), ((0,), "Q4_K", None, False),
    ((0, 0, 0, 1), "Q6_K", None, False), ((0,), "Q5_K", None, True), ((1,), "Q6_K", None, True),
    ((0, 0, 0, 1), "Q5_K", None, True)])
def test_gguf_engine_matches_oracle_model(orc, E, tmp_path, pattern, emb_type, rope_factor, mixed):
    """mixed: a Q5_K_M-like file - Q5_K / Q4_K / Q8_0 / Q6_K matrices, groups of mixed type on the per-part fallback"""
    n_layer = len(pattern)
    bound, corr, row_bound, exact_frac = (1e-2, 0.9999, 3e-2, 0.8) if n_layer == 1 else (5e-2, 0.999, 6e-2, 0.0)
    t, meta = build_model(orc, seed=3, emb_type=emb_type, rope_factor=rope_factor, pattern=pattern, mixed=mixed)
    eng = E.Engine.from_gguf(write(t, meta, tmp_path / "m.gguf"), max_ctx=512)
    c = eng.cfg
    assert (c.n_embd, c.n_ff, c.n_vocab, c.n_layer, c.n_head, c.n_kv, c.head_dim, c.n_rot) == \
        (N_EMBD, N_FF, N_VOCAB, n_layer, N_HEAD, N_KV, HD, 64)
    if not all(pattern):
        assert (c.ssm_h_k, c.ssm_h_v) == (H_K, H_V)
    assert c.rope_factor == (rope_factor or 1.0)
    m = oracle_model(orc, t, n_layer, rope_factor=rope_factor or 1.0, rope_orig_ctx=4096.0)
    prompt = [int(x) for x in np.random.default_rng(9).integers(0, N_VOCAB, 7)]
    first = eng.prefill(prompt, batch=1)
    lo, h = m.prefill(prompt)
    logits = eng.read(E.BUF_LOGITS, 0, 4 * N_VOCAB).view(np.float32)
    close(logits, lo, bound, "logits")
    assert np.corrcoef(logits, lo)[0, 1] > corr
    close(eng.read(E.BUF_HIDDEN, 0, 4 * N_EMBD).view(np.float32), h, bound, "hidden")
    top = np.sort(lo)[-2:]
    if top[1] - top[0] > 2 * bound * np.abs(lo).max():
        assert first == int(np.argmax(lo))
    for il in range(n_layer):
        if not pattern[il]:
            st = eng.read(E.BUF_GDN_STATE, il, 4 * 128 * H_V * 128).view(np.float32)
            close(st, m.state[il], bound, f"GDN state of layer {il}")
    n = len(prompt) * N_KV * HD
    for il in [i for i in range(n_layer) if pattern[i]] + [n_layer]:   # trunk attention layers and the draft block
        for which, ref in ((E.BUF_K_CACHE, m.kc[il]), (E.BUF_V_CACHE, m.vc[il])):
            got = eng.read(which, il, 2 * n).view(np.float16).astype(np.float64)
            check_rows(got, ref[:n].view(np.float16).astype(np.float64), N_KV * HD, exact_frac, row_bound,
                       f"cache {which} layer {il}")
    # the chunked ingest of the same file leaves the same state
    h1 = eng.read(E.BUF_HIDDEN, 0, 4 * N_EMBD)
    assert eng.prefill(prompt, batch=16) == first
    assert np.array_equal(eng.read(E.BUF_HIDDEN, 0, 4 * N_EMBD), h1)
    eng.close()


def test_gguf_engine_greedy_and_mtp_streams(orc, E, tmp_path):
    """greedy tokens after the prompt follow the oracle model (while its top-2 margin is clear of the bound), and MTP
    on the loaded model reproduces the greedy stream"""
    t, meta = build_model(orc, seed=5)
    eng = E.Engine.from_gguf(write(t, meta, tmp_path / "g.gguf"), max_ctx=512)
    m = oracle_model(orc, t, N_LAYER)
    prompt = [11, 222, 3333, 44]
    first = eng.prefill(prompt, batch=4)
    lo, h = m.prefill(prompt)
    pos0, cur0 = eng.state()
    eng.save_state()
    toks, _ = eng.generate(12, mode=E.GREEDY)
    stream = [first] + toks
    checked = 0
    for i in range(len(toks)):   # the oracle follows the engine's tokens; each clear-margin step must agree
        lo, h = m.forward(stream[i], len(prompt) + i)
        top = np.sort(lo)[-2:]
        if top[1] - top[0] > 3e-2 * np.abs(lo).max():
            assert stream[i + 1] == int(np.argmax(lo)), f"greedy token {i}"
            checked += 1
    assert checked >= 4, "too few tokens with a clear margin"
    eng.restore_state(pos0, cur0)
    mtp, st = eng.generate(12, mode=E.MTP)
    assert mtp == toks
    eng.close()


def test_gguf_engine_swiglu_packing_at_4096(orc, E, tmp_path, monkeypatch):
    """at 4096-wide rows the loader packs up||gate in the SwiGLU row order: the fused up||gate + SwiGLU kernel (decode)
    and the interleaved SwiGLU (ingest chunks) must still follow the oracle model, and agree bit for bit"""
    import sys
    mod = sys.modules[__name__]
    monkeypatch.setattr(mod, "N_EMBD", 4096)
    t, meta = build_model(orc, seed=4, pattern=(0,))
    eng = E.Engine.from_gguf(write(t, meta, tmp_path / "w.gguf"), max_ctx=512)
    assert eng.cfg.n_embd == 4096
    m = oracle_model(orc, t, 1, rope_factor=1.0, rope_orig_ctx=4096.0)
    prompt = [int(x) for x in np.random.default_rng(13).integers(0, N_VOCAB, 7)]
    first = eng.prefill(prompt, batch=1)
    lo, h = m.prefill(prompt)
    close(eng.read(E.BUF_LOGITS, 0, 4 * N_VOCAB).view(np.float32), lo, 1e-2, "logits")
    close(eng.read(E.BUF_HIDDEN, 0, 4 * 4096).view(np.float32), h, 1e-2, "hidden")
    h1 = eng.read(E.BUF_HIDDEN, 0, 4 * 4096)
    assert eng.prefill(prompt, batch=16) == first
    assert np.array_equal(eng.read(E.BUF_HIDDEN, 0, 4 * 4096), h1)
    eng.close()


def clear_margin(lo, bound):
    top = np.sort(lo)[-2:]
    return top[1] - top[0] > 2 * bound * np.abs(lo).max()


@pytest.mark.parametrize("pattern,emb_type", [((0,), "Q6_K"), ((1,), "Q5_K"), ((0, 0, 0, 1), "Q6_K")])
def test_gguf_draft_head_matches_oracle(orc, E, tmp_path, pattern, emb_type):
    """the draft head (draft_predict with_head, qw:1316-1406: [enorm(emb) | hnorm(h)] -> eh_proj -> blk.<n_layer> ->
    shared_head_norm -> lm_head -> argmax) against Qwen35.draft(with_head=True): the 1-column first draft after the
    prompt, then the 2-column draft of one verify round (column 0 = (c0, hidden of verify column 0) at pos + 1,
    column 1 = (c1, hidden of column 1) at pos + 2).  Logits within the module's flip-tolerant bars, the candidate the
    engine keeps equal to the argmax of its own draft logits, and to the oracle's wherever its top-2 margin is clear."""
    n_layer = len(pattern)
    bound, corr = (1e-2, 0.9999) if n_layer == 1 else (5e-2, 0.999)
    t, meta = build_model(orc, seed=7, emb_type=emb_type, pattern=pattern)
    eng = E.Engine.from_gguf(write(t, meta, tmp_path / "d.gguf"), max_ctx=512)
    m = oracle_model(orc, t, n_layer)
    prompt = [int(x) for x in np.random.default_rng(21).integers(0, N_VOCAB, 6)]
    n = len(prompt)
    first = eng.prefill(prompt, batch=1)
    lo, h = m.prefill(prompt)
    V = N_VOCAB

    def logits(col):
        return eng.read(E.BUF_LOGITS, 0, 4 * V, offset=4 * V * col).view(np.float32)

    checked = 0
    # first draft: (current token, hidden of the last forward) at the current position
    eng.gen_begin(E.MTP)
    s = eng.round_slots()
    assert (s["pos"], s["cur"]) == (n, first)
    d = m.draft(first, n, h, with_head=True)
    got = logits(0)
    close(got, d, bound, "first draft logits")
    assert np.corrcoef(got, d)[0, 1] > corr
    assert s["c0"] == int(np.argmax(got)) == s["cand"]
    if clear_margin(d, bound):
        assert s["cand"] == int(np.argmax(d))
        checked += 1
    # one verify round: the oracle runs both verify columns, then both draft columns on the engine's tokens
    cand = s["cand"]
    emitted = eng.gen_step()
    s = eng.round_slots()
    lo0, h0 = m.forward(first, n)
    lo1, h1 = m.forward(cand, n + 1)
    assert emitted[0] == s["v0"]
    if clear_margin(lo0, bound):
        assert s["v0"] == int(np.argmax(lo0))
    d0 = m.draft(s["v0"], n + 1, h0, with_head=True)
    d1 = m.draft(s["v1"], n + 2, h1, with_head=True)
    for col, ref in ((0, d0), (1, d1)):
        got = logits(col)
        close(got, ref, bound, f"draft column {col} logits")
        assert np.corrcoef(got, ref)[0, 1] > corr
        assert s[f"c{col}"] == int(np.argmax(got))
        if clear_margin(ref, bound):
            assert s[f"c{col}"] == int(np.argmax(ref)), f"draft column {col} argmax"
            checked += 1
    assert s["cand"] == (s["c1"] if s["accept"] else s["c0"])
    assert checked >= 1, "no draft step with a clear oracle margin"
    eng.close()


# ---- full width: the 9B shapes (hidden 4096, FFN 12288, vocab 248320, 16 / 32 GDN heads, 16 / 4 attention heads) ----
FULL = dict(N_EMBD=4096, N_FF=12288, N_VOCAB=248320, H_K=16, H_V=32, N_HEAD=16, N_KV=4)


@pytest.fixture(scope="module")
def full_width(orc, tmp_path_factory):
    """a 2.6 GB file of the 9B widths with three GDN layers, one attention layer and the nextn block: every GEMV at
    its round shape (in-projections 12352 / 10240 x 4096, up||gate 24576 x 4096, down 4096 x 12288, eh_proj
    4096 x 8192, lm_head 248320 x 4096) and the embedding / argmax / top-k over the full vocabulary"""
    import sys
    mod = sys.modules[__name__]
    saved = {k: getattr(mod, k) for k in FULL}
    for k, v in FULL.items():
        setattr(mod, k, v)
    try:
        t, meta = build_model(orc, seed=31, pattern=(0, 0, 0, 1))
        path = write(t, meta, tmp_path_factory.mktemp("full") / "full.gguf")
    finally:
        for k, v in saved.items():
            setattr(mod, k, v)
    yield t, path
    os.unlink(path)


@pytest.mark.timeout(400)
def test_gguf_full_width_matches_oracle_model(orc, E, full_width):
    """qw:1773-1824 at full width: a 5-token prompt through the engine and through oracle/model.py; logits, hidden and
    GDN states within the 4-layer bars of this module (5e-2 of max|.|, correlation > 0.999), K/V rows within 6e-2, the
    first token the oracle's argmax where its margin is clear; the chunked ingest leaves the per-token state"""
    t, path = full_width
    V, D = FULL["N_VOCAB"], FULL["N_EMBD"]
    eng = E.Engine.from_gguf(str(path), max_ctx=512)
    c = eng.cfg
    assert (c.n_embd, c.n_ff, c.n_vocab, c.ssm_h_k, c.ssm_h_v, c.n_head, c.n_kv) == \
        (D, FULL["N_FF"], V, FULL["H_K"], FULL["H_V"], FULL["N_HEAD"], FULL["N_KV"])
    m = oracle_model(orc, t, 4)
    prompt = [5, 77, 12345, 248000, 9]
    first = eng.prefill(prompt, batch=1)
    lo, h = m.prefill(prompt)
    logits = eng.read(E.BUF_LOGITS, 0, 4 * V).view(np.float32)
    close(logits, lo, 5e-2, "logits")
    assert np.corrcoef(logits, lo)[0, 1] > 0.999
    close(eng.read(E.BUF_HIDDEN, 0, 4 * D).view(np.float32), h, 5e-2, "hidden")
    if clear_margin(lo, 5e-2):
        assert first == int(np.argmax(lo))
    for il in range(3):
        st = eng.read(E.BUF_GDN_STATE, il, 4 * 128 * FULL["H_V"] * 128).view(np.float32)
        close(st, m.state[il], 5e-2, f"GDN state of layer {il}")
    n = len(prompt) * FULL["N_KV"] * HD
    for il in (3, 4):   # the trunk attention layer and the draft block
        for which, ref in ((E.BUF_K_CACHE, m.kc[il]), (E.BUF_V_CACHE, m.vc[il])):
            got = eng.read(which, il, 2 * n).view(np.float16).astype(np.float64)
            check_rows(got, ref[:n].view(np.float16).astype(np.float64), FULL["N_KV"] * HD, 0.0, 6e-2,
                       f"cache {which} layer {il}")
    h1 = eng.read(E.BUF_HIDDEN, 0, 4 * D)
    assert eng.prefill(prompt, batch=16) == first
    assert np.array_equal(eng.read(E.BUF_HIDDEN, 0, 4 * D), h1)
    eng.close()


@pytest.mark.timeout(400)
def test_gguf_full_width_greedy_and_mtp(orc, E, full_width):
    """greedy tokens at full width follow the oracle model where its top-2 margin is clear (the oracle fed the
    engine's tokens), and MTP on the same file reproduces the greedy stream"""
    t, path = full_width
    eng = E.Engine.from_gguf(str(path), max_ctx=512)
    m = oracle_model(orc, t, 4)
    prompt = [11, 222, 3333, 44]
    first = eng.prefill(prompt, batch=4)
    m.prefill(prompt)
    pos0, cur0 = eng.state()
    eng.save_state()
    toks, _ = eng.generate(6, mode=E.GREEDY)
    stream = [first] + toks
    checked = 0
    for i in range(len(toks)):
        lo, _ = m.forward(stream[i], len(prompt) + i)
        if clear_margin(lo, 1.5e-2):
            assert stream[i + 1] == int(np.argmax(lo)), f"greedy token {i}"
            checked += 1
    assert checked >= 2, "too few tokens with a clear margin"
    eng.restore_state(pos0, cur0)
    mtp, _ = eng.generate(6, mode=E.MTP)
    assert mtp == toks
    eng.close()
