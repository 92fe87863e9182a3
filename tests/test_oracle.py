"""Pins the CPU oracle before anything is compared against it.

Each check uses a form independent of the oracle's own code: ggml's published dequantize_row_q6_K loop, the
reference's lane-mapped dp4a form (mmvq:733-748), numpy fp64 matrix forms, the Gated DeltaNet paper's
S(I - beta k k^T) update, complex-multiplication RoPE, and special cases with closed-form answers.
"""
import numpy as np
import pytest


# ---- fp16 ---------------------------------------------------------------------------------------------------------

def test_f16_round_trip_matches_numpy(orc):
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.normal(size=2000).astype(np.float32),
        (rng.normal(size=2000) * 1e-6).astype(np.float32),      # subnormal halves
        (rng.normal(size=500) * 7e4).astype(np.float32),        # overflow region (numpy warns on inf)
        np.array([0.0, -0.0, 65504.0, 65519.996, 65520.0, 2.0 ** -25, 2.0 ** -24, 1.5 * 2.0 ** -25], np.float32),
    ])
    L = orc.lib()
    ours = np.array([L.orc_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)
    ref = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)
    back = np.array([L.orc_f16_to_f32(int(h)) for h in ours], dtype=np.float32)
    assert np.array_equal(back.view(np.uint32), ref.view(np.float16).astype(np.float32).view(np.uint32))


def test_f16_saturation_policy(orc):
    L = orc.lib()
    assert L.orc_f16_sat(1e9) == 0x7BFF and L.orc_f16_sat(-1e9) == 0xFBFF
    assert L.orc_f16_sat(1.0) == 0x3C00


# ---- Q6_K layout ----------------------------------------------------------------------------------------------------

def ggml_dequant_q6k_block(b):
    """ggml dequantize_row_q6_K for one 210-byte block, transcribed from its published loop structure."""
    b = np.asarray(b, dtype=np.uint8)
    ql, qh = b[0:128].astype(np.int32), b[128:192].astype(np.int32)
    sc = b[192:208].view(np.int8).astype(np.int32)
    d = np.float64(b[208:210].view(np.float16)[0])
    y = np.zeros(256)
    for half in range(2):
        qlp, qhp, scp, yo = ql[64 * half:], qh[32 * half:], sc[8 * half:], 128 * half
        for l in range(32):
            is_ = l // 16
            q1 = ((qlp[l] & 0xF) | (((qhp[l] >> 0) & 3) << 4)) - 32
            q2 = ((qlp[l + 32] & 0xF) | (((qhp[l] >> 2) & 3) << 4)) - 32
            q3 = ((qlp[l] >> 4) | (((qhp[l] >> 4) & 3) << 4)) - 32
            q4 = ((qlp[l + 32] >> 4) | (((qhp[l] >> 6) & 3) << 4)) - 32
            y[yo + l] = d * scp[is_ + 0] * q1
            y[yo + l + 32] = d * scp[is_ + 2] * q2
            y[yo + l + 64] = d * scp[is_ + 4] * q3
            y[yo + l + 96] = d * scp[is_ + 6] * q4
    return y


def test_q6k_generator_matches_ggml_layout(orc):
    n_in, n_out = 512, 3
    w = orc.gen_q6k(n_out, n_in, seed=11)
    assert w.size == n_out * 2 * 210
    deq = orc.q6k_dequant(w, n_out, n_in)
    for r in range(n_out):
        for bi in range(2):
            blk = w[(r * 2 + bi) * 210:(r * 2 + bi + 1) * 210]
            np.testing.assert_array_equal(deq[r, 256 * bi:256 * (bi + 1)].astype(np.float64),
                                          ggml_dequant_q6k_block(blk).astype(np.float32).astype(np.float64))


def test_q6k_generator_distribution(orc):
    w = orc.gen_q6k(64, 4096, seed=5).reshape(-1, 210)
    codes = np.array([[orc.lib().orc_q6k_code(np.ascontiguousarray(b), e) for e in range(256)] for b in w[:40]])
    assert codes.min() == 0 and codes.max() == 63 and abs(codes.mean() - 31.5) < 1.0
    sc = w[:, 192:208].view(np.int8)
    assert sc.min() == -32 and sc.max() == 31
    d = w[:, 208:210].copy().view(np.float16).astype(np.float64)
    assert (d >= 0).all() and 0.5e-3 < np.sqrt((d ** 2).mean()) < 1.5e-3


def test_q6k_known_answer_block(orc):
    # every code 33 (q = +1), sub-scales 1..16, d = 1: element e dequantizes to sc[8n + l/16 + 2k]
    b = np.zeros(210, dtype=np.uint8)
    b[0:128] = 0x11            # low and high nibble 1
    b[128:192] = 0xAA          # every 2-bit field = 2  -> code = 1 | 2 << 4 = 33
    b[192:208] = np.arange(1, 17, dtype=np.int8).view(np.uint8)
    b[208:210] = np.array([1.0], dtype=np.float16).view(np.uint8)
    y = orc.q6k_dequant(b, 1, 256)[0]
    for e in range(256):
        n, k, l = e // 128, (e % 128) // 32, e % 32
        assert y[e] == 1 + 8 * n + l // 16 + 2 * k


# ---- Q8_1 quantizer -------------------------------------------------------------------------------------------------

def np_tree_sum32(v):
    a = v.astype(np.float32).copy()
    idx = np.arange(32)
    for off in (16, 8, 4, 2, 1):
        a = (a + a[idx ^ off]).astype(np.float32)
    return a[0]


def np_roundf(v):
    r = np.trunc(v)
    return r + np.sign(v) * (np.abs(v - r) >= 0.5)


def np_quant_q8_1(x):
    blocks = []
    for blk in x.reshape(-1, 32).astype(np.float32):
        amax = np.max(np.abs(blk))
        d = np.float32(amax) / np.float32(127.0)
        q = np.zeros(32, np.int8) if amax == 0 else np_roundf(blk / d).astype(np.int8)
        s = np_tree_sum32(blk)
        dh = np.float16(np.clip(d, -65504, 65504)).view(np.uint16)
        sh = np.float16(np.clip(s, -65504, 65504)).view(np.uint16)
        blocks.append(np.concatenate([np.array([dh, sh], np.uint16).view(np.uint8), q.view(np.uint8)]))
    return np.concatenate(blocks)


def test_quantize_q8_1_closed_form(orc):
    x = orc.normal(4096 * 2, seed=3)
    x[64:96] *= 1e4            # the finite-guard block: |sum| can exceed 65504
    x[128:160] = 0.0           # amax == 0
    x[160:192] = np.arange(32, dtype=np.float32) - 15.5   # exact halves
    y = orc.quantize_q8_1(x, 4096, 2)
    assert np.array_equal(y, np_quant_q8_1(x))
    d, s, q = orc.q8_1_fields(y)
    assert np.isfinite(d.view(np.float16)).all() and np.isfinite(s.view(np.float16)).all()
    assert (q[4] == 0).all() and d[4] == 0


def test_quantize_q8_1_dequant_error_bound(orc):
    x = orc.normal(8192, seed=4)
    deq = orc.dequantize_q8_1(orc.quantize_q8_1(x, 8192), 8192)
    amax = np.abs(x.reshape(-1, 32)).max(axis=1, keepdims=True)
    assert (np.abs(deq.reshape(-1, 32) - x.reshape(-1, 32)) <= amax / 127 * 0.5 + amax * 2e-3).all()


# ---- integer block dots ---------------------------------------------------------------------------------------------

@pytest.mark.parametrize("n_in,n_out", [(256, 1), (512, 7), (2048, 5)])
def test_q6k_block_dots_match_reference_lane_form(orc, n_in, n_out):
    w = orc.gen_q6k(n_out, n_in, seed=n_in + n_out)
    xq = orc.quantize_q8_1(orc.normal(n_in, seed=9), n_in)
    a = orc.q6k_block_dots(w, xq, n_in, n_out)
    b = orc.q6k_block_dots(w, xq, n_in, n_out, lanes=True)
    assert np.array_equal(a, b)


def test_q6k_block_dots_match_dequant_dot(orc):
    n_in, n_out = 1024, 4
    w = orc.gen_q6k(n_out, n_in, seed=21)
    xq = orc.quantize_q8_1(orc.normal(n_in, seed=22), n_in)
    dots = orc.q6k_block_dots(w, xq, n_in, n_out)
    _, _, q8 = orc.q8_1_fields(xq)
    for r in range(n_out):
        for bi in range(n_in // 256):
            blk = w[(r * (n_in // 256) + bi) * 210:][:210].copy()
            blk[208:210] = np.array([1.0], np.float16).view(np.uint8)      # d = 1: dequant = sc * (code - 32)
            wdeq = ggml_dequant_q6k_block(blk)
            for jj in range(8):
                j = 8 * bi + jj
                assert dots[r, j] == int(np.dot(wdeq[32 * jj:32 * jj + 32], q8[j].astype(np.float64)))


def test_q8_0_block_dots(orc):
    n_in, n_out = 512, 3
    w = orc.gen_q8_0(n_out, n_in, seed=2)
    xq = orc.quantize_q8_1(orc.normal(n_in, seed=8), n_in)
    dots = orc.q8_0_block_dots(w, xq, n_in, n_out)
    wq = w.reshape(n_out, n_in // 32, 34)[:, :, 2:].copy().view(np.int8).astype(np.int64)
    _, _, q8 = orc.q8_1_fields(xq)
    assert np.array_equal(dots, (wq * q8.astype(np.int64)[None]).sum(-1))


# ---- fp64 GEMVs and their invariants ----------------------------------------------------------------------------------

def test_q6k_gemv_matches_fp64_dequant_matmul(orc):
    n_in, n_out = 2048, 37
    w = orc.gen_q6k(n_out, n_in, seed=31)
    x = orc.normal(2 * n_in, seed=32)
    xq = orc.quantize_q8_1(x, n_in, 2)
    y = orc.q6k_gemv(w, xq, n_in, n_out, ncols=2).reshape(2, n_out)
    W = np.stack([np.concatenate([ggml_dequant_q6k_block(w[(r * 8 + b) * 210:][:210]) for b in range(8)])
                  for r in range(n_out)])
    d, _, q8 = orc.q8_1_fields(xq)
    X = (d.view(np.float16).astype(np.float64)[:, None] * q8.astype(np.float64)).reshape(2, n_in)
    ref = X @ W.T
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-12 * np.abs(ref).max())


def test_q6k_gemv_invariants(orc):
    n_in, n_out = 1024, 30
    w = orc.gen_q6k(n_out, n_in, seed=41)
    xq = orc.quantize_q8_1(orc.normal(2 * n_in, seed=42), n_in, 2)
    res = orc.normal(2 * n_out, seed=43)
    y2, p2 = orc.q6k_gemv(w, xq, n_in, n_out, ncols=2, res=res, partials=True)
    col_bytes = n_in // 32 * 36
    for c in range(2):
        y1 = orc.q6k_gemv(w, xq[c * col_bytes:(c + 1) * col_bytes], n_in, n_out)
        assert np.array_equal(y2[c * n_out:(c + 1) * n_out], y1 + res[c * n_out:(c + 1) * n_out].astype(np.float64))
        yc = y2[c * n_out:(c + 1) * n_out]
        groups = [yc[4 * g:4 * g + 4] for g in range((n_out + 3) // 4)]
        np.testing.assert_allclose(p2[c * 8:(c + 1) * 8], [np.sum(g ** 2) for g in groups], rtol=1e-14)


def test_q8_0_gemv(orc):
    n_in, n_out = 1024, 9
    w = orc.gen_q8_0(n_out, n_in, seed=51)
    xq = orc.quantize_q8_1(orc.normal(n_in, seed=52), n_in)
    y = orc.q8_0_gemv(w, xq, n_in, n_out)
    blk = w.reshape(n_out, n_in // 32, 34)
    dw = blk[:, :, :2].copy().view(np.float16)[..., 0].astype(np.float64)
    Wd = (dw[:, :, None] * blk[:, :, 2:].copy().view(np.int8)).reshape(n_out, n_in)
    X = orc.dequantize_q8_1(xq, n_in).astype(np.float64)
    np.testing.assert_allclose(y, Wd @ X, rtol=1e-12, atol=1e-12)


def test_f32_timing_build_close_to_fp64(orc):
    n_in, n_out = 4096, 64
    w = orc.gen_q6k(n_out, n_in, seed=61)
    xq = orc.quantize_q8_1(orc.normal(2 * n_in, seed=62), n_in, 2)
    res = orc.normal(2 * n_out, seed=63)
    y64 = orc.q6k_gemv(w, xq, n_in, n_out, ncols=2, res=res)
    y32, _ = orc.q6k_gemv_f32(w, xq, n_in, n_out, ncols=2, res=res, threads=2)
    np.testing.assert_allclose(y32, y64, rtol=1e-4, atol=1e-4 * np.abs(y64).max())


# ---- GDN ---------------------------------------------------------------------------------------------------------------

def test_gdn_conv_l2(orc):
    ch, qk = 8192, 32
    hist = orc.normal(3 * ch, seed=71, std=0.5)
    w = orc.normal(4 * ch, seed=72, std=0.5)
    x = orc.normal(ch, seed=73)
    h, hist2 = orc.gdn_conv_l2(hist, x, w, qk, 1e-6)
    win = np.concatenate([hist.reshape(ch, 3), x[:, None]], axis=1).astype(np.float64)
    s = (win * w.reshape(ch, 4)).sum(1)
    ref = s / (1 + np.exp(-s))
    ref[:qk * 128] = (ref[:qk * 128].reshape(qk, 128) /
                      np.sqrt((ref[:qk * 128].reshape(qk, 128) ** 2).sum(1, keepdims=True) + 1e-6)).reshape(-1)
    np.testing.assert_allclose(h, ref, rtol=1e-12, atol=1e-14)
    assert np.array_equal(hist2.reshape(ch, 3), win[:, 1:].astype(np.float32))
    # identity tap: w = [0,0,0,1] gives silu(x) on the v channels
    w_id = np.tile(np.array([0, 0, 0, 1], np.float32), ch)
    h_id, _ = orc.gdn_conv_l2(hist, x, w_id, 0, 1e-6)
    np.testing.assert_allclose(h_id, x / (1 + np.exp(-x.astype(np.float64))), rtol=1e-12)


def _gdn_inputs(orc, h_k=16, h_v=32, seed=80):
    S = 128
    state = orc.normal(S * h_v * S, seed=seed, std=0.05).astype(np.float64)
    q = orc.normal(h_k * S, seed=seed + 1); q /= np.linalg.norm(q.reshape(h_k, S), axis=1).repeat(S)
    k = orc.normal(h_k * S, seed=seed + 2); k /= np.linalg.norm(k.reshape(h_k, S), axis=1).repeat(S)
    v = orc.normal(h_v * S, seed=seed + 3)
    gate = -np.abs(orc.normal(h_v, seed=seed + 4)).astype(np.float64)
    beta = 1 / (1 + np.exp(-orc.normal(h_v, seed=seed + 5).astype(np.float64)))
    z = orc.normal(h_v * S, seed=seed + 6)
    gamma = (1 + orc.normal(S, seed=seed + 7, std=0.1)).astype(np.float32)
    return state, q.astype(np.float64), k.astype(np.float64), v.astype(np.float64), gate, beta, z, gamma


def test_gdn_step_matches_delta_rule_matrix_form(orc):
    h_k, h_v, S, eps = 16, 32, 128, 1e-6
    state, q, k, v, gate, beta, z, gamma = _gdn_inputs(orc)
    y, st = orc.gdn_step_norm(state, q, k, v, gate, beta, z, gamma, eps, h_k, h_v)
    St = state.reshape(S, h_v, S)
    st = st.reshape(S, h_v, S)
    for h in range(h_v):
        qh = h % h_k
        P = St[:, h, :].T                               # paper layout: d_v x d_k
        kk, qq = k[qh * S:(qh + 1) * S], q[qh * S:(qh + 1) * S]
        a, b = np.exp(gate[h]), beta[h]
        Pn = a * P @ (np.eye(S) - b * np.outer(kk, kk)) + b * np.outer(v[h * S:(h + 1) * S], kk)
        np.testing.assert_allclose(st[:, h, :].T, Pn, rtol=1e-10, atol=1e-13)
        o = Pn @ qq / np.sqrt(S)
        zz = z[h * S:(h + 1) * S].astype(np.float64)
        ref = o / np.sqrt(np.mean(o ** 2) + eps) * gamma * zz / (1 + np.exp(-zz))
        np.testing.assert_allclose(y[h * S:(h + 1) * S], ref, rtol=1e-9, atol=1e-12)


def test_gdn_step_zero_key_only_decays(orc):
    h_k, h_v = 16, 32
    state, q, k, v, gate, beta, z, gamma = _gdn_inputs(orc, seed=90)
    _, st = orc.gdn_step_norm(state, q, np.zeros_like(k), v, gate, beta, z, gamma, 1e-6, h_k, h_v)
    g = np.exp(gate)[None, :, None]
    np.testing.assert_allclose(st.reshape(128, h_v, 128), g * state.reshape(128, h_v, 128), rtol=1e-14)


# ---- attention ---------------------------------------------------------------------------------------------------------

def _kv(orc, n_tok, n_kv=4, hd=256, seed=100):
    k = orc.normal(n_tok * n_kv * hd, seed=seed).astype(np.float16).view(np.uint16)
    v = orc.normal(n_tok * n_kv * hd, seed=seed + 1).astype(np.float16).view(np.uint16)
    return k, v


def test_gqa_decode_softmax(orc):
    n_head, n_kv, hd, n_tok = 16, 4, 256, 77
    q = orc.normal(n_head * hd, seed=110)
    k, v = _kv(orc, n_tok)
    o = orc.gqa_decode(q, k, v, n_head, n_kv, hd, n_tok, 1 / 16).reshape(n_head, hd)
    K = k.view(np.float16).astype(np.float64).reshape(n_tok, n_kv, hd)
    V = v.view(np.float16).astype(np.float64).reshape(n_tok, n_kv, hd)
    for h in range(n_head):
        s = K[:, h // 4, :] @ q[h * hd:(h + 1) * hd].astype(np.float64) / 16
        p = np.exp(s - s.max()); p /= p.sum()
        np.testing.assert_allclose(o[h], p @ V[:, h // 4, :], rtol=1e-12, atol=1e-13)


def test_gqa_decode_special_cases(orc):
    n_head, n_kv, hd = 16, 4, 256
    q = orc.normal(n_head * hd, seed=120)
    k, v = _kv(orc, 9, seed=121)
    o1 = orc.gqa_decode(q, k, v, n_head, n_kv, hd, 1, 1 / 16).reshape(n_head, hd)
    V = v.view(np.float16).astype(np.float64).reshape(9, n_kv, hd)
    for h in range(n_head):
        np.testing.assert_allclose(o1[h], V[0, h // 4], rtol=1e-15)
    kc = np.tile(k.reshape(9, -1)[0], 9)
    oc = orc.gqa_decode(q, kc, v, n_head, n_kv, hd, 9, 1 / 16).reshape(n_head, hd)
    for h in range(n_head):
        np.testing.assert_allclose(oc[h], V[:, h // 4].mean(0), rtol=1e-12, atol=1e-14)


def test_rope_neox_complex_form(orc):
    heads, hd, n_rot, pos, theta = 3, 256, 64, 1234, 1e7
    x = orc.normal(heads * hd, seed=130).astype(np.float64)
    y = orc.rope_neox(x, heads, hd, n_rot, pos, theta).reshape(heads, hd)
    X = x.reshape(heads, hd)
    half = n_rot // 2
    ang = pos * theta ** (-np.arange(half) * 2.0 / n_rot)
    zc = (X[:, :half] + 1j * X[:, half:n_rot]) * np.exp(1j * ang)
    np.testing.assert_allclose(y[:, :half], zc.real, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(y[:, half:n_rot], zc.imag, rtol=1e-12, atol=1e-12)
    assert np.array_equal(y[:, n_rot:], X[:, n_rot:])
    assert np.allclose(orc.rope_neox(x, heads, hd, n_rot, 0, theta), x, rtol=0, atol=0)


def test_argmax_lowest_index_tie(orc):
    l = np.zeros(1000, np.float32)
    l[[17, 400, 999]] = 3.0
    assert orc.argmax(l) == 17
    l[5] = np.float32(3.0000002)
    assert orc.argmax(l) == 5


def test_beta_gate_and_norms(orc):
    b_in = orc.normal(32, seed=140); a = orc.normal(32, seed=141)
    dt = np.zeros(32, np.float32); ssm_a = -np.exp(orc.normal(32, seed=142, std=0.5))
    b, g = orc.beta_gate(b_in, a, dt, ssm_a)
    np.testing.assert_allclose(b, 1 / (1 + np.exp(-b_in.astype(np.float64))), rtol=1e-14)
    np.testing.assert_allclose(g, np.log(1 + np.exp(a.astype(np.float64))) * ssm_a, rtol=1e-12)
    big = np.full(32, 30.0, np.float32)
    _, g2 = orc.beta_gate(b_in, big, dt, ssm_a)
    np.testing.assert_allclose(g2, 30.0 * ssm_a.astype(np.float64), rtol=1e-14)   # softplus cut-over above 20
    x = orc.normal(4096, seed=143)
    p = orc.row_sum_partials(x)
    inv = orc.rms_inv(p, 4096, 1e-6)
    np.testing.assert_allclose(inv, 1 / np.sqrt(np.mean(x.astype(np.float64) ** 2) + 1e-6), rtol=1e-13)


def _rms_norm_def(x, w, eps):
    """RMSNorm from its definition, rowwise in fp64: x * w / sqrt(mean(x^2) + eps)."""
    x = np.asarray(x, dtype=np.float64)
    return x * np.asarray(w, dtype=np.float64) / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)


def _norm_out(orc, x, w, eps):
    """The engine's output-norm chain (qw:602-623, 658-672): 4-row partials, their sum, inverse RMS, (x*w)*inv."""
    return orc.rms_norm_out(x, w, orc.rms_inv(orc.row_sum_partials(x), x.size, eps))


def test_swiglu_special_cases(orc):
    """swiglu_quant's value silu(gate) * up (qw:676-689), pinned without retyping it: gate 0 gives 0, a gate of 40
    gives 40 * up exactly (sigmoid(40) rounds to 1 in fp64), -40 gives ~0, silu(g) - silu(-g) = g, and the hand-worked
    silu(1) * 2 = 2 sigmoid(1) (an up / gate swap would give silu(2) * 1 = 1.7616)"""
    up = np.array([0.5, -3.0, 7.25, 2.0], np.float32)
    assert np.array_equal(orc.swiglu(up, np.zeros(4, np.float32)), np.zeros(4))
    assert np.array_equal(orc.swiglu(up, np.full(4, 40.0, np.float32)), 40.0 * up.astype(np.float64))
    assert np.abs(orc.swiglu(up, np.full(4, -40.0, np.float32))).max() < 1e-14
    g = np.array([0.3, -1.7, 4.0, 9.5], np.float32)
    one = np.ones(4, np.float32)
    np.testing.assert_allclose(orc.swiglu(one, g) - orc.swiglu(one, -g), g.astype(np.float64), rtol=0, atol=1e-15)
    assert abs(orc.swiglu(np.array([2.0], np.float32), np.array([1.0], np.float32))[0] - 1.4621171572600098) < 1e-15


def test_sig_mul_special_cases(orc):
    """sig_mul_quant's value o * sigmoid(g) (qw:692-704): g 0 halves o exactly, 40 keeps it, -40 gives ~0,
    sig_mul(o, g) + sig_mul(o, -g) = o, and the hand-worked 2 * sigmoid(1) (an o / g swap gives sigmoid(2) = 0.8808)"""
    o = np.array([0.5, -3.0, 7.25, 1e4], np.float32)
    assert np.array_equal(orc.sig_mul(o, np.zeros(4, np.float32)), 0.5 * o.astype(np.float64))
    assert np.array_equal(orc.sig_mul(o, np.full(4, 40.0, np.float32)), o.astype(np.float64))
    assert np.abs(orc.sig_mul(o, np.full(4, -40.0, np.float32))).max() < 1e-13
    g = np.array([0.3, -1.7, 4.0, 9.5], np.float32)
    np.testing.assert_allclose(orc.sig_mul(o, g) + orc.sig_mul(o, -g), o.astype(np.float64), rtol=1e-15, atol=0)
    assert abs(orc.sig_mul(np.array([2.0], np.float32), np.array([1.0], np.float32))[0] - 1.4621171572600098) < 1e-15


def test_rms_norm_out_matches_definition(orc):
    for n, seed in ((4096, 150), (12288, 151), (8, 152)):
        x = orc.normal(n, seed=seed, std=3.0)
        w = orc.normal(n, seed=seed + 10, mean=1.0, std=0.1)
        np.testing.assert_allclose(_norm_out(orc, x, w, 1e-6), _rms_norm_def(x, w, 1e-6), rtol=1e-13, atol=0)


def test_rms_norm_out_hand_worked_row(orc):
    # sum of squares 1 + 4 + 4 + 16 = 25, mean 6.25, rms 2.5 (eps 0): inv = 0.4 exactly in the chain's arithmetic
    x = np.array([1.0, -2.0, 2.0, 4.0], np.float32)
    w = np.array([1.0, 1.0, 0.5, 2.0], np.float32)
    np.testing.assert_allclose(_norm_out(orc, x, w, 0.0), [0.4, -0.8, 0.4, 3.2], rtol=1e-15, atol=0)
    # w is applied elementwise: swapping two weights swaps exactly those two outputs
    out = _norm_out(orc, x, w[[0, 1, 3, 2]], 0.0)
    np.testing.assert_allclose(out, [0.4, -0.8, 1.6, 0.8], rtol=1e-15, atol=0)


def test_rms_norm_out_scale_invariance_and_unit_rms(orc):
    x = orc.normal(4096, seed=153)
    w = orc.normal(4096, seed=154, mean=1.0, std=0.1)
    base = _norm_out(orc, x, w, 0.0)
    for c in (0.25, 8.0, 1024.0):   # powers of two: every step of the chain scales exactly, so the output is equal
        assert np.array_equal(_norm_out(orc, (x * np.float32(c)).astype(np.float32), w, 0.0), base)
    c = np.float32(3.7)              # any other factor: equal up to the fp32 rounding of c*x
    np.testing.assert_allclose(_norm_out(orc, (x * c).astype(np.float32), w, 0.0), base, rtol=2e-7, atol=0)
    ones = np.ones(4096, np.float32)
    for eps in (0.0, 1e-6, 1e-2):    # w = 1: mean(out^2) = ms / (ms + eps)
        out = _norm_out(orc, x, ones, eps)
        ms = np.mean(x.astype(np.float64) ** 2)
        np.testing.assert_allclose(np.mean(out * out), ms / (ms + eps), rtol=1e-12)


def test_rms_norm_heads_matches_definition(orc):
    rows, cols = 16, 256
    x = orc.normal(rows * cols, seed=155, std=2.0).reshape(rows, cols)
    x[3] *= np.float32(100.0)        # rows are normed independently: one loud head changes no other row
    w = orc.normal(cols, seed=156, mean=1.0, std=0.1)
    out = orc.rms_norm_heads(x, w, rows, cols, 1e-6).reshape(rows, cols)
    np.testing.assert_allclose(out, _rms_norm_def(x, w, 1e-6), rtol=1e-13, atol=0)
    quiet = orc.rms_norm_heads(np.delete(x, 3, axis=0), w, rows - 1, cols, 1e-6).reshape(rows - 1, cols)
    assert np.array_equal(np.delete(out, 3, axis=0), quiet)
    # hand-worked: two 4-wide heads, weights shared by every head (indexed by column)
    hx = np.array([[1, -2, 2, 4], [3, 0, 0, 4]], np.float32)
    hw = np.array([1.0, 1.0, 0.5, 2.0], np.float32)
    ref = [[0.4, -0.8, 0.4, 3.2], [3 / 2.5, 0.0, 0.0, 2 * 4 / 2.5]]   # rms 2.5 for both rows
    np.testing.assert_allclose(orc.rms_norm_heads(hx, hw, 2, 4, 0.0).reshape(2, 4), ref, rtol=1e-15, atol=0)
    for c in (0.5, 64.0):            # per-row scale invariance, exact for powers of two at eps 0
        assert np.array_equal(orc.rms_norm_heads((x * np.float32(c)).astype(np.float32), w, rows, cols, 0.0),
                              orc.rms_norm_heads(x, w, rows, cols, 0.0))


# ---- K-quant token-embedding formats (qw:109-115; ggml dequantize_row_q4_K / q5_K) -------------------------------
from tests.kquant import k_blocks, pack_k_scales  # noqa: E402

@pytest.mark.parametrize("five_bit", [False, True])
def test_k_quant_dequant_from_fields(orc, five_bit):
    """every element = d * scale_j * q - dmin * min_j (both products exact in fp32, one rounding), for blocks packed
    from their fields with ggml's packing rule: pins the 12-byte scale/min unpacking (including the high bits of
    sub-blocks 4..7), the nibble order and, for Q5_K, the qh bit of each sub-block"""
    rng = np.random.default_rng(11 + five_bit)
    w, fields = k_blocks(rng, 6, five_bit)
    assert w.size == 6 * (orc.Q5K_BYTES if five_bit else orc.Q4K_BYTES)
    y = (orc.q5k_dequant if five_bit else orc.q4k_dequant)(w, 1, 6 * 256)
    for b, (d, dmin, sc, mn, q) in enumerate(fields):
        j = np.arange(256) // 32
        want = (np.float64(d) * sc[j] * q - np.float64(dmin) * mn[j]).astype(np.float32)
        assert np.array_equal(y[256 * b:256 * (b + 1)], want), f"block {b}"


def test_k_quant_scale_unpacking_extremes(orc):
    """all 6-bit scales / mins 63 (every high bit set) and 0, Q4_K: the unpacked values reach 63 in every slot"""
    for val in (0, 63):
        sc = np.full(8, val)
        blk = np.concatenate([np.array([1.0, 1.0], np.float16).view(np.uint8), pack_k_scales(sc, sc),
                              np.full(128, 0x11, np.uint8)])
        y = orc.q4k_dequant(blk, 1, 256)
        assert np.array_equal(y, np.full(256, val * 1.0 - val * 1.0, np.float32))
        blk2 = blk.copy()
        blk2[16:] = 0x32                                 # low nibble 2, high nibble 3
        y2 = orc.q4k_dequant(blk2, 1, 256).reshape(4, 2, 32)
        assert np.all(y2[:, 0] == 2 * val - val) and np.all(y2[:, 1] == 3 * val - val)


# ---- YaRN RoPE (qw:1991-1999 parameters) ----------------------------------------------------------------------
def test_rope_yarn_factor_one_is_plain_rope(orc):
    x = orc.normal(4 * 256, seed=71).astype(np.float64)
    for pos in (0, 1, 777, 200000):
        a = orc.rope_yarn(x, 4, 256, 64, pos, 1e7, 1.0, 262144.0)
        b = orc.rope_neox(x, 4, 256, 64, pos, 1e7)
        assert np.allclose(a, b, rtol=0, atol=1e-12)


def test_rope_yarn_limits(orc):
    """ext_factor 0 is linear position interpolation (plain RoPE at pos / factor, unit magnitude); with ext_factor 1
    the fastest-rotating pairs (i <= low) keep the extrapolated angle and the slowest (i >= high) take the interpolated
    one, both scaled by 1 + 0.1 ln(factor)"""
    hd, n_rot, base, factor, orig = 256, 64, 1e7, 4.0, 65536.0
    x = orc.normal(hd, seed=72).astype(np.float64)
    pos = 4 * 9001
    pi_ = orc.rope_yarn(x, 1, hd, n_rot, pos, base, factor, orig, ext_factor=0.0)
    assert np.allclose(pi_, orc.rope_neox(x, 1, hd, n_rot, pos // 4, base), rtol=0, atol=1e-10)
    y = orc.rope_yarn(x, 1, hd, n_rot, pos, base, factor, orig)
    m = 1 + 0.1 * np.log(factor)
    corr = lambda b: n_rot * np.log(orig / (b * 2 * np.pi)) / (2 * np.log(base))  # noqa: E731
    low, high = max(0, np.floor(corr(32.0))), min(n_rot - 1, np.ceil(corr(1.0)))
    half = n_rot // 2
    ext = orc.rope_neox(x, 1, hd, n_rot, pos, base)
    interp = orc.rope_neox(x, 1, hd, n_rot, pos // 4, base)
    for i in range(half):
        pair = [i, i + half]
        if i <= low:
            assert np.allclose(y[pair], m * ext[pair], rtol=0, atol=1e-10), i
        elif i >= high:
            assert np.allclose(y[pair], m * interp[pair], rtol=0, atol=1e-10), i
        # every pair is a rotation scaled by m
        assert np.isclose(np.hypot(*y[pair]), m * np.hypot(*x[pair]), rtol=1e-12)
    assert np.array_equal(y[n_rot:], x[n_rot:])
    assert 0 < low < high < half, "the ramp covers interior dims for these parameters"


@pytest.mark.parametrize("five_bit", [False, True])
def test_k_quant_gemv_matches_dequant_matmul(orc, five_bit):
    """the integer-dot GEMV equals the fp64 product of the dequantized weights (pinned above) and the dequantized
    Q8_1 activations: the min term must use the code sum of exactly the sub-block's 32 activations.  Each dequantized
    weight is one fp32 rounding of its exact value, so the bound is 2^-24 of sum |w x| per output."""
    from tests.kquant import k_blocks
    n_in, n_out, ncols = 768, 9, 2
    w, _ = k_blocks(np.random.default_rng(31 + five_bit), n_out * n_in // 256, five_bit)
    xq = orc.quantize_q8_1(orc.normal(ncols * n_in, seed=32), n_in, ncols)
    y = (orc.q5k_gemv if five_bit else orc.q4k_gemv)(w, xq, n_in, n_out, ncols=ncols)
    wd = (orc.q5k_dequant if five_bit else orc.q4k_dequant)(w, n_out, n_in).reshape(n_out, n_in).astype(np.float64)
    xd = orc.dequantize_q8_1(xq, ncols * n_in).reshape(ncols, n_in).astype(np.float64)
    bound = 2.0 ** -24 * (np.abs(xd) @ np.abs(wd).T) * 1.01
    assert np.all(np.abs(y.reshape(ncols, n_out) - xd @ wd.T) <= bound)
    assert np.abs(y).max() > 1e3 * bound.max(), "a nontrivial product"


# ---- the CPU baseline's SIMD timing build (oracle/cpu_round.c) against the oracle --------------------------------

@pytest.mark.parametrize("simd", [1, 2])
def test_timing_gemv_close_to_fp64(orc, simd):
    """AVX2 (simd 1) and, where the CPU has it, AVX-512 VNNI (simd 2) Q6_K x Q8_1 GEMV: 1 and 2 columns, residual and
    partials, within 1e-4 of the fp64 oracle (fp32 lane sums in another order)"""
    n_in, n_out = 4096, 96
    w = orc.gen_q6k(n_out, n_in, seed=171)
    xq = orc.quantize_q8_1(orc.normal(2 * n_in, seed=172), n_in, 2)
    res = orc.normal(2 * n_out, seed=173)
    y64, p64 = orc.q6k_gemv(w, xq, n_in, n_out, ncols=2, res=res, partials=True)
    y32, p32 = orc.cpr_q6k_gemv(w, xq, n_in, n_out, ncols=2, res=res, partials=True, threads=3, simd=simd)
    np.testing.assert_allclose(y32, y64, rtol=1e-4, atol=1e-4 * np.abs(y64).max())
    np.testing.assert_allclose(p32, p64, rtol=1e-4, atol=1e-4 * np.abs(p64).max())
    y1 = orc.cpr_q6k_gemv(w, xq[:n_in // 32 * 36], n_in, n_out, ncols=1, threads=1, simd=simd)
    np.testing.assert_allclose(y1, orc.q6k_gemv(w, xq, n_in, n_out, ncols=1), rtol=1e-4,
                               atol=1e-4 * np.abs(y64).max())


def test_timing_gdn_layer_close_to_oracle(orc):
    h_k, h_v, S, ntok = 2, 4, 128, 2
    ch = (2 * h_k + h_v) * S
    stride = ch + h_v * S
    qkvz = orc.normal(ntok * stride, seed=181)
    ab = orc.normal(ntok * 2 * h_v, seed=182)
    conv_w = orc.normal(4 * ch, seed=183, std=0.5)
    hist = orc.normal(3 * ch, seed=184, std=0.5)
    state = orc.normal(S * h_v * S, seed=185, std=0.05)
    dt = np.zeros(h_v, np.float32)
    ssm_a = (-np.exp(orc.normal(h_v, seed=186, std=0.5))).astype(np.float32)
    gamma = (1 + orc.normal(S, seed=187, std=0.1)).astype(np.float32)
    y, hist2, st2 = orc.cpr_gdn_layer(qkvz, stride, ab, conv_w, dt, ssm_a, gamma, 1e-6, hist, state, h_k, h_v, ntok,
                                      threads=2)
    st, hs = state.astype(np.float64), hist.copy()
    for t in range(ntok):
        x = qkvz[t * stride:(t + 1) * stride]
        h, hs = orc.gdn_conv_l2(hs, x[:ch], conv_w, 2 * h_k, 1e-6)
        b, g = orc.beta_gate(ab[t * 2 * h_v:t * 2 * h_v + h_v], ab[t * 2 * h_v + h_v:(t + 1) * 2 * h_v], dt, ssm_a)
        yr, st = orc.gdn_step_norm(st, h[:h_k * S], h[h_k * S:2 * h_k * S], h[2 * h_k * S:], g, b, x[ch:], gamma,
                                   1e-6, h_k, h_v)
        np.testing.assert_allclose(y[t * h_v * S:(t + 1) * h_v * S], yr, rtol=1e-4, atol=1e-5 * np.abs(yr).max())
    assert np.array_equal(hist2, hs)
    assert np.abs(st2 - st).max() < 1e-5


def test_timing_gqa_decode_close_to_oracle(orc):
    nh, nkv, hd, ctx, ntok = 16, 4, 256, 700, 2
    k = orc.normal(ctx * nkv * hd, seed=191).astype(np.float16).view(np.uint16)
    v = orc.normal(ctx * nkv * hd, seed=192).astype(np.float16).view(np.uint16)
    q = orc.normal(ntok * nh * hd, seed=193)
    p0 = ctx - ntok - 5
    o = orc.cpr_gqa_decode(q, k, v, nh, nkv, hd, p0, ntok, 1 / 16, threads=4)
    for t in range(ntok):
        ref = orc.gqa_decode(q[t * nh * hd:(t + 1) * nh * hd], k, v, nh, nkv, hd, p0 + t + 1, 1 / 16)
        np.testing.assert_allclose(o[t * nh * hd:(t + 1) * nh * hd], ref, rtol=1e-4, atol=1e-5 * np.abs(ref).max())
