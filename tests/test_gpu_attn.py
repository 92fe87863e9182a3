"""GPU parity of the GQA decode attention (config 4: 16 q heads, 4 KV heads, head_dim 256, 2 query positions, fp16 KV
cache N(0,1) at contexts 4096 / 32768 / 65536, RoPE'd fp32 queries N(0,1), sigmoid output gate, Q8_1 output).

Bars (written here): gated fp32 output within 1e-3 relative of the oracle's fp64 softmax over the same fp16 K/V;
Q8_1 within half a quantization step.  Invariants, bit for bit: each column of the 2-query launch equals the
1-query launch at that position (chunking depends only on the query position).  attn_prep (per-head RMSNorm,
NEOX RoPE, fp16 store) is checked against the oracle's RMSNorm and complex-form-pinned RoPE.
"""
import numpy as np
import pytest

from tests.gpu_util import assert_close_rel, dev, empty, host, torch

pytestmark = pytest.mark.gpu

NH, NKV, HD = 16, 4, 256
Q3 = NH * 2 * HD + 2 * NKV * HD     # 10240: [16 x (q | gate) | k | v]
SCALE = 1.0 / 16.0


@pytest.fixture(scope="module")
def rmi():
    import rapier_amd
    rapier_amd.lib()
    return rapier_amd


def kv_cache(orc, ctx, seed):
    k = orc.normal(ctx * NKV * HD, seed=seed).astype(np.float16).view(np.uint16)
    v = orc.normal(ctx * NKV * HD, seed=seed + 1).astype(np.float16).view(np.uint16)
    return k, v


def flash(rmi, q, kc, vc, p0, gate, ntok, max_ctx, nsub):
    ws = empty(rmi.gqa_workspace_bytes(max_ctx, NKV, nsub), "uint8")
    y = empty(ntok * NH * HD)
    q8 = empty(ntok * NH * HD // 32 * 36, "uint8")
    rmi.gqa_flash_decode(q, kc, vc, dev(np.array([p0], np.int32)), gate, Q3, y, NH * HD, q8, NH * HD // 32 * 36, ws,
                         NH, NKV, HD, ntok, max_ctx, nsub, SCALE)
    return host(y), host(q8)


# The engine sizes the chunk so that a full cache is one partial workgroup per CU (at least 128 positions): nsub 2 at
# 4K-class caches, 16 at a 65536-position cache and 17 at the 66048 positions a 64K context with room for generation
# takes (1088-position chunks, the last one 768 long) on 256 CUs, so the merge path the round runs is checked against
# the oracle at its real chunk counts
@pytest.mark.parametrize("ctx,nsub", [(4096, 1), (4096, 2), (32768, 4), (65536, 4), (65536, 8), (65536, 16),
                                      (66048, 17)])
def test_flash_decode_matches_oracle(orc, rmi, ctx, nsub):
    kc, vc = kv_cache(orc, ctx, seed=ctx)
    q = orc.normal(2 * NH * HD, seed=ctx + 7)
    g = orc.normal(2 * Q3, seed=ctx + 8)
    p0 = ctx - 2
    dk, dv, dq, dg = dev(kc), dev(vc), dev(q), dev(g)
    y, q8 = flash(rmi, dq, dk, dv, p0, dg, 2, ctx, nsub)
    for t in range(2):
        o = orc.gqa_decode(q[t * NH * HD:(t + 1) * NH * HD], kc, vc, NH, NKV, HD, p0 + t + 1, SCALE)
        gate = np.concatenate([g[t * Q3 + h * 2 * HD + HD:t * Q3 + h * 2 * HD + 2 * HD] for h in range(NH)])
        ref = o / (1 + np.exp(-gate.astype(np.float64)))
        assert_close_rel(y[t * NH * HD:(t + 1) * NH * HD], ref, rtol=1e-3, atol_frac=1e-5, what=f"ctx {ctx} t{t}")
        blk = NH * HD // 32 * 36
        deq = orc.dequantize_q8_1(q8[t * blk:(t + 1) * blk], NH * HD).reshape(-1, 32).astype(np.float64)
        r = ref.reshape(-1, 32)
        amax = np.abs(r).max(1, keepdims=True)
        assert (np.abs(deq - r) <= 0.5 * amax / 127 * 1.001 + 2e-3 * amax).all(), f"q8 t{t}"
    # each verify column is bitwise the single-query launch at its position
    for t in range(2):
        y1, q81 = flash(rmi, dq[t * NH * HD:], dk, dv, p0 + t, dg[t * Q3:], 1, ctx, nsub)
        assert np.array_equal(y1.view(np.uint32), y[t * NH * HD:(t + 1) * NH * HD].view(np.uint32))


@pytest.mark.parametrize("p0", [0, 1, 63, 64, 200])
def test_flash_decode_short_contexts(orc, rmi, p0):
    """edge cases: a single visible position (o = V0), chunk boundaries at 64."""
    ctx = 320
    kc, vc = kv_cache(orc, ctx, seed=900 + p0)
    q = orc.normal(2 * NH * HD, seed=901)
    g = np.full(2 * Q3, 40.0, np.float32)            # sigmoid(40) == 1: y is the attention output itself
    y, _ = flash(rmi, dev(q), dev(kc), dev(vc), p0, dev(g), 2, ctx, 1)
    for t in range(2):
        o = orc.gqa_decode(q[t * NH * HD:(t + 1) * NH * HD], kc, vc, NH, NKV, HD, p0 + t + 1, SCALE)
        assert_close_rel(y[t * NH * HD:(t + 1) * NH * HD], o, rtol=1e-3, atol_frac=1e-5, what=f"p0 {p0} t{t}")
    if p0 == 0:
        v0 = vc[:NKV * HD].view(np.float16).astype(np.float32).reshape(NKV, HD)
        assert np.array_equal(y[:NH * HD].reshape(NH, HD), np.repeat(v0, NH // NKV, axis=0))


@pytest.mark.parametrize("ntok", [2, 16])
def test_attn_prep_matches_oracle(orc, rmi, ntok):
    """2 tokens (the verify pair) and 16 (an ingest chunk): every token at its own position p0 + t"""
    t_ = torch()
    max_ctx, p0, theta, eps = 1024, 777, 1e7, 1e-6
    q3 = orc.normal(ntok * Q3, seed=950)
    qn = (1 + orc.normal(HD, seed=951, std=0.1)).astype(np.float32)
    kn = (1 + orc.normal(HD, seed=952, std=0.1)).astype(np.float32)
    kc = t_.zeros(max_ctx * NKV * HD, dtype=t_.int16, device="cuda:0")
    vc = t_.zeros(max_ctx * NKV * HD, dtype=t_.int16, device="cuda:0")
    qo = empty(ntok * NH * HD)
    rmi.attn_prep(dev(q3), Q3, dev(qn), dev(kn), kc, vc, dev(np.array([p0], np.int32)), qo, NH, NKV, HD, 64, theta,
                  eps, ntok, max_ctx)
    qh, kh, vh = host(qo), host(kc).view(np.float16), host(vc).view(np.float16)
    for t in range(ntok):
        src = q3[t * Q3:(t + 1) * Q3]
        qx = np.concatenate([src[h * 2 * HD:h * 2 * HD + HD] for h in range(NH)])
        qref = orc.rope_neox(orc.rms_norm_heads(qx, qn, NH, HD, eps), NH, HD, 64, p0 + t, theta)
        assert_close_rel(qh[t * NH * HD:(t + 1) * NH * HD], qref, rtol=1e-5, atol_frac=2e-6, what=f"q t{t}")
        kref = orc.rope_neox(orc.rms_norm_heads(src[NH * 2 * HD:NH * 2 * HD + NKV * HD], kn, NKV, HD, eps),
                             NKV, HD, 64, p0 + t, theta)
        kg = kh[(p0 + t) * NKV * HD:(p0 + t + 1) * NKV * HD].astype(np.float64)
        assert np.abs(kg - kref).max() <= np.abs(kref).max() * 1e-3, f"k t{t}"
        vref = src[NH * 2 * HD + NKV * HD:].astype(np.float16)
        assert np.array_equal(vh[(p0 + t) * NKV * HD:(p0 + t + 1) * NKV * HD], vref)
    assert not host(kc)[:p0 * NKV * HD].any(), "attn_prep wrote outside its positions"
    assert not host(kc)[(p0 + ntok) * NKV * HD:].any(), "attn_prep wrote outside its positions"


@pytest.mark.parametrize("ctx,nsub,ntok", [(4096, 2, 16), (2048, 1, 13), (65536, 8, 16), (65536, 16, 16),
                                           (66048, 17, 16)])
def test_flash_decode_chunk_bitwise_equals_single_queries(orc, rmi, ctx, nsub, ntok):
    """an ingest chunk: ntok query tokens (ntok * 4 = up to 64 query vectors per KV head, 8 slot groups) in one launch;
    each token's y and Q8_1 are bitwise the 1-token launch at its position; token 0 within 1e-3 of the oracle"""
    kc, vc = kv_cache(orc, ctx, seed=ctx + ntok)
    q = orc.normal(ntok * NH * HD, seed=ctx + 17)
    g = orc.normal(ntok * Q3, seed=ctx + 18)
    p0 = ctx - ntok - 3
    dk, dv, dq, dg = dev(kc), dev(vc), dev(q), dev(g)
    y, q8 = flash(rmi, dq, dk, dv, p0, dg, ntok, ctx, nsub)
    blk = NH * HD // 32 * 36
    for t in range(ntok):
        y1, q81 = flash(rmi, dq[t * NH * HD:], dk, dv, p0 + t, dg[t * Q3:], 1, ctx, nsub)
        assert np.array_equal(y1.view(np.uint32), y[t * NH * HD:(t + 1) * NH * HD].view(np.uint32)), f"token {t}"
        assert np.array_equal(q81, q8[t * blk:(t + 1) * blk]), f"q8 token {t}"
    o = orc.gqa_decode(q[:NH * HD], kc, vc, NH, NKV, HD, p0 + 1, SCALE)
    gate = np.concatenate([g[h * 2 * HD + HD:h * 2 * HD + 2 * HD] for h in range(NH)])
    assert_close_rel(y[:NH * HD], o / (1 + np.exp(-gate.astype(np.float64))), rtol=1e-3, atol_frac=1e-5, what="t0")


@pytest.mark.parametrize("factor,ntok", [(4.0, 3), (1.0, 2)])
def test_attn_prep_yarn_matches_oracle(orc, rmi, factor, ntok):
    """YaRN RoPE (rope.scaling.factor 4, original context 65536, the reference's ext 1 / attn 1 / beta 32, 1):
    q within 1e-5 of the oracle's fp64 YaRN; factor 1 is bitwise the plain-RoPE entry point"""
    t_ = torch()
    max_ctx, p0, base, eps, orig = 1 << 18, 150001, 1e7, 1e-6, 65536.0
    q3 = orc.normal(ntok * Q3, seed=960)
    qn = (1 + orc.normal(HD, seed=961, std=0.1)).astype(np.float32)
    kn = (1 + orc.normal(HD, seed=962, std=0.1)).astype(np.float32)
    kc = t_.zeros(max_ctx * NKV * HD, dtype=t_.int16, device="cuda:0")
    vc = t_.zeros(max_ctx * NKV * HD, dtype=t_.int16, device="cuda:0")
    qo = empty(ntok * NH * HD)
    dpos = dev(np.array([p0], np.int32))
    rmi.attn_prep_rope(dev(q3), Q3, dev(qn), dev(kn), kc, vc, dpos, qo, NH, NKV, HD, 64, base, factor, orig, eps, ntok,
                       max_ctx)
    qh = host(qo)
    for t in range(ntok):
        src = q3[t * Q3:(t + 1) * Q3]
        qx = np.concatenate([src[h * 2 * HD:h * 2 * HD + HD] for h in range(NH)])
        qref = orc.rope_yarn(orc.rms_norm_heads(qx, qn, NH, HD, eps), NH, HD, 64, p0 + t, base, factor, orig)
        assert_close_rel(qh[t * NH * HD:(t + 1) * NH * HD], qref, rtol=1e-5, atol_frac=2e-6, what=f"q t{t}")
    if factor == 1.0:
        qo2 = empty(ntok * NH * HD)
        rmi.attn_prep(dev(q3), Q3, dev(qn), dev(kn), kc, vc, dpos, qo2, NH, NKV, HD, 64, base, eps, ntok, max_ctx)
        assert np.array_equal(host(qo2).view(np.uint32), qh.view(np.uint32))


@pytest.mark.parametrize("factor", [1.0, 4.0])
def test_standalone_norm_and_rope_match_oracle_and_attn_prep(orc, rmi, factor):
    """the reference's separate calls (rms_norm_weighted qw:971-975, then native_rope_apply in place qw:1542-1544, each
    head at its own device position, as dpos_b holds per-head positions at qw:2380): within 1e-5 of the oracle's
    RMSNorm + RoPE / YaRN, and bitwise attn_prep's fused q (same norm tree, same rotation)"""
    max_ctx, p0, base, eps, orig, ntok = 1 << 18, 150001, 1e7, 1e-6, 65536.0, 2
    q3 = orc.normal(ntok * Q3, seed=970)
    qn = (1 + orc.normal(HD, seed=971, std=0.1)).astype(np.float32)
    kn = (1 + orc.normal(HD, seed=972, std=0.1)).astype(np.float32)
    qx = np.concatenate([q3[t * Q3 + h * 2 * HD:t * Q3 + h * 2 * HD + HD] for t in range(ntok) for h in range(NH)])
    x = dev(qx)
    rmi.rms_norm_weighted(x, dev(qn), ntok * NH, HD, eps)
    normed = host(x).copy()
    pos = dev(np.repeat(np.arange(p0, p0 + ntok, dtype=np.int32), NH))
    rmi.native_rope_apply(x, x, ntok * NH, HD, 64, pos, base, factor, orig)
    got = host(x)
    for t in range(ntok):
        sl = slice(t * NH * HD, (t + 1) * NH * HD)
        nref = orc.rms_norm_heads(qx[sl], qn, NH, HD, eps)
        assert_close_rel(normed[sl], nref, rtol=1e-6, atol_frac=1e-7, what=f"norm t{t}")
        rope = (orc.rope_yarn(nref, NH, HD, 64, p0 + t, base, factor, orig) if factor > 1 else
                orc.rope_neox(nref, NH, HD, 64, p0 + t, base))
        assert_close_rel(got[sl], rope, rtol=1e-5, atol_frac=2e-6, what=f"rope t{t}")
    t_ = torch()
    kc = t_.zeros(max_ctx * NKV * HD, dtype=t_.int16, device="cuda:0")
    vc = t_.zeros(max_ctx * NKV * HD, dtype=t_.int16, device="cuda:0")
    qo = empty(ntok * NH * HD)
    rmi.attn_prep_rope(dev(q3), Q3, dev(qn), dev(kn), kc, vc, dev(np.array([p0], np.int32)), qo, NH, NKV, HD, 64, base,
                       factor, orig, eps, ntok, max_ctx)
    assert np.array_equal(host(qo).view(np.uint32), got.view(np.uint32))
    # out of place: y gets the rotation, dims past n_rot copied, x untouched
    y = empty(ntok * NH * HD)
    xin = dev(normed)
    rmi.native_rope_apply(xin, y, ntok * NH, HD, 64, pos, base, factor, orig)
    assert np.array_equal(host(y).view(np.uint32), got.view(np.uint32))
    assert np.array_equal(host(xin).view(np.uint32), normed.view(np.uint32))


def test_elementwise_inplace(orc, rmi):
    """add_inplace (x += y), scale_inplace (x *= s), silu_inplace against numpy fp32 (the --split path's glue)"""
    n = 4096 + 37
    a, b = orc.normal(n, seed=980), orc.normal(n, seed=981)
    x = dev(a)
    rmi.add_inplace(x, dev(b), n)
    assert np.array_equal(host(x), a + b)
    rmi.scale_inplace(x, n, 0.0883883476)
    assert np.array_equal(host(x), (a + b) * np.float32(0.0883883476))
    x = dev(a)
    rmi.silu_inplace(x, n)
    ref = a.astype(np.float64) / (1 + np.exp(-a.astype(np.float64)))
    assert_close_rel(host(x), ref, rtol=1e-6, atol_frac=1e-7, what="silu")


@pytest.mark.parametrize("ctx,nsub,p0,ntok,factor", [(4096, 2, 4096 - 300, 2, 1.0), (4096, 2, 255, 2, 1.0),
                                                     (65536, 16, 65536 - 700, 2, 1.0), (320, 1, 0, 2, 1.0),
                                                     (66048, 17, 65279, 2, 1.0),
                                                     (4096, 2, 1000, 1, 1.0), (8192, 2, 5000, 2, 4.0)])
def test_flash_decode_prep_bitwise_equals_prep_then_flash(orc, rmi, ctx, nsub, p0, ntok, factor):
    """rmi_gqa_flash_decode_prep (attn_prep folded into the partial) against rmi_attn_prep_rope followed by
    rmi_gqa_flash_decode on copies of the same caches: y and Q8_1 bitwise, and the caches bitwise after the call (the
    new K / V rows written, nothing else).  p0 = 255 puts the verify pair on both sides of a 128-position chunk
    boundary; p0 = 0 is a context of one position; factor 4 is YaRN."""
    t_ = torch()
    kc, vc = kv_cache(orc, ctx, seed=ctx + p0)
    q3 = orc.normal(ntok * Q3, seed=p0 + 990)
    qn = (1 + orc.normal(HD, seed=991, std=0.1)).astype(np.float32)
    kn = (1 + orc.normal(HD, seed=992, std=0.1)).astype(np.float32)
    dq3, dqn, dkn, dpos = dev(q3), dev(qn), dev(kn), dev(np.array([p0], np.int32))
    ka, va, kb, vb = dev(kc), dev(vc), dev(kc), dev(vc)
    ws = empty(rmi.gqa_workspace_bytes(ctx, NKV, nsub), "uint8")
    qo = empty(ntok * NH * HD)
    rmi.attn_prep_rope(dq3, Q3, dqn, dkn, ka, va, dpos, qo, NH, NKV, HD, 64, 1e7, factor, 4096.0, 1e-6, ntok, ctx)
    ya, q8a = empty(ntok * NH * HD), empty(ntok * NH * HD // 32 * 36, "uint8")
    rmi.gqa_flash_decode(qo, ka, va, dpos, dq3, Q3, ya, NH * HD, q8a, NH * HD // 32 * 36, ws, NH, NKV, HD, ntok, ctx,
                         nsub, SCALE)
    ws2 = empty(rmi.gqa_workspace_bytes(ctx, NKV, nsub), "uint8")
    yb, q8b = empty(ntok * NH * HD), empty(ntok * NH * HD // 32 * 36, "uint8")
    rmi.gqa_flash_decode_prep(dq3, Q3, dqn, dkn, kb, vb, dpos, yb, NH * HD, q8b, NH * HD // 32 * 36, ws2, NH, NKV, HD,
                              64, 1e7, factor, 4096.0, 1e-6, ntok, ctx, nsub, SCALE)
    t_.cuda.synchronize()
    assert np.array_equal(host(yb).view(np.uint32), host(ya).view(np.uint32))
    assert np.array_equal(host(q8b), host(q8a))
    assert np.array_equal(host(kb), host(ka)) and np.array_equal(host(vb), host(va))


@pytest.mark.parametrize("ctx,nsub,p0,ntok,factor", [(4096, 2, 4096 - 300, 2, 1.0), (4096, 2, 1000, 1, 1.0),
                                                     (66048, 17, 65279, 2, 1.0), (8192, 2, 5000, 2, 4.0),
                                                     (320, 1, 0, 2, 1.0)])
def test_flash_decode_prep_rope_table_bitwise(orc, rmi, ctx, nsub, p0, ntok, factor):
    """rmi_gqa_flash_decode_prep_rt as a forward pass runs it: layer A in table mode 1 (computes its rotation and stores
    the table), then layer B (other rows, weights and caches, same positions) in mode 2 (loads the table).  Both
    bitwise the table-free call on copies of the same inputs (y, Q8_1, the caches after the call); the table holds the
    (cos, sin) of the fp64 angle at pos + t, within 1e-6 of numpy's."""
    t_ = torch()
    half = 32
    table = empty(rmi.gqa_rope_table_bytes(64) // 4)
    assert rmi.gqa_rope_table_bytes(64) == 2 * half * 2 * 4
    dpos = dev(np.array([p0], np.int32))
    outs = {}
    for layer, mode in (("a", 1), ("b", 2)):
        seed = 1200 + (0 if layer == "a" else 50)
        kc, vc = kv_cache(orc, ctx, seed=seed)
        q3 = orc.normal(ntok * Q3, seed=seed + 1)
        qn = (1 + orc.normal(HD, seed=seed + 2, std=0.1)).astype(np.float32)
        kn = (1 + orc.normal(HD, seed=seed + 3, std=0.1)).astype(np.float32)
        dq3, dqn, dkn = dev(q3), dev(qn), dev(kn)
        res = []
        for m in (0, mode):
            k_, v_ = dev(kc), dev(vc)
            ws = empty(rmi.gqa_workspace_bytes(ctx, NKV, nsub), "uint8")
            y, q8 = empty(ntok * NH * HD), empty(ntok * NH * HD // 32 * 36, "uint8")
            rmi.gqa_flash_decode_prep_rt(dq3, Q3, dqn, dkn, k_, v_, dpos, y, NH * HD, q8, NH * HD // 32 * 36, ws, NH,
                                         NKV, HD, 64, 1e7, factor, 4096.0, 1e-6, ntok, ctx, nsub, SCALE, table, m)
            t_.cuda.synchronize()
            res.append((host(y).view(np.uint32), host(q8), host(k_), host(v_)))
        for a, b in zip(res[0], res[1]):
            assert np.array_equal(a, b), f"layer {layer}, table mode {mode}"
        outs[layer] = res[1]
    tab = host(table).reshape(2, half, 2)
    for t in range(ntok):
        i = np.arange(half)
        ang = (p0 + t) * np.power(1e7, -2.0 * i / 64)
        if factor > 1.0:
            continue   # the YaRN ramp is checked through the bitwise comparison above
        assert np.allclose(tab[t, :, 0], np.cos(ang), atol=1e-6) and np.allclose(tab[t, :, 1], np.sin(ang), atol=1e-6)
