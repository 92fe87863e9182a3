"""GPU parity of the norm / activation epilogues, argmax, the device embedding row and the Q8_0 GEMV.

Bars: Q8_1 outputs of a transcendental epilogue match the oracle's fp64 values within half a quantization step plus the
fp16 rounding of d and 1e-5 of the block maximum (q may differ by one at a boundary); fp32 outputs within 1e-5 relative; argmax,
embedding rows and partials of exact inputs bit-exact.
"""
import numpy as np
import pytest

from tests.gpu_util import assert_close_rel, dev, empty, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rmi():
    import rapier_amd
    rapier_amd.lib()
    return rapier_amd


def check_q8(orc, q8_bytes, ref, what):
    """Q8_1 bytes vs fp64 reference values, per block: |deq - ref| <= d/2 (rounding of q) + 127 d 2^-11 (the fp16
    rounding of d that deq multiplies by) + 1e-5 amax (the fp32 value itself)."""
    deq = orc.dequantize_q8_1(q8_bytes, ref.size).astype(np.float64).reshape(-1, 32)
    r = np.asarray(ref, np.float64).reshape(-1, 32)
    amax = np.abs(r).max(1, keepdims=True)
    d = amax / 127
    bad = np.abs(deq - r) > 0.5 * d + 127 * d * 2.0 ** -11 + 1e-5 * amax + 1e-30
    assert not bad.any(), f"{what}: {bad.sum()} elements outside the quantization bound"


def test_rms_quant_apply_two_columns(orc, rmi):
    cols, eps = 4096, 1e-6
    x = orc.normal(2 * cols, seed=1)
    w = (1 + orc.normal(cols, seed=2, std=0.1)).astype(np.float32)
    parts = np.concatenate([orc.row_sum_partials(x[:cols]), orc.row_sum_partials(x[cols:])]).astype(np.float32)
    y = empty(2 * cols // 32 * 36, "uint8")
    rmi.rms_quant_apply(dev(x), dev(w), dev(parts), y, cols, eps, ncols=2)
    yh = host(y)
    for c in range(2):
        inv = orc.rms_inv(parts[c * 1024:(c + 1) * 1024].astype(np.float64), cols, eps)
        ref = orc.rms_norm_out(x[c * cols:(c + 1) * cols], w, inv)
        check_q8(orc, yh[c * 4608:(c + 1) * 4608], ref, f"rms_quant_apply col {c}")
    # column 1 of the 2-column launch equals a 1-column launch on that column, bit for bit
    y1 = empty(4608, "uint8")
    rmi.rms_quant_apply(dev(x[cols:]), dev(w), dev(parts[1024:]), y1, cols, eps, ncols=1)
    assert np.array_equal(host(y1), yh[4608:])


def test_rms_quant_apply_pair_equals_two_norms_then_quantize(orc, rmi):
    """The draft's input (qwythos.cpp:1327-1332): [enorm(emb) | hnorm(h)] per column as one Q8_1 row of 2 cols, in
    one launch; bitwise the reference's two rms_norm_out calls into eh_cat and the quantize of eh_cat."""
    cols, eps, nc = 4096, 1e-6, 2
    e = orc.normal(nc * cols, seed=11)
    h = orc.normal(nc * cols, seed=12, std=3.0)
    we = (1 + orc.normal(cols, seed=13, std=0.1)).astype(np.float32)
    wh = (1 + orc.normal(cols, seed=14, std=0.1)).astype(np.float32)
    pe = np.concatenate([orc.row_sum_partials(e[c * cols:(c + 1) * cols]) for c in range(nc)]).astype(np.float32)
    ph = np.concatenate([orc.row_sum_partials(h[c * cols:(c + 1) * cols]) for c in range(nc)]).astype(np.float32)
    row = 2 * cols // 32 * 36
    y = empty(nc * row, "uint8")
    rmi.rms_quant_apply_pair(dev(e), dev(we), dev(pe), dev(h), dev(wh), dev(ph), y, cols, eps, ncols=nc)
    yh = host(y)
    cat = empty(nc * 2 * cols)
    rmi.rms_norm_out_strided(dev(e), dev(we), dev(pe), cat, 2 * cols, None, cols, eps, ncols=nc)
    rmi.rms_norm_out_strided(dev(h), dev(wh), dev(ph), cat[cols:], 2 * cols, None, cols, eps, ncols=nc)
    yq = empty(nc * row, "uint8")
    rmi.native_quantize_q8_1(cat, yq, 2 * cols, nc)
    assert np.array_equal(yh, host(yq))
    for c in range(nc):
        ref = np.concatenate([
            orc.rms_norm_out(x[c * cols:(c + 1) * cols], w, orc.rms_inv(p[c * 1024:(c + 1) * 1024].astype(np.float64),
                                                                        cols, eps))
            for x, w, p in ((e, we, pe), (h, wh, ph))])
        check_q8(orc, yh[c * row:(c + 1) * row], ref, f"rms_quant_apply_pair col {c}")


def test_rms_norm_out_and_partials(orc, rmi):
    cols, eps = 4096, 1e-6
    x = orc.normal(cols, seed=3)
    w = (1 + orc.normal(cols, seed=4, std=0.1)).astype(np.float32)
    parts = orc.row_sum_partials(x).astype(np.float32)
    out, op = empty(cols), empty(cols // 4)
    rmi.rms_norm_out(dev(x), dev(w), dev(parts), out, op, cols, eps)
    ref = orc.rms_norm_out(x, w, orc.rms_inv(parts.astype(np.float64), cols, eps))
    assert_close_rel(host(out), ref, rtol=1e-5, atol_frac=1e-6, what="rms_norm_out")
    o = host(out).astype(np.float64)
    np.testing.assert_allclose(host(op), (o.reshape(-1, 4) ** 2).sum(1), rtol=1e-6)


def test_row_sum_and_add_partials(orc, rmi):
    n = 4096
    x, o = orc.normal(2 * n, seed=5), orc.normal(2 * n, seed=6)
    p = empty(2 * n // 4)
    rmi.row_sum_partials(dev(x), p, n, ncols=2)
    np.testing.assert_allclose(host(p), (x.astype(np.float64).reshape(-1, 4) ** 2).sum(1), rtol=1e-6)
    dx = dev(x)
    rmi.add_partials(dx, dev(o), p, n, ncols=2)
    xs = (x + o).astype(np.float32)
    assert np.array_equal(host(dx), xs)
    np.testing.assert_allclose(host(p), (xs.astype(np.float64).reshape(-1, 4) ** 2).sum(1), rtol=1e-6)


def test_swiglu_and_sig_mul_quant(orc, rmi):
    n = 12288
    ug = orc.normal(2 * 2 * n, seed=7)            # two columns of [up n | gate n]
    y = empty(2 * n // 32 * 36, "uint8")
    rmi.swiglu_quant(dev(ug), dev(ug[n:]), y, n, ncols=2, col_stride=2 * n)
    yh = host(y)
    for c in range(2):
        up, gate = ug[c * 2 * n:c * 2 * n + n], ug[c * 2 * n + n:(c + 1) * 2 * n]
        check_q8(orc, yh[c * n // 32 * 36:(c + 1) * n // 32 * 36], orc.swiglu(up, gate), "swiglu")
    n2 = 4096
    o, g = orc.normal(n2, seed=8), orc.normal(n2, seed=9)
    y2 = empty(n2 // 32 * 36, "uint8")
    rmi.sig_mul_quant(dev(o), dev(g), y2, n2)
    check_q8(orc, host(y2), orc.sig_mul(o, g), "sig_mul")


def test_beta_gate(orc, rmi):
    n = 32
    ab = orc.normal(2 * 2 * n, seed=10)
    ab[2 * n + n:2 * n + n + 4] = 25.0     # softplus linear branch
    dt = orc.normal(n, seed=11, std=0.1)
    ssm_a = (-np.exp(orc.normal(n, seed=12, std=0.5))).astype(np.float32)
    dab, gg = dev(ab), empty(2 * n)
    rmi.beta_gate(dab, dev(dt), dev(ssm_a), gg, n, ncols=2)
    abh, ggh = host(dab), host(gg)
    for c in range(2):
        b, g = orc.beta_gate(ab[c * 2 * n:c * 2 * n + n], ab[c * 2 * n + n:(c + 1) * 2 * n], dt, ssm_a)
        assert_close_rel(abh[c * 2 * n:c * 2 * n + n], b, rtol=1e-5, atol_frac=1e-7, what="beta")
        assert_close_rel(ggh[c * n:(c + 1) * n], g, rtol=1e-5, atol_frac=1e-7, what="gate")


@pytest.mark.parametrize("n", [248320, 1000, 1])
def test_argmax_ties_lowest_index(orc, rmi, n):
    l = orc.normal(2 * n, seed=n)
    if n > 10:
        l[[77, 500, n - 1]] = 9.0           # column 0: a three-way tie -> 77
        l[n + n - 1] = 9.5                  # column 1: the last element
        l[n + 3] = 9.5                      # ... tied with an earlier one -> 3
    ws = empty(rmi.argmax_workspace_bytes(2), "uint8")
    out = empty(2, "int32")
    rmi.argmax(dev(l), n, out, ws, ncols=2, col_stride=n)
    got = host(out)
    assert got[0] == orc.argmax(l[:n]) and got[1] == orc.argmax(l[n:])
    if n > 10:
        assert got[0] == 77 and got[1] == 3


def test_embed_q6_k_rows(orc, rmi):
    n_embd, n_vocab = 4096, 300
    emb = orc.gen_q6k(n_vocab, n_embd, seed=13)
    toks = np.array([7, 299], dtype=np.int32)
    x, p = empty(2 * n_embd), empty(2 * n_embd // 4)
    rmi.embed_q6_k(dev(emb), dev(toks), x, p, n_embd, n_vocab, ncols=2)
    deq = orc.q6k_dequant(emb, n_vocab, n_embd)
    xh = host(x).reshape(2, n_embd)
    assert np.array_equal(xh[0], deq[7]) and np.array_equal(xh[1], deq[299])
    np.testing.assert_allclose(host(p), (xh.astype(np.float64).reshape(-1, 4) ** 2).sum(1), rtol=1e-6)


@pytest.mark.parametrize("ggml_type", [13, 12])
def test_embed_k_quant_rows(orc, rmi, ggml_type):
    """Q5_K / Q4_K token_embd tables (Q5_K_M files): rows bit-exact vs the oracle's ggml dequant, ids clamped"""
    from tests.kquant import k_blocks
    n_embd, n_vocab = 1024, 40
    emb, _ = k_blocks(np.random.default_rng(ggml_type), n_vocab * n_embd // 256, ggml_type == 13)
    toks = np.array([0, 39, 17, 1000], dtype=np.int32)          # 1000 is clamped to the last row
    x, p = empty(4 * n_embd), empty(4 * n_embd // 4)
    rmi.embed(ggml_type, dev(emb), dev(toks), x, p, n_embd, n_vocab, ncols=4)
    deq = (orc.q5k_dequant if ggml_type == 13 else orc.q4k_dequant)(emb, n_vocab, n_embd).reshape(n_vocab, n_embd)
    xh = host(x).reshape(4, n_embd)
    for c, t in enumerate([0, 39, 17, 39]):
        assert np.array_equal(xh[c], deq[t]), f"column {c}"
    np.testing.assert_allclose(host(p), (xh.astype(np.float64).reshape(-1, 4) ** 2).sum(1), rtol=1e-6)


@pytest.mark.parametrize("n_in,n_out,ncols", [(4096, 1000, 1), (4096, 257, 2), (1024, 64, 5)])
def test_q8_0_gemv(orc, rmi, n_in, n_out, ncols):
    w = orc.gen_q8_0(n_out, n_in, seed=n_out)
    xq = orc.quantize_q8_1(orc.normal(ncols * n_in, seed=n_in), n_in, ncols)
    y = empty(ncols * n_out)
    dw, dxq = dev(w), dev(xq)        # keep the device copies alive until the kernel has run
    rmi._call("rmi_native_mmvq", 8, rmi._p(dw), rmi._p(dxq), rmi._p(y), n_in, n_out, ncols, rmi._stream(None))
    assert_close_rel(host(y), orc.q8_0_gemv(w, xq, n_in, n_out, ncols=ncols), what="q8_0")
    res = orc.normal(n_out, seed=3)
    yr, pr = dev(res), empty((n_out + 3) // 4)
    dx1 = dev(xq[:n_in // 32 * 36])
    rmi._call("rmi_native_q8_0_mmvq_res", rmi._p(dw), rmi._p(dx1), rmi._p(yr), rmi._p(yr), rmi._p(pr), n_in, n_out,
              rmi._stream(None))
    ref, pref = orc.q8_0_gemv(w, xq[:n_in // 32 * 36], n_in, n_out, res=res, partials=True)
    assert_close_rel(host(yr), ref, what="q8_0 res")
    assert_close_rel(host(pr), pref, rtol=1e-5, atol_frac=1e-6, what="q8_0 partials")


@pytest.mark.parametrize("n_in,n_out,ncols", [(4096, 1000, 2), (12288, 257, 1)])
def test_q8_0_gemv_integer_exact(orc, rmi, n_in, n_out, ncols):
    """the Q8_0 GEMV on blocks whose every fp32 step is exact (weight and activation scales 1, codes bounded so the
    sums stay below 2^24): bitwise the oracle's exact-integer fp64 GEMV, plain and with the residual"""
    rng = np.random.default_rng(n_in + n_out)
    nb = n_out * (n_in // 32)
    wb = np.empty((nb, 34), np.uint8)
    wb[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    wb[:, 2:] = rng.integers(-127, 128, size=(nb, 32)).astype(np.int8).view(np.uint8)
    w = wb.reshape(-1)
    bound = min(63, (1 << 24) // (n_in * 127))
    xb = np.empty((ncols * (n_in // 32), 36), np.uint8)
    q = rng.integers(-bound, bound + 1, size=(xb.shape[0], 32)).astype(np.int8)
    xb[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    xb[:, 2:4] = q.astype(np.float32).sum(axis=1).astype(np.float16).view(np.uint8).reshape(-1, 2)
    xb[:, 4:] = q.view(np.uint8)
    xq = xb.reshape(-1)
    ref = orc.q8_0_gemv(w, xq, n_in, n_out, ncols=ncols)
    assert np.all(ref == np.round(ref)) and np.abs(ref).max() < (1 << 24)
    y = empty(ncols * n_out)
    dw, dxq = dev(w), dev(xq)
    rmi._call("rmi_native_mmvq", 8, rmi._p(dw), rmi._p(dxq), rmi._p(y), n_in, n_out, ncols, rmi._stream(None))
    assert np.array_equal(host(y), ref.astype(np.float32))
    res = rng.integers(-1000, 1001, size=n_out).astype(np.float32)
    yr, pr = dev(res.copy()), empty((n_out + 3) // 4)
    dx1 = dev(xq[:n_in // 32 * 36])
    rmi._call("rmi_native_q8_0_mmvq_res", rmi._p(dw), rmi._p(dx1), rmi._p(yr), rmi._p(yr), rmi._p(pr), n_in, n_out,
              rmi._stream(None))
    assert np.array_equal(host(yr), ref[:n_out].astype(np.float32) + res)


@pytest.mark.parametrize("cols,ncols", [(4096, 2), (12288, 1), (8192, 3)])
def test_rms_quant_apply_self_equals_partials_then_norm(orc, rmi, cols, ncols):
    """rmi_rms_quant_apply_self (the partials formed in the workgroup) == rmi_row_sum_partials then
    rmi_rms_quant_apply, Q8_1 bytes"""
    x = orc.normal(ncols * cols, seed=cols + ncols)
    x[:32] *= 1e4
    w = (1 + orc.normal(cols, seed=9, std=0.1)).astype(np.float32)
    xd, wd = dev(x), dev(w)
    part = empty(ncols * (cols // 4))
    rmi.row_sum_partials(xd, part, cols, ncols)
    ref = empty(rmi.native_q8_1_bytes(cols, ncols), "uint8")
    rmi.rms_quant_apply(xd, wd, part, ref, cols, 1e-6, ncols)
    got = empty(rmi.native_q8_1_bytes(cols, ncols), "uint8")
    rmi.rms_quant_apply_self(xd, wd, got, cols, 1e-6, ncols)
    assert np.array_equal(host(got), host(ref))


@pytest.mark.parametrize("ggml_type,cols,ncols", [(14, 4096, 2), (14, 4096, 1), (13, 1024, 3), (12, 2048, 2)])
def test_embed_quant_apply_pair_equals_embed_then_pair(orc, rmi, ggml_type, cols, ncols):
    """rmi_embed_quant_apply_pair (the embedding rows dequantized and their partials formed in the norm's workgroups)
    == rmi_embed then rmi_rms_quant_apply_pair, Q8_1 bytes; an out-of-range id clamps as in rmi_embed"""
    from tests.kquant import k_blocks
    n_vocab = 50
    if ggml_type == 14:
        emb = orc.gen_q6k(n_vocab, cols, seed=cols)
    else:
        emb, _ = k_blocks(np.random.default_rng(cols), n_vocab * cols // 256, ggml_type == 13)
    toks = np.array([3, 49, 1000][:ncols], dtype=np.int32)
    h = orc.normal(ncols * cols, seed=ncols, std=3.0)
    we = (1 + orc.normal(cols, seed=13, std=0.1)).astype(np.float32)
    wh = (1 + orc.normal(cols, seed=14, std=0.1)).astype(np.float32)
    ph = np.concatenate([orc.row_sum_partials(h[c * cols:(c + 1) * cols]) for c in range(ncols)]).astype(np.float32)
    ed, td, hd, wed, whd, phd = dev(emb), dev(toks), dev(h), dev(we), dev(wh), dev(ph)
    x, p = empty(ncols * cols), empty(ncols * cols // 4)
    rmi.embed(ggml_type, ed, td, x, p, cols, n_vocab, ncols)
    ref = empty(ncols * 2 * cols // 32 * 36, "uint8")
    rmi.rms_quant_apply_pair(x, wed, p, hd, whd, phd, ref, cols, 1e-6, ncols=ncols)
    got = empty(ncols * 2 * cols // 32 * 36, "uint8")
    rmi.embed_quant_apply_pair(ggml_type, ed, td, wed, hd, whd, phd, got, cols, n_vocab, 1e-6, ncols)
    assert np.array_equal(host(got), host(ref))
