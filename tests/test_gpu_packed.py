"""GPU parity of the packed Q6_K GEMV (caller-owned wave-tiled copy of the weights).

Bars: within 1e-3 relative of the oracle's fp64 GEMV (|err| <= 1e-3 |ref| + 1e-5 max|ref|); bitwise equal to the
drop-in entry points on the GGUF layout, which run the GGUF stream kernel at rows of 4096 / 8192 / 12288 and 16-row
tiles where the dispatcher picks them (same lane ownership and reduction tree); ncols = 2 columns bitwise equal to
ncols = 1; residual variant bitwise plain + res with partials = sum of the
4 rows' squares in row order (src/test_res.cpp:57-112).  Ragged n_out pads the last 4-row group with zeros.
At one or two columns, n_in = 4096 and 8192 run the split kernel (up to 16384 rows at 4096) or the stream kernel
(more rows, and n_in = 12288); the other shapes the pipelined loop kernel.  All must give the same bits.
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


def packed(rmi, w_dev, n_in, n_out):
    wp = empty(rmi.q6_k_packed_bytes(n_in, n_out), "uint8")
    rmi.q6_k_pack(w_dev, wp, n_in, n_out)
    return wp


# (n_in, n_out): config-1 shape, the GDN in-projection, a ragged count, the FFN down projection, the draft eh_proj
SHAPES = [(4096, 12288), (4096, 12352), (2048, 1001), (12288, 4096), (8192, 4096), (4096, 70)]


@pytest.mark.parametrize("n_in,n_out", SHAPES)
def test_packed_matches_oracle_and_columns(orc, rmi, n_in, n_out):
    w = orc.gen_q6k(n_out, n_in, seed=n_in + 3 * n_out)
    x = orc.normal(2 * n_in, seed=n_out + 1)
    xq = orc.quantize_q8_1(x, n_in, 2)
    wd, xd = dev(w), dev(xq)
    wp = packed(rmi, wd, n_in, n_out)
    y2 = empty(2 * n_out)
    rmi.native_q6_k_mmvq_packed(wp, xd, y2, n_in, n_out, 2)
    y2h = host(y2)
    ref = orc.q6k_gemv(w, xq, n_in, n_out, ncols=2)
    for c in range(2):
        assert_close_rel(y2h[c * n_out:(c + 1) * n_out], ref[c * n_out:(c + 1) * n_out], what=f"packed col {c}")
        y1 = empty(n_out)
        xc = dev(xq[c * (n_in // 32) * 36:(c + 1) * (n_in // 32) * 36])
        rmi.native_q6_k_mmvq_packed(wp, xc, y1, n_in, n_out, 1)
        assert np.array_equal(host(y1).view(np.uint32), y2h[c * n_out:(c + 1) * n_out].view(np.uint32))


def test_lm_head_shape_matches_oracle(orc, rmi):
    """the round's lm_head launch at its full shape (248320 x 4096 Q6_K, 834 MB, two columns: the stream kernel with
    two quads per wave on the packed copy, qw:1591-1597) and the drop-in entry point on the GGUF blocks, against the
    oracle's fp64 GEMV; columns bitwise the 1-column launch, both layouts bitwise equal"""
    n_in, n_out = 4096, 248320
    w = orc.gen_q6k(n_out, n_in, seed=248320)
    xq = orc.quantize_q8_1(orc.normal(2 * n_in, seed=4097), n_in, 2)
    ref = orc.q6k_gemv(w, xq, n_in, n_out, ncols=2)
    wd, xd = dev(w), dev(xq)
    wp = packed(rmi, wd, n_in, n_out)
    y2 = empty(2 * n_out)
    rmi.native_q6_k_mmvq_packed(wp, xd, y2, n_in, n_out, 2)
    y2h = host(y2)
    for c in range(2):
        assert_close_rel(y2h[c * n_out:(c + 1) * n_out], ref[c * n_out:(c + 1) * n_out], what=f"lm_head col {c}")
    y1 = empty(n_out)
    rmi.native_q6_k_mmvq_packed(wp, dev(xq[(n_in // 32) * 36:]), y1, n_in, n_out, 1)
    assert np.array_equal(host(y1).view(np.uint32), y2h[n_out:].view(np.uint32))
    del wp
    yg = empty(2 * n_out)
    rmi.native_q6_k_mmvq(wd, xd, yg, n_in, n_out, 2)
    assert np.array_equal(host(yg).view(np.uint32), y2h.view(np.uint32))


# n_in 4096: the split kernel (a quad's two chunks on two waves) up to 16384 rows, the stream kernel (two quads per
# wave) above, ragged at 33001; (2048, 1001) the pipelined loop kernel
@pytest.mark.parametrize("n_in,n_out", [(4096, 12352), (4096, 10240), (2048, 1001), (4096, 24576), (4096, 33001)])
def test_packed_bitwise_equals_16_row_tiles(orc, rmi, n_in, n_out):
    w = orc.gen_q6k(n_out, n_in, seed=7 * n_out)
    xq = orc.quantize_q8_1(orc.normal(2 * n_in, seed=n_in), n_in, 2)
    wd, xd = dev(w), dev(xq)
    wp = packed(rmi, wd, n_in, n_out)
    yp, yt = empty(2 * n_out), empty(2 * n_out)
    rmi.native_q6_k_mmvq_packed(wp, xd, yp, n_in, n_out, 2)
    rmi.native_q6_k_mmvq(wd, xd, yt, n_in, n_out, 2)     # the GGUF stream kernel (n_in 4096), 16-row tiles (2048)
    assert np.array_equal(host(yp).view(np.uint32), host(yt).view(np.uint32))


@pytest.mark.parametrize("n_in,n_out,ncols", [(12288, 4096, 2), (12288, 1001, 1), (4096, 4096, 1), (4096, 4096, 2),
                                              (8192, 1001, 2), (2048, 1001, 3), (4096, 520, 5)])
def test_packed_residual(orc, rmi, n_in, n_out, ncols):
    w = orc.gen_q6k(n_out, n_in, seed=n_out + ncols)
    xq = orc.quantize_q8_1(orc.normal(ncols * n_in, seed=n_in + 2), n_in, ncols)
    res = orc.normal(ncols * n_out, seed=n_out + 9)
    wd, xd = dev(w), dev(xq)
    wp = packed(rmi, wd, n_in, n_out)
    y0 = empty(ncols * n_out)
    rmi.native_q6_k_mmvq_packed(wp, xd, y0, n_in, n_out, ncols)
    y = dev(res.copy())                                   # y aliases res, as the engine calls it
    np_ = (n_out + 3) // 4
    part = empty(ncols * np_)
    rmi.native_q6_k_mmvq_packed_res_n(wp, xd, y, y, part, n_in, n_out, ncols)
    yh, ph = host(y), host(part)
    assert np.array_equal(yh.view(np.uint32), (host(y0) + res).view(np.uint32))
    for c in range(ncols):
        v = yh[c * n_out:(c + 1) * n_out]
        vp = np.zeros(4 * np_, np.float64)
        vp[:n_out] = v
        want = (vp.reshape(np_, 4) ** 2).sum(1)
        assert np.allclose(ph[c * np_:(c + 1) * np_], want, rtol=1e-6, atol=0), f"partials col {c}"


def test_packed_layout_roundtrip(orc, rmi):
    """the pack is a permutation of the GGUF bytes (plus zero padding): same multiset of bytes per wave tile set"""
    n_in, n_out = 2048, 6
    w = orc.gen_q6k(n_out, n_in, seed=5)
    wp = host(packed(rmi, dev(w), n_in, n_out))
    assert wp.size == 2 * 6720
    tile0 = wp[:6720]
    rows0 = w.reshape(n_out, -1)[:4].reshape(-1)
    assert np.array_equal(np.sort(tile0), np.sort(rows0))
    # lane l = 4 hb + r holds row r, half-block hb (block hb // 2, half hb % 2): ql unit u at u * 1024 + 16 l, qh unit
    # u at 4096 + u * 1024 + 16 l, the 8 sub-scales at 6144 + 8 l; block (r, b)'s d at 6656 + 2 (4 b + r)
    nb = n_in // 256
    for lane in (0, 1, 3, 4, 5, 31, 63):
        r, hb = lane % 4, lane // 4
        b, n = hb // 2, hb % 2
        blk = w[(r * nb + b) * 210:(r * nb + b + 1) * 210]
        for u in range(4):
            assert np.array_equal(tile0[u * 1024 + 16 * lane:u * 1024 + 16 * lane + 16], blk[64 * n + 16 * u:64 * n + 16 * u + 16])
        for u in range(2):
            o = 4096 + u * 1024 + 16 * lane
            assert np.array_equal(tile0[o:o + 16], blk[128 + 32 * n + 16 * u:128 + 32 * n + 16 * u + 16])
        assert np.array_equal(tile0[6144 + 8 * lane:6152 + 8 * lane], blk[192 + 8 * n:200 + 8 * n])
        assert np.array_equal(tile0[6656 + 2 * (4 * b + r):6658 + 2 * (4 * b + r)], blk[208:210])



@pytest.mark.parametrize("n_in,n_out", [(4096, 12352), (12288, 4096), (8192, 4096), (2048, 1001), (12288, 1001),
                                        (8192, 1001), (4096, 1001)])
@pytest.mark.parametrize("ncols", [16, 13, 8])
def test_packed_wide_passes_bitwise_equal_single_column(orc, rmi, n_in, n_out, ncols):
    """ingest widths: 16 / 8 columns in one weight pass (one 8-wave workgroup per CU, up to 160 KB of staged
    activations; rows of 8192 / 12288 at 16 columns in two K halves, the 4096-row outputs with a wave pair per quad,
    the row sums through LDS; ragged row counts), remainders in passes of up to 4; every column bitwise the ncols = 1
    result, residual variant bitwise plain + res"""
    w = orc.gen_q6k(n_out, n_in, seed=n_in + n_out + ncols)
    xq = orc.quantize_q8_1(orc.normal(ncols * n_in, seed=ncols + n_out), n_in, ncols)
    wd, xd = dev(w), dev(xq)
    wp = packed(rmi, wd, n_in, n_out)
    y = empty(ncols * n_out)
    rmi.native_q6_k_mmvq_packed(wp, xd, y, n_in, n_out, ncols)
    yh = host(y)
    xcol = (n_in // 32) * 36
    for c in range(ncols):
        y1 = empty(n_out)
        rmi.native_q6_k_mmvq_packed(wp, dev(xq[c * xcol:(c + 1) * xcol]), y1, n_in, n_out, 1)
        assert np.array_equal(host(y1).view(np.uint32), yh[c * n_out:(c + 1) * n_out].view(np.uint32)), f"column {c}"
    ref = orc.q6k_gemv(w, xq[:xcol], n_in, n_out, ncols=1)
    assert_close_rel(yh[:n_out], ref, what="wide col 0")
    res = orc.normal(ncols * n_out, seed=n_out + 5)
    yr = dev(res.copy())
    np_ = (n_out + 3) // 4
    part = empty(ncols * np_)
    rmi.native_q6_k_mmvq_packed_res_n(wp, xd, yr, yr, part, n_in, n_out, ncols)
    assert np.array_equal(host(yr).view(np.uint32), (yh + res).view(np.uint32))


def swiglu_perm(ff):
    """packed row p of the SwiGLU order -> source row of [up ff | gate ff]"""
    p = np.arange(2 * ff)
    g, j = p // 64, p % 64
    return np.where(j < 32, ff + 32 * g + j, 32 * g + j - 32)


@pytest.mark.parametrize("ff", [12288, 320])
def test_swiglu_pack_is_a_row_permutation(orc, rmi, ff):
    """a plain packed GEMV over the SwiGLU packing returns the natural rows in the SwiGLU order, bit for bit"""
    n_in = 4096
    w = orc.gen_q6k(2 * ff, n_in, seed=ff + 1)
    xq = orc.quantize_q8_1(orc.normal(3 * n_in, seed=5), n_in, 3)
    wd, xd = dev(w), dev(xq)
    wn = packed(rmi, wd, n_in, 2 * ff)
    ws = empty(rmi.q6_k_packed_bytes(n_in, 2 * ff), "uint8")
    rmi.q6_k_pack_swiglu(wd, ws, n_in, ff)
    yn, ys = empty(3 * 2 * ff), empty(3 * 2 * ff)
    rmi.native_q6_k_mmvq_packed(wn, xd, yn, n_in, 2 * ff, 3)
    rmi.native_q6_k_mmvq_packed(ws, xd, ys, n_in, 2 * ff, 3)
    yn, ys = host(yn).reshape(3, 2 * ff), host(ys).reshape(3, 2 * ff)
    assert np.array_equal(ys.view(np.uint32), yn[:, swiglu_perm(ff)].view(np.uint32))


@pytest.mark.parametrize("ff", [12288, 320])
@pytest.mark.parametrize("ncols", [1, 2])
def test_fused_swiglu_gemv_bitwise_equals_gemv_then_swiglu(orc, rmi, ff, ncols):
    """rmi_native_q6_k_swiglu_packed == packed GEMV + swiglu_quant (Q8_1 bytes), and the interleaved SwiGLU over the
    SwiGLU-order rows gives the same bytes"""
    n_in = 4096
    w = orc.gen_q6k(2 * ff, n_in, seed=7 * ff + ncols)
    xq = orc.quantize_q8_1(orc.normal(ncols * n_in, seed=ff), n_in, ncols)
    wd, xd = dev(w), dev(xq)
    wn = packed(rmi, wd, n_in, 2 * ff)
    ws = empty(rmi.q6_k_packed_bytes(n_in, 2 * ff), "uint8")
    rmi.q6_k_pack_swiglu(wd, ws, n_in, ff)
    ug = empty(ncols * 2 * ff)
    rmi.native_q6_k_mmvq_packed(wn, xd, ug, n_in, 2 * ff, ncols)
    qbytes = rmi.native_q8_1_bytes(ff, ncols)
    ref = empty(qbytes, "uint8")
    rmi.swiglu_quant(ug, ug[ff:], ref, ff, ncols, 2 * ff)
    fused = empty(qbytes, "uint8")
    rmi.native_q6_k_swiglu_packed(ws, xd, fused, n_in, ff, ncols)
    assert np.array_equal(host(fused), host(ref))
    ugs = empty(ncols * 2 * ff)
    rmi.native_q6_k_mmvq_packed(ws, xd, ugs, n_in, 2 * ff, ncols)
    inter = empty(qbytes, "uint8")
    rmi.swiglu_quant_interleaved(ugs, inter, ff, ncols)
    assert np.array_equal(host(inter), host(ref))
    # and the Q8_1 blocks hold silu(gate) * up of the oracle's GEMV within the quantizer's step
    yo = orc.q6k_gemv(w, xq, n_in, 2 * ff, ncols=ncols).reshape(ncols, 2 * ff).astype(np.float64)
    a = yo[:, ff:] / (1.0 + np.exp(-yo[:, ff:])) * yo[:, :ff]
    blk = host(fused).reshape(ncols, ff // 32, 36)
    d = blk[:, :, 0:2].copy().view(np.float16).astype(np.float64)[..., 0]
    q = blk[:, :, 4:].view(np.int8).astype(np.float64)
    deq = (q * d[..., None]).reshape(ncols, ff)
    assert np.all(np.abs(deq - a) <= 0.51 * np.repeat(d, 32, axis=1) + 1e-3 * np.abs(a) + 1e-6)


# the drop-in GGUF-layout entry points run the GGUF stream kernel at rows of 4096 / 8192 / 12288 (ragged n_out
# included) for 1-4 columns and in passes of 4 above; (2048, 1001) keeps the 16-row tiled kernel
@pytest.mark.parametrize("n_in,n_out", [(4096, 12352), (4096, 1001), (8192, 4096), (12288, 4096), (12288, 1001),
                                        (4096, 24576), (2048, 1001)])
@pytest.mark.parametrize("ncols", [1, 2, 3, 5])
def test_gguf_entry_points_bitwise_equal_packed(orc, rmi, n_in, n_out, ncols):
    """every column of rmi_native_q6_k_mmvq / _res_n on GGUF blocks is bitwise the packed kernel's single-column
    result on the same matrix, and the residual variant is bitwise plain + res with the packed kernel's partials"""
    w = orc.gen_q6k(n_out, n_in, seed=3 * n_in + n_out + ncols)
    xq = orc.quantize_q8_1(orc.normal(ncols * n_in, seed=n_out + 5 * ncols), n_in, ncols)
    res = orc.normal(ncols * n_out, seed=n_in + 17)
    wd, xd = dev(w), dev(xq)
    wp = packed(rmi, wd, n_in, n_out)
    y = empty(ncols * n_out)
    rmi.native_q6_k_mmvq(wd, xd, y, n_in, n_out, ncols)
    yr = dev(res.copy())                                  # y aliases res, as the reference engine calls it
    np_ = (n_out + 3) // 4
    part = empty(ncols * np_)
    rmi.native_q6_k_mmvq_res_n(wd, xd, yr, yr, part, n_in, n_out, ncols)
    yh, yrh, ph = host(y), host(yr), host(part)
    xcol = (n_in // 32) * 36
    for c in range(ncols):
        xc = dev(xq[c * xcol:(c + 1) * xcol])
        y1 = empty(n_out)
        rmi.native_q6_k_mmvq_packed(wp, xc, y1, n_in, n_out, 1)
        y1r = dev(res[c * n_out:(c + 1) * n_out].copy())
        p1 = empty(np_)
        rmi.native_q6_k_mmvq_packed_res_n(wp, xc, y1r, y1r, p1, n_in, n_out, 1)
        sl = slice(c * n_out, (c + 1) * n_out)
        assert np.array_equal(yh[sl].view(np.uint32), host(y1).view(np.uint32)), f"plain column {c}"
        assert np.array_equal(yrh[sl].view(np.uint32), host(y1r).view(np.uint32)), f"residual column {c}"
        assert np.array_equal(ph[c * np_:(c + 1) * np_].view(np.uint32), host(p1).view(np.uint32)), f"partials {c}"


def exact_q6k(n_out, n_in, seed):
    """Q6_K rows whose GEMV epilogue is exact in fp32: block scale d = 1, sub-scales in [-3, 3], codes 16..47 (every
    qh field 1 or 2, the ql nibbles free), so each output is an integer below 2^24 when the activations are bounded"""
    rng = np.random.default_rng(seed)
    nb = n_out * (n_in // 256)
    blk = np.empty((nb, 210), np.uint8)
    blk[:, :128] = rng.integers(0, 256, size=(nb, 128), dtype=np.uint8)
    f = rng.integers(1, 3, size=(nb, 64, 4), dtype=np.uint8)
    blk[:, 128:192] = f[..., 0] | (f[..., 1] << 2) | (f[..., 2] << 4) | (f[..., 3] << 6)
    blk[:, 192:208] = rng.integers(-3, 4, size=(nb, 16)).astype(np.int8).view(np.uint8)
    blk[:, 208:210] = np.array([1.0], np.float16).view(np.uint8)
    return blk.reshape(-1)


def exact_q8_1(n_in, ncols, bound, seed):
    """Q8_1 columns with d = 1 and codes in [-bound, bound] (the stored sum is the codes' sum)"""
    rng = np.random.default_rng(seed)
    nb = ncols * (n_in // 32)
    q = rng.integers(-bound, bound + 1, size=(nb, 32)).astype(np.int8)
    blk = np.empty((nb, 36), np.uint8)
    blk[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[:, 2:4] = q.astype(np.float32).sum(axis=1).astype(np.float16).view(np.uint8).reshape(nb, 2)
    blk[:, 4:] = q.view(np.uint8)
    return blk.reshape(-1)


@pytest.mark.parametrize("n_in,n_out", [(4096, 12352), (4096, 4096), (12288, 4096), (8192, 4096), (4096, 24576),
                                        (12288, 1001)])
@pytest.mark.parametrize("ncols", [1, 2, 8, 16])
def test_engine_gemvs_integer_exact(orc, rmi, n_in, n_out, ncols):
    """The engine's GEMV kernels themselves against the oracle's exact integer block dots (the closed form of the
    Q6_K x Q8_1 dot, pinned in tests/test_oracle.py): with every fp32 scale 1 and the sums below 2^24, each output is
    the integer sum of its row's block dots, bit for bit - the packed decode kernels (1 / 2 columns), the MFMA ingest
    kernel (8 / 16 columns), the GGUF-layout stream kernel and the residual variants; a wrong code, sub-scale or
    correction index changes an integer"""
    bound = min(63, (1 << 24) // ((n_in // 32) * 2 * 16 * 16 * 3))
    w = exact_q6k(n_out, n_in, seed=n_in + 7 * n_out)
    xq = exact_q8_1(n_in, ncols, bound, seed=ncols + n_out)
    xcol = (n_in // 32) * 36
    want = np.stack([orc.q6k_block_dots(w, xq[c * xcol:(c + 1) * xcol], n_in, n_out).astype(np.int64).sum(axis=1)
                     for c in range(ncols)])
    assert np.abs(want).max() < (1 << 24)
    want = want.astype(np.float32).reshape(-1)
    wd, xd = dev(w), dev(xq)
    wp = packed(rmi, wd, n_in, n_out)
    y = empty(ncols * n_out)
    rmi.native_q6_k_mmvq_packed(wp, xd, y, n_in, n_out, ncols)
    assert np.array_equal(host(y), want), "packed"
    yg = empty(ncols * n_out)
    rmi.native_q6_k_mmvq(wd, xd, yg, n_in, n_out, ncols)
    assert np.array_equal(host(yg), want), "GGUF layout"
    res = np.random.default_rng(n_out).integers(-1000, 1001, size=ncols * n_out).astype(np.float32)
    yr = dev(res.copy())
    part = empty(ncols * ((n_out + 3) // 4))
    rmi.native_q6_k_mmvq_packed_res_n(wp, xd, yr, yr, part, n_in, n_out, ncols)
    assert np.array_equal(host(yr), want + res), "packed residual"


@pytest.mark.parametrize("n_in,n_out", [(4096, 24576), (12288, 4096), (4096, 1001)])
@pytest.mark.parametrize("ncols", [1, 2, 5])
def test_registry_copy_behind_drop_in_entry_points(orc, rmi, n_in, n_out, ncols):
    """native_q6_k_pack's library-owned copy (mmvq:2930-2960, looked up by native_q6_k_mmvq at mmvq:3629): once the
    GGUF matrix is packed, rmi_native_q6_k_mmvq / _res_n on the same pointer and shape give bitwise the results of
    the GGUF-layout kernels; another shape on the same pointer keeps the GGUF kernels; unpack frees the copy"""
    w = orc.gen_q6k(n_out, n_in, seed=n_in + 7 * n_out + ncols)
    x = orc.normal(ncols * n_in, seed=n_out + 5)
    xq = orc.quantize_q8_1(x, n_in, ncols)
    r = orc.normal(ncols * n_out, seed=n_out + 6)
    wd, xd = dev(w), dev(xq)
    npart = ncols * ((n_out + 3) // 4)

    def run():
        y = empty(ncols * n_out)
        rmi.native_q6_k_mmvq(wd, xd, y, n_in, n_out, ncols)
        yr, pr = dev(r), empty(npart)
        rmi.native_q6_k_mmvq_res_n(wd, xd, yr, yr, pr, n_in, n_out, ncols)
        return host(y), host(yr), host(pr)

    base = run()
    n0 = rmi.native_q6_k_packed_copies()
    assert rmi.native_q6_k_pack(wd, n_in, n_out)
    assert rmi.native_q6_k_pack(wd, n_in, n_out)          # packed already: no second copy
    assert rmi.native_q6_k_packed_copies() == n0 + 1
    got = run()
    for a, b in zip(base, got):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    # the copy is keyed by pointer and shape: the first rows of the same matrix still run (on the GGUF kernels)
    rows = max(1, n_out // 2)
    y0, y1 = empty(rows), empty(rows)
    rmi.native_q6_k_mmvq(wd, xd, y1, n_in, rows, 1)
    rmi.native_q6_k_unpack(wd)
    assert rmi.native_q6_k_packed_copies() == n0
    rmi.native_q6_k_mmvq(wd, xd, y0, n_in, rows, 1)
    assert np.array_equal(host(y0).view(np.uint32), host(y1).view(np.uint32))
    got = run()                                            # after unpack: the GGUF kernels again, same bits
    for a, b in zip(base, got):
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    rmi.native_q6_k_unpack(wd)                             # no copy: a no-op


def test_registry_copy_shapes_it_does_not_take(orc, rmi):
    """n_in not a multiple of 2048: native_q6_k_pack returns False, as the reference does for shapes its packed kernel
    does not take, and the drop-in entry point keeps the GGUF kernels"""
    w = dev(orc.gen_q6k(64, 1024, seed=11))
    n0 = rmi.native_q6_k_packed_copies()
    assert not rmi.native_q6_k_pack(w, 1024, 64)
    assert rmi.native_q6_k_packed_copies() == n0
