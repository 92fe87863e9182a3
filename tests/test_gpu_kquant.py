"""GPU parity of the Q4_K / Q5_K x Q8_1 GEMVs (the matrices of Q5_K_M files; mmvq:185-300, 562-640, residual
3202-3324).  Bars (written here): within 1e-3 relative of the oracle's exact-integer fp64 GEMV (|err| <= 1e-3 |ref| +
1e-5 max|ref|); every column of an ncols >= 2 call bitwise the ncols = 1 result; the residual variant bitwise
plain + res with partials = sum of each 4 rows' squares (within 1e-6 relative of an fp64 recomputation)."""
import numpy as np
import pytest

from tests.gpu_util import assert_close_rel, dev, empty, host
from tests.kquant import k_blocks

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rmi():
    import rapier_amd
    rapier_amd.lib()
    return rapier_amd


# (n_in, n_out): the 9B in-projection and FFN shapes, a ragged row count, the down projection, a short row
SHAPES = [(4096, 1000), (4096, 12352), (2048, 257), (12288, 4096), (256, 70)]


@pytest.mark.parametrize("ggml_type", [12, 13])
@pytest.mark.parametrize("n_in,n_out", SHAPES)
def test_kquant_gemv_matches_oracle(orc, rmi, ggml_type, n_in, n_out):
    rng = np.random.default_rng(n_in + n_out + ggml_type)
    w, _ = k_blocks(rng, n_out * n_in // 256, ggml_type == 13)
    ncols = 3
    xq = orc.quantize_q8_1(orc.normal(ncols * n_in, seed=n_out), n_in, ncols)
    wd, xd = dev(w), dev(xq)
    y = empty(ncols * n_out)
    rmi.native_kquant_mmvq(ggml_type, wd, xd, y, n_in, n_out, ncols)
    yh = host(y)
    ref = (orc.q5k_gemv if ggml_type == 13 else orc.q4k_gemv)(w, xq, n_in, n_out, ncols=ncols)
    for c in range(ncols):
        assert_close_rel(yh[c * n_out:(c + 1) * n_out], ref[c * n_out:(c + 1) * n_out], what=f"type {ggml_type} col {c}")
        y1 = empty(n_out)
        xc = dev(xq[c * (n_in // 32) * 36:(c + 1) * (n_in // 32) * 36])
        rmi.native_kquant_mmvq(ggml_type, wd, xc, y1, n_in, n_out, 1)
        assert np.array_equal(host(y1).view(np.uint32), yh[c * n_out:(c + 1) * n_out].view(np.uint32))
    # through the type dispatcher
    y2 = empty(ncols * n_out)
    rmi._call("rmi_native_mmvq", ggml_type, rmi._p(wd), rmi._p(xd), rmi._p(y2), n_in, n_out, ncols, rmi._stream(None))
    assert np.array_equal(host(y2).view(np.uint32), yh.view(np.uint32))


@pytest.mark.parametrize("ggml_type", [12, 13])
@pytest.mark.parametrize("n_in,n_out,ncols", [(12288, 4096, 2), (4096, 1001, 1), (2048, 520, 6)])
def test_kquant_gemv_residual(orc, rmi, ggml_type, n_in, n_out, ncols):
    rng = np.random.default_rng(7 * n_out + ggml_type)
    w, _ = k_blocks(rng, n_out * n_in // 256, ggml_type == 13)
    xq = orc.quantize_q8_1(orc.normal(ncols * n_in, seed=n_in + 5), n_in, ncols)
    res = orc.normal(ncols * n_out, seed=n_out + 11)
    wd, xd = dev(w), dev(xq)
    y0 = empty(ncols * n_out)
    rmi.native_kquant_mmvq(ggml_type, wd, xd, y0, n_in, n_out, ncols)
    y = dev(res.copy())                                  # y aliases res, as the engine calls it
    np_ = (n_out + 3) // 4
    part = empty(ncols * np_)
    rmi.native_kquant_mmvq_res_n(ggml_type, wd, xd, y, y, part, n_in, n_out, ncols)
    yh, ph = host(y), host(part)
    assert np.array_equal(yh.view(np.uint32), (host(y0) + res).view(np.uint32))
    for c in range(ncols):
        v = np.zeros(4 * np_, np.float64)
        v[:n_out] = yh[c * n_out:(c + 1) * n_out]
        assert np.allclose(ph[c * np_:(c + 1) * np_], (v.reshape(np_, 4) ** 2).sum(1), rtol=1e-6, atol=0)


def exact_k_blocks(rng, nblocks, five_bit):
    """K-quant blocks whose GEMV epilogue is exact in fp32: d = dmin = 1, six-bit scales and mins in 0..3, codes free
    (vectorized form of tests/kquant.py's packing)"""
    from tests.kquant import pack_k_scales
    q = rng.integers(0, 32 if five_bit else 16, size=(nblocks, 256))
    sc = rng.integers(0, 4, size=(nblocks, 8))
    mn = rng.integers(0, 4, size=(nblocks, 8))
    head = np.empty((nblocks, 16), np.uint8)
    head[:, 0:4] = np.array([1.0, 1.0], np.float16).view(np.uint8)
    scales = np.stack([pack_k_scales(sc[b], mn[b]) for b in range(min(nblocks, 64))])
    # the scale bytes of every block from the 64 packed patterns above (the packing is per block, the values repeat)
    pick = rng.integers(0, scales.shape[0], size=nblocks)
    head[:, 4:16] = scales[pick]
    sc, mn = sc[pick], mn[pick]
    qq = q.reshape(nblocks, 4, 2, 32)                       # [block][pair c][half h][lane l]: element 64 c + 32 h + l
    qs = ((qq[:, :, 0, :] & 15) | ((qq[:, :, 1, :] & 15) << 4)).astype(np.uint8).reshape(nblocks, 128)
    if five_bit:
        bits = (q.reshape(nblocks, 8, 32) >> 4) & 1          # [block][sub-block j][lane l]
        qh = np.zeros((nblocks, 32), np.uint8)
        for j in range(8):
            qh |= (bits[:, j, :] << j).astype(np.uint8)
        return np.concatenate([head, qh, qs], axis=1).reshape(-1)
    return np.concatenate([head, qs], axis=1).reshape(-1)


def exact_q8_1(n_in, ncols, bound, seed):
    rng = np.random.default_rng(seed)
    nb = ncols * (n_in // 32)
    q = rng.integers(-bound, bound + 1, size=(nb, 32)).astype(np.int8)
    blk = np.empty((nb, 36), np.uint8)
    blk[:, 0:2] = np.array([1.0], np.float16).view(np.uint8)
    blk[:, 2:4] = q.astype(np.float32).sum(axis=1).astype(np.float16).view(np.uint8).reshape(nb, 2)
    blk[:, 4:] = q.view(np.uint8)
    return blk.reshape(-1)


@pytest.mark.parametrize("ggml_type", [12, 13])
@pytest.mark.parametrize("n_in,n_out,ncols", [(4096, 1000, 2), (12288, 513, 1), (4096, 700, 6)])
def test_kquant_gemv_integer_exact(orc, rmi, ggml_type, n_in, n_out, ncols):
    """the K-quant GEMV kernels on blocks whose every fp32 step is exact (d = dmin = 1, scales and mins 0..3, Q8_1
    scales 1, code sums exact in fp16, sums below 2^24): each output equals the oracle's exact-integer fp64 GEMV bit for
    bit - the codes, the fifth bit, the 6-bit scale / min unpacking and the min term, with no tolerance"""
    rng = np.random.default_rng(n_in + n_out + ggml_type)
    w = exact_k_blocks(rng, n_out * n_in // 256, ggml_type == 13)
    bound = min(63, (1 << 24) // ((n_in // 32) * 3 * 32 * 31 + (n_in // 32) * 3 * 32))
    xq = exact_q8_1(n_in, ncols, bound, seed=n_out)
    ref = (orc.q5k_gemv if ggml_type == 13 else orc.q4k_gemv)(w, xq, n_in, n_out, ncols=ncols)
    assert np.all(ref == np.round(ref)) and np.abs(ref).max() < (1 << 24)
    y = empty(ncols * n_out)
    rmi.native_kquant_mmvq(ggml_type, dev(w), dev(xq), y, n_in, n_out, ncols)
    assert np.array_equal(host(y), ref.astype(np.float32))
