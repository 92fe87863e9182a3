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
