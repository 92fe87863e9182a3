"""GPU parity of the Q8_1 quantizer and the Q6_K x Q8_1 GEMVs against the oracle.

Bars: integer block dots and Q8_1 bytes bit-exact; fp32 GEMV outputs within 1e-3 relative of the oracle's fp64
result (|err| <= 1e-3 |ref| + 1e-5 max|ref|); ncols = 2 columns bitwise equal to ncols = 1 (mmvq:902-920);
residual variant bitwise equal to plain + res, partials = sum of the 4 rows' squares (src/test_res.cpp:57-112).
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


def _case(orc, n_out, n_in, seed, ncols=1):
    w = orc.gen_q6k(n_out, n_in, seed=seed)
    x = orc.normal(ncols * n_in, seed=seed + 1)
    xq = orc.quantize_q8_1(x, n_in, ncols)
    return w, x, xq


@pytest.mark.parametrize("n_in,ncols", [(4096, 1), (4096, 2), (12288, 2), (256, 3)])
def test_quantize_q8_1_bit_exact(orc, rmi, n_in, ncols):
    x = orc.normal(n_in * ncols, seed=n_in + ncols)
    x[32:64] *= 1e4          # finite-guard block: |sum| saturates to 65504
    x[96:128] = 0.0
    dq = empty(rmi.native_q8_1_bytes(n_in, ncols), "uint8")
    rmi.native_quantize_q8_1(dev(x), dq, n_in, ncols)
    assert np.array_equal(host(dq), orc.quantize_q8_1(x, n_in, ncols))


@pytest.mark.parametrize("n_in,n_out", [(256, 1), (512, 33), (2048, 16), (4096, 70)])
def test_block_dots_bit_exact(orc, rmi, n_in, n_out):
    w, _, xq = _case(orc, n_out, n_in, seed=n_in * 7 + n_out)
    out = empty(n_out * (n_in // 32), "int32")
    rmi.q6_k_block_dots(dev(w), dev(xq), out, n_in, n_out)
    assert np.array_equal(host(out).reshape(n_out, -1), orc.q6k_block_dots(w, xq, n_in, n_out))


# shapes: the config-1 matrix, the generic path (n_in % 2048 != 0), ragged n_out on both tiled widths
SHAPES = [(4096, 12288), (512, 37), (2304, 9), (2048, 1000), (4096, 100), (12288, 4096), (8192, 4096)]


@pytest.mark.parametrize("n_in,n_out", SHAPES)
def test_gemv_ncols1_matches_oracle(orc, rmi, n_in, n_out):
    w, _, xq = _case(orc, n_out, n_in, seed=n_out + n_in)
    y = empty(n_out)
    rmi.native_q6_k_mmvq(dev(w), dev(xq), y, n_in, n_out, 1)
    assert_close_rel(host(y), orc.q6k_gemv(w, xq, n_in, n_out), what=f"q6k {n_out}x{n_in}")


@pytest.mark.parametrize("n_in,n_out", SHAPES)
def test_gemv_ncols2_columns_bitwise_equal_ncols1(orc, rmi, n_in, n_out):
    w, _, xq = _case(orc, n_out, n_in, seed=3 * n_out + n_in, ncols=2)
    dw, dxq = dev(w), dev(xq)
    y2 = empty(2 * n_out)
    rmi.native_q6_k_mmvq(dw, dxq, y2, n_in, n_out, 2)
    col = n_in // 32 * 36
    y2h = host(y2)
    for c in range(2):
        y1 = empty(n_out)
        rmi.native_q6_k_mmvq(dw, dev(xq[c * col:(c + 1) * col]), y1, n_in, n_out, 1)
        assert np.array_equal(y2h[c * n_out:(c + 1) * n_out].view(np.uint32), host(y1).view(np.uint32))
    assert_close_rel(y2h, orc.q6k_gemv(w, xq, n_in, n_out, ncols=2), what="q6k ncols=2")


@pytest.mark.parametrize("ncols", [3, 4, 7])
def test_gemv_many_columns(orc, rmi, ncols):
    n_in, n_out = 4096, 200
    w, _, xq = _case(orc, n_out, n_in, seed=90 + ncols, ncols=ncols)
    y = empty(ncols * n_out)
    rmi.native_q6_k_mmvq(dev(w), dev(xq), y, n_in, n_out, ncols)
    assert_close_rel(host(y), orc.q6k_gemv(w, xq, n_in, n_out, ncols=ncols), what=f"ncols={ncols}")


@pytest.mark.parametrize("n_in,n_out", [(4096, 12288), (12288, 4096), (4096, 4096), (512, 38)])
def test_residual_epilogue(orc, rmi, n_in, n_out):
    """config 1 (12288 x 4096 + residual) and the verify down/ssm_out shapes: res == plain + res bitwise."""
    w, _, xq = _case(orc, n_out, n_in, seed=5 * n_out + n_in)
    res = orc.normal(n_out, seed=77)
    dw, dxq = dev(w), dev(xq)
    y = empty(n_out)
    rmi.native_q6_k_mmvq(dw, dxq, y, n_in, n_out, 1)
    plain = host(y)
    yr = dev(res)                                   # in place: y aliases res, as the engine calls it (qw:843)
    part = empty((n_out + 3) // 4)
    rmi.native_q6_k_mmvq_res(dw, dxq, yr, yr, part, n_in, n_out)
    got = host(yr)
    assert np.array_equal(got.view(np.uint32), (plain + res).astype(np.float32).view(np.uint32))
    ref, pref = orc.q6k_gemv(w, xq, n_in, n_out, res=res, partials=True)
    assert_close_rel(got, ref, what="res y")
    assert_close_rel(host(part), pref, rtol=1e-5, atol_frac=1e-6, what="partials")
    g = np.pad(got.astype(np.float64), (0, (-n_out) % 4)).reshape(-1, 4)
    np.testing.assert_allclose(host(part), (g ** 2).sum(1), rtol=1e-6)


@pytest.mark.parametrize("n_in,n_out", [(12288, 4096), (4096, 4096), (4096, 24576), (1024, 22)])
def test_residual_epilogue_two_columns(orc, rmi, n_in, n_out):
    """config 2's fused down epilogue at ncols = 2: column j == the ncols = 1 residual call, bitwise."""
    w, _, xq = _case(orc, n_out, n_in, seed=11 * n_out + n_in, ncols=2)
    res = orc.normal(2 * n_out, seed=78)
    dw, dxq = dev(w), dev(xq)
    np_ = (n_out + 3) // 4
    y2, p2 = dev(res), empty(2 * np_)
    rmi.native_q6_k_mmvq_res_n(dw, dxq, y2, y2, p2, n_in, n_out, 2)
    y2h, p2h = host(y2), host(p2)
    col = n_in // 32 * 36
    for c in range(2):
        y1, p1 = dev(res[c * n_out:(c + 1) * n_out]), empty(np_)
        rmi.native_q6_k_mmvq_res(dw, dev(xq[c * col:(c + 1) * col]), y1, y1, p1, n_in, n_out)
        assert np.array_equal(y2h[c * n_out:(c + 1) * n_out].view(np.uint32), host(y1).view(np.uint32))
        assert np.array_equal(p2h[c * np_:(c + 1) * np_].view(np.uint32), host(p1).view(np.uint32))
    ref, pref = orc.q6k_gemv(w, xq, n_in, n_out, ncols=2, res=res, partials=True)
    assert_close_rel(y2h, ref, what="res_n y")
    assert_close_rel(p2h, pref, rtol=1e-5, atol_frac=1e-6, what="res_n partials")


def test_gemv_rejects_bad_arguments(rmi):
    t = empty(4096)
    with pytest.raises(ValueError, match="divisible"):
        rmi.native_q6_k_mmvq(t, t, t, 100, 4, 1)
    with pytest.raises(ValueError, match="ncols"):
        rmi.native_q6_k_mmvq(t, t, t, 256, 4, 17)
    with pytest.raises(ValueError, match="stream"):
        rmi.native_q6_k_mmvq(t, t, t, 256, 4, 1, stream=0)
