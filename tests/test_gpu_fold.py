"""The folded RMSNorm (rmi_native_q6_k_mmvq_packed_res_fold / _scaled, rmi_native_q6_k_swiglu_packed_scaled,
rmi_quantize_q8_1_weighted): the reference runs rms_quant_apply (qw:627-655) between a residual GEMV and the next
normed GEMV; folded, the residual GEMV's epilogue writes Q8_1(x * w_next) and the normed GEMV scales its rows by
inv = rsqrt(sum of x's partials / n + eps).

Bars (written here):
- the fold epilogue leaves y and the partials bit for bit as the plain residual GEMV, and its Q8_1 equals
  rmi_quantize_q8_1_weighted of that y, which equals the oracle quantizer on the fp32 product x * w, byte for byte;
- a scaled GEMV's columns are bitwise its single-column call at every pass width (1, 2, 3, 4 columns on the narrow
  kernels, 8 and 16 on the MFMA kernel), so the engine's decode, verify and ingest agree bit for bit;
- scaled GEMV and SwiGLU within 1e-3 relative of the oracle's fp64 inv * (W Q8_1(x * w)); against the unfolded pair
  (rms_quant_apply + plain GEMV), whose rounding they move (a few activation codes land on the neighbouring code),
  within 1e-3 of max|.| and correlated > 0.999999;
- the fused SwiGLU scaled kernel bitwise the scaled GEMV + rmi_swiglu_quant_interleaved pair."""
import numpy as np
import pytest

from tests.gpu_util import assert_close_rel, dev, empty, host

pytestmark = pytest.mark.gpu
EPS = 1e-6


@pytest.fixture(scope="module")
def rmi():
    import rapier_amd
    rapier_amd.lib()
    return rapier_amd


def packed(rmi, w, n_in, n_out, swiglu=False):
    wp = empty(rmi.q6_k_packed_bytes(n_in, n_out), "uint8")
    (rmi.q6_k_pack_swiglu(dev(w), wp, n_in, n_out // 2) if swiglu else rmi.q6_k_pack(dev(w), wp, n_in, n_out))
    return wp


def u32(a):
    return np.ascontiguousarray(a).view(np.uint32)


@pytest.mark.parametrize("n_in,n_out", [(4096, 4096), (12288, 4096), (4096, 1024)])
@pytest.mark.parametrize("ncols", [1, 2])
def test_res_fold_epilogue(orc, rmi, n_in, n_out, ncols):
    w = orc.gen_q6k(n_out, n_in, seed=n_in + n_out)
    x = orc.normal(ncols * n_in, seed=31)
    res = orc.normal(ncols * n_out, seed=32, std=3.0)
    wn = orc.normal(n_out, seed=33, mean=1.0, std=0.1)
    xq = dev(orc.quantize_q8_1(x, n_in, ncols))
    wp = packed(rmi, w, n_in, n_out)
    assert rmi.lib().rmi_q6_k_packed_fold_supported(n_in, n_out, ncols) == 1
    y0, p0 = dev(res), empty(ncols * n_out // 4)
    rmi.native_q6_k_mmvq_packed_res_n(wp, xq, y0, y0, p0, n_in, n_out, ncols)
    y1, p1 = dev(res), empty(ncols * n_out // 4)
    q8 = empty(ncols * n_out // 32 * 36, "uint8")
    rmi.native_q6_k_mmvq_packed_res_fold(wp, xq, y1, y1, p1, dev(wn), q8, n_in, n_out, ncols)
    yh = host(y1)
    assert np.array_equal(u32(yh), u32(host(y0))), "y"
    assert np.array_equal(u32(host(p1)), u32(host(p0))), "partials"
    q8w = empty(ncols * n_out // 32 * 36, "uint8")
    rmi.quantize_q8_1_weighted(y1, dev(wn), q8w, n_out, ncols)
    assert np.array_equal(host(q8), host(q8w)), "epilogue Q8_1 vs quantize_q8_1_weighted"
    prod = (yh.reshape(ncols, n_out) * wn).astype(np.float32).reshape(-1)
    assert np.array_equal(host(q8), orc.quantize_q8_1(prod, n_out, ncols)), "Q8_1 of y * w vs the oracle quantizer"


def test_fold_rejects_other_shapes(rmi):
    f = empty(64, "uint8")
    assert rmi.lib().rmi_q6_k_packed_fold_supported(8192, 4096, 2) == 0
    assert rmi.lib().rmi_q6_k_packed_fold_supported(4096, 4100, 1) == 0
    assert rmi.lib().rmi_q6_k_packed_fold_supported(4096, 4096, 3) == 0
    with pytest.raises(ValueError, match="next norm"):
        rmi.native_q6_k_mmvq_packed_res_fold(f, f, f, f, f, f, f, 8192, 4096, 2)


def inv64(orc, x, cols, ncols):
    return np.array([orc.rms_inv(orc.row_sum_partials(x[c * cols:(c + 1) * cols]), cols, EPS) for c in range(ncols)])


@pytest.mark.parametrize("n_in,n_out", [(4096, 12352), (4096, 10240), (4096, 33001), (2048, 1001)])
def test_scaled_gemv_columns_and_oracle(orc, rmi, n_in, n_out):
    """pass widths 1..4 (narrow kernels: split, stream, loop) and 8 / 16 (MFMA) give each column the bits of its
    single-column call; within 1e-3 of the fp64 oracle and of the unfolded pair"""
    nmax = 16
    w = orc.gen_q6k(n_out, n_in, seed=3 * n_out)
    x = orc.normal(nmax * n_in, seed=41, std=2.0)
    wn = orc.normal(n_in, seed=42, mean=1.0, std=0.1)
    parts = np.concatenate([orc.row_sum_partials(x[c * n_in:(c + 1) * n_in]) for c in range(nmax)]).astype(np.float32)
    xw = (x.reshape(nmax, n_in) * wn).astype(np.float32).reshape(-1)
    xq = orc.quantize_q8_1(xw, n_in, nmax)
    wp, xd, pd = packed(rmi, w, n_in, n_out), dev(xq), dev(parts)
    qb, pb = n_in // 32 * 36, n_in // 4
    single = []
    for c in range(nmax):
        y = empty(n_out)
        rmi.native_q6_k_mmvq_packed_scaled(wp, xd[c * qb:], pd[c * pb:], EPS, y, n_in, n_out, 1)
        single.append(host(y))
    for nc in (2, 3, 4, 8, 16):
        y = empty(nc * n_out)
        rmi.native_q6_k_mmvq_packed_scaled(wp, xd, pd, EPS, y, n_in, n_out, nc)
        yh = host(y)
        for c in range(nc):
            assert np.array_equal(u32(yh[c * n_out:(c + 1) * n_out]), u32(single[c])), f"ncols {nc} column {c}"
    inv = inv64(orc, x, n_in, 2)
    ref = orc.q6k_gemv(w, xq[:2 * qb], n_in, n_out, ncols=2).reshape(2, n_out) * inv[:, None]
    for c in range(2):
        assert_close_rel(single[c], ref[c], what=f"scaled column {c} vs oracle")
    # the unfolded pair: rms_quant_apply then the plain GEMV
    q8n = empty(2 * qb, "uint8")
    rmi.rms_quant_apply(dev(x[:2 * n_in]), dev(wn), dev(parts[:2 * pb]), q8n, n_in, EPS, ncols=2)
    yn = empty(2 * n_out)
    rmi.native_q6_k_mmvq_packed(wp, q8n, yn, n_in, n_out, 2)
    ynh = host(yn)
    for c in range(2):
        # Q8_1 of x * w and of (x * w) * inv round a few activations to the neighbouring code (their fp32 values
        # differ by ulps); one such flip moves every output row by about d8 * |w_row|: a bar on max|.|, not per row
        a, b = single[c].astype(np.float64), ynh[c * n_out:(c + 1) * n_out].astype(np.float64)
        assert np.abs(a - b).max() <= 1e-3 * np.abs(b).max(), f"folded vs unfolded column {c}"
        assert np.corrcoef(a, b)[0, 1] > 0.999999


@pytest.mark.parametrize("ncols", [1, 2])
def test_swiglu_scaled(orc, rmi, ncols):
    n_in, ff = 4096, 12288
    w = orc.gen_q6k(2 * ff, n_in, seed=77)
    x = orc.normal(ncols * n_in, seed=78, std=2.0)
    wn = orc.normal(n_in, seed=79, mean=1.0, std=0.1)
    parts = np.concatenate([orc.row_sum_partials(x[c * n_in:(c + 1) * n_in]) for c in range(ncols)]).astype(np.float32)
    xq = orc.quantize_q8_1((x.reshape(ncols, n_in) * wn).astype(np.float32).reshape(-1), n_in, ncols)
    wp = packed(rmi, w, n_in, 2 * ff, swiglu=True)
    xd, pd = dev(xq), dev(parts)
    out = empty(ncols * ff // 32 * 36, "uint8")
    rmi.native_q6_k_swiglu_packed_scaled(wp, xd, pd, EPS, out, n_in, ff, ncols)
    ug = empty(ncols * 2 * ff)
    rmi.native_q6_k_mmvq_packed_scaled(wp, xd, pd, EPS, ug, n_in, 2 * ff, ncols)
    out2 = empty(ncols * ff // 32 * 36, "uint8")
    rmi.swiglu_quant_interleaved(ug, out2, ff, ncols, 2 * ff)
    assert np.array_equal(host(out), host(out2)), "fused scaled SwiGLU vs scaled GEMV + swiglu_quant_interleaved"
    inv = inv64(orc, x, n_in, ncols)
    yu = orc.q6k_gemv(w, xq, n_in, 2 * ff, ncols=ncols).reshape(ncols, 2 * ff) * inv[:, None]
    up, gate = yu[:, :ff], yu[:, ff:]
    act = (gate / (1 + np.exp(-gate)) * up).reshape(-1)
    got = orc.dequantize_q8_1(host(out), ncols * ff)
    step = np.repeat(np.abs(act.reshape(-1, 32)).max(1) / 127, 32)
    assert np.all(np.abs(got - act) <= 0.5 * step + 2e-3 * np.abs(act) + 1e-6), "SwiGLU vs oracle"
