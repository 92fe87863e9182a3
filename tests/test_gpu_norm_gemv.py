"""GPU parity of the normed-input GEMVs (rmi_native_q6_k_mmvq_packed_norm, rmi_native_q6_k_swiglu_packed_norm): the
reference's rms_quant_apply (qw:627-655) and the GEMV that reads its Q8_1 output, as one launch whose workgroups
quantize the normed vector into their own activation stage.

Bar: bitwise equal to rmi_rms_quant_apply followed by the packed GEMV (or the fused SwiGLU GEMV) on the same inputs -
every output float and every Q8_1 byte - on random columns, on a x1e4 block, a zero block, a block of subnormal values
(d not a normal number: the true divide) and blocks whose values sit exactly on, or one ulp either side of,
half-integer multiples of d (the divide-free rounding's fallback window)."""
import numpy as np
import pytest

from tests.gpu_util import dev, empty, host

pytestmark = pytest.mark.gpu
N = 4096


@pytest.fixture(scope="module")
def rmi():
    import rapier_amd
    rapier_amd.lib()
    return rapier_amd


def columns(orc, ncols, seed, special):
    x = orc.normal(ncols * N, seed=seed).astype(np.float32).reshape(ncols, N)
    if special:
        x[0, 64:96] *= 1e4                                    # a x1e4 block
        x[-1, 128:160] = 0.0                                  # a zero block
        x[0, 160:192] = np.float32(1e-41) * np.arange(32)     # subnormal values (the norm's inv keeps them tiny)
        half = (np.arange(32) - 15.5).astype(np.float32)      # +-0.5 .. +-15.5: exact half-integer ratios to d ...
        half[0] = 127.0                                       # ... once amax = 127 d
        x[-1, 256:288] = half * 0.25
        x[-1, 288:320] = np.nextafter(half * 0.25, np.float32(np.inf))
        x[0, 320:352] = np.nextafter(half * 0.25, np.float32(-np.inf))
    return x.reshape(-1)


def partials(rmi, xd, ncols):
    p = empty(ncols * (N // 4))
    rmi.row_sum_partials(xd, p, N, ncols)
    return p


@pytest.mark.parametrize("n_out", [12352, 10240, 4096, 70, 24576])
@pytest.mark.parametrize("ncols", [1, 2])
@pytest.mark.parametrize("special", [False, True])
def test_norm_gemv_bitwise_equals_norm_then_gemv(orc, rmi, n_out, ncols, special):
    w = orc.gen_q6k(n_out, N, seed=n_out + ncols)
    wp = empty(rmi.q6_k_packed_bytes(N, n_out), "uint8")
    rmi.q6_k_pack(dev(w), wp, N, n_out)
    xd = dev(columns(orc, ncols, seed=n_out + 7, special=special))
    gamma = dev((1.0 + 0.1 * orc.normal(N, seed=3)).astype(np.float32))
    pd = partials(rmi, xd, ncols)
    eps = 1e-6
    q8 = empty(rmi.native_q8_1_bytes(N, ncols), "uint8")
    rmi.rms_quant_apply(xd, gamma, pd, q8, N, eps, ncols)
    ref = empty(ncols * n_out)
    rmi.native_q6_k_mmvq_packed(wp, q8, ref, N, n_out, ncols)
    got = empty(ncols * n_out)
    rmi.native_q6_k_mmvq_packed_norm(wp, xd, gamma, pd, eps, got, N, n_out, ncols)
    assert np.array_equal(host(got).view(np.uint32), host(ref).view(np.uint32))


@pytest.mark.parametrize("ff", [12288, 320])
@pytest.mark.parametrize("ncols", [1, 2])
@pytest.mark.parametrize("special", [False, True])
def test_norm_swiglu_bitwise_equals_norm_then_swiglu_gemv(orc, rmi, ff, ncols, special):
    w = orc.gen_q6k(2 * ff, N, seed=3 * ff + ncols)
    ws = empty(rmi.q6_k_packed_bytes(N, 2 * ff), "uint8")
    rmi.q6_k_pack_swiglu(dev(w), ws, N, ff)
    xd = dev(columns(orc, ncols, seed=ff + 11, special=special))
    gamma = dev((1.0 + 0.1 * orc.normal(N, seed=4)).astype(np.float32))
    pd = partials(rmi, xd, ncols)
    eps = 1e-6
    q8 = empty(rmi.native_q8_1_bytes(N, ncols), "uint8")
    rmi.rms_quant_apply(xd, gamma, pd, q8, N, eps, ncols)
    qb = rmi.native_q8_1_bytes(ff, ncols)
    ref = empty(qb, "uint8")
    rmi.native_q6_k_swiglu_packed(ws, q8, ref, N, ff, ncols)
    got = empty(qb, "uint8")
    rmi.native_q6_k_swiglu_packed_norm(ws, xd, gamma, pd, eps, got, N, ff, ncols)
    assert np.array_equal(host(got), host(ref))


def test_norm_stage_half_integer_ratios_take_the_divide(orc, rmi):
    """partials chosen so that inv = 1 exactly (sum 4096, eps 0) and weights 1: the normed values are x itself, and a
    block of x = (k + 1/2) with amax 127 puts every ratio v / d exactly on a half-integer, where the divide-free
    rounding must hand over to the true divide (round half away from zero)"""
    x = np.zeros(N, np.float32)
    blk = (np.arange(32) - 15.5).astype(np.float32)
    blk[0] = 127.0
    x[:32] = blk
    x[32:64] = -blk
    xd, gamma = dev(x), dev(np.ones(N, np.float32))
    pd = dev(np.full(N // 4, 4.0, np.float32))
    n_out = 64
    w = orc.gen_q6k(n_out, N, seed=99)
    wp = empty(rmi.q6_k_packed_bytes(N, n_out), "uint8")
    rmi.q6_k_pack(dev(w), wp, N, n_out)
    q8 = empty(rmi.native_q8_1_bytes(N, 1), "uint8")
    rmi.rms_quant_apply(xd, gamma, pd, q8, N, 0.0, 1)
    codes = host(q8)[4:36].view(np.int8).astype(int)
    assert list(codes) == [127] + [int(np.sign(v) * np.floor(abs(v) + 0.5)) for v in blk[1:]]
    ref, got = empty(n_out), empty(n_out)
    rmi.native_q6_k_mmvq_packed(wp, q8, ref, N, n_out, 1)
    rmi.native_q6_k_mmvq_packed_norm(wp, xd, gamma, pd, 0.0, got, N, n_out, 1)
    assert np.array_equal(host(got).view(np.uint32), host(ref).view(np.uint32))
