"""The reference-named C++ surface (include/rapier_mi.hpp, strata::kernels) on the device: tests/cpp/shim_device calls
it the way src/qwythos.cpp does and checks the invariants of the reference's own src/test_res.cpp (residual kernel ==
plain GEMV + residual with y aliasing res, 4-row partials, 2-column == two 1-column calls), bit for bit; this file
feeds it oracle-generated inputs and compares what it wrote against the CPU oracle:
- Q8_1 bytes bit-exact; Q6_K / Q8_0 GEMVs within 1e-3 relative of the fp64 oracle;
- fused GDN conv (1e-3), history (bit-exact), state (2e-3 max-abs), y (1e-3);
- per-head RMSNorm (1e-6) and YaRN RoPE at per-head positions (1e-5) against the oracle's RMSNorm and fp64 YaRN;
- add / scale / silu against numpy."""
import os
import subprocess

import numpy as np
import pytest

from tests.gpu_util import assert_close_rel

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "tests", "cpp", "shim_device")
N_IN, N_OUT = 4096, 1024
H_K, H_V, S = 2, 4, 128
CH = (2 * H_K + H_V) * S


def put(d, name, a):
    np.ascontiguousarray(a).tofile(os.path.join(d, name + ".bin"))


def got(d, name, dtype):
    return np.fromfile(os.path.join(d, "out_" + name + ".bin"), dtype=dtype)


def test_shim_device_program(orc, tmp_path):
    if not os.path.exists(BIN):
        pytest.fail(f"{BIN} is not built (__graft_entry__.build())")
    d = str(tmp_path)
    w = orc.gen_q6k(N_OUT, N_IN, seed=501)
    w8 = orc.gen_q8_0(N_OUT, N_IN, seed=502)
    x = orc.normal(2 * N_IN, seed=503)
    x[N_IN + 64:N_IN + 96] *= 1e4                      # one column-1 block x 1e4 (the finite d / sum path)
    res = orc.normal(N_OUT, seed=504)
    hist = orc.normal(3 * CH, seed=505, std=0.5)
    qkv = orc.normal(CH, seed=506)
    conv_w = orc.normal(4 * CH, seed=507, std=0.5)
    state = orc.normal(S * H_V * S, seed=508, std=0.05)
    b_in, a_in = orc.normal(H_V, seed=509), orc.normal(H_V, seed=510)
    ssm_a = (-np.exp(orc.normal(H_V, seed=511, std=0.5))).astype(np.float32)
    beta, gate = orc.beta_gate(b_in, a_in, np.zeros(H_V, np.float32), ssm_a)
    z = orc.normal(H_V * S, seed=512)
    gamma = (1 + orc.normal(S, seed=513, std=0.1)).astype(np.float32)
    rx = orc.normal(16 * 256, seed=514, std=2.0)
    rw = (1 + orc.normal(256, seed=515, std=0.1)).astype(np.float32)
    rpos = (np.arange(16, dtype=np.int32) * 9001 + 7).astype(np.int32)     # every head at its own position
    ea, eb = orc.normal(3000, seed=516), orc.normal(3000, seed=517)
    for name, a in (("w_q6k", w), ("w_q8_0", w8), ("x", x), ("res", res), ("gdn_hist", hist), ("gdn_qkv", qkv),
                    ("gdn_conv_w", conv_w), ("gdn_state", state), ("gdn_gate", gate.astype(np.float32)),
                    ("gdn_beta", beta.astype(np.float32)), ("gdn_z", z), ("gdn_gamma", gamma), ("rope_x", rx),
                    ("rope_w", rw), ("rope_pos", rpos), ("ew_a", ea), ("ew_b", eb)):
        put(d, name, a)
    print(f"running {BIN} on {d}", flush=True)
    r = subprocess.run([BIN, d], capture_output=True, text=True, timeout=120)
    print(r.stdout, r.stderr, flush=True)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.count("PASS") == 8 and "FAIL" not in r.stdout

    xq = orc.quantize_q8_1(x, N_IN, 2)
    assert np.array_equal(got(d, "xq", np.uint8), xq), "Q8_1 bytes"
    ref = orc.q6k_gemv(w, xq, N_IN, N_OUT, ncols=2)
    assert_close_rel(got(d, "y", np.float32), ref, rtol=1e-3, atol_frac=1e-5, what="native_q6_k_mmvq")
    ref_r, ref_p = orc.q6k_gemv(w, xq[:N_IN // 32 * 36], N_IN, N_OUT, ncols=1, res=res, partials=True)
    assert_close_rel(got(d, "y_res", np.float32), ref_r, rtol=1e-3, atol_frac=1e-5, what="native_q6_k_mmvq_res")
    assert_close_rel(got(d, "partials", np.float32), ref_p, rtol=1e-3, atol_frac=1e-5, what="partials")
    ref8 = orc.q8_0_gemv(w8, xq[:N_IN // 32 * 36], N_IN, N_OUT)
    assert_close_rel(got(d, "y_q8_0", np.float32), ref8, rtol=1e-3, atol_frac=1e-5, what="native_q8_0_mmvq")

    h, hist_ref = orc.gdn_conv_l2(hist, qkv, conv_w, 2 * H_K, 1e-6)
    assert_close_rel(got(d, "gdn_h", np.float32), h, rtol=1e-3, atol_frac=1e-5, what="fused_gdn_conv_l2")
    assert np.array_equal(got(d, "gdn_hist", np.float32), hist_ref), "conv history"
    y, st = orc.gdn_step_norm(state.astype(np.float64), h[:H_K * S], h[H_K * S:2 * H_K * S], h[2 * H_K * S:], gate,
                              beta, z, gamma, 1e-6, H_K, H_V)
    assert np.abs(got(d, "gdn_state", np.float32) - st).max() <= 2e-3, "GDN state"
    assert_close_rel(got(d, "gdn_y", np.float32), y, rtol=1e-3, atol_frac=1e-5, what="fused_gdn_step y")

    nref = orc.rms_norm_heads(rx, rw, 16, 256, 1e-6)
    assert_close_rel(got(d, "norm", np.float32), nref, rtol=1e-6, atol_frac=1e-7, what="rms_norm_weighted")
    rope = np.concatenate([orc.rope_yarn(nref[h * 256:(h + 1) * 256], 1, 256, 64, int(rpos[h]), 1e7, 4.0, 65536.0)
                           for h in range(16)])
    assert_close_rel(got(d, "rope", np.float32), rope, rtol=1e-5, atol_frac=2e-6, what="native_rope_apply")

    s = ((ea + eb) * np.float32(0.5)).astype(np.float64)
    assert_close_rel(got(d, "ew", np.float32), s / (1 + np.exp(-s)), rtol=1e-6, atol_frac=1e-7, what="elementwise")
