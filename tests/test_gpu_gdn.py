"""GPU parity of the Gated DeltaNet chain (config 3: 16 key heads, 32 value heads, head_dim 128, 2 tokens).

Bars (tolerances written here): conv output and y within 1e-3 relative of the oracle's fp64 chain; the recurrent
state within 2e-3 max-abs; Q8_1 within half a quantization step; the conv history bit-exact.  Invariants, bit for bit:
the 2-token call's token 0 and token 1 equal two sequential 1-token calls; the rollback buffer holds exactly the
state / history after token 0; the reference-surface entry points (conv_l2, step_norm_silu_q8) agree with the layer
call.  The layer call keeps its conv history per value head ([h_v][q 128 | k 128 | v 128][3], value head h reading
k-head h % h_k); the tests expand the oracle's [channels][3] history to that layout.
"""
import numpy as np
import pytest

from tests.gpu_util import assert_close_rel, dev, empty, host, torch

pytestmark = pytest.mark.gpu

H_K, H_V, S = 16, 32, 128
CH = 2 * H_K * S + H_V * S          # 8192 conv channels
QKVZ = CH + H_V * S                 # 12288 per token: q | k | v | z
EPS = 1e-6


@pytest.fixture(scope="module")
def rmi():
    import rapier_amd
    rapier_amd.lib()
    return rapier_amd


def make_inputs(orc, seed=300):
    qkvz = orc.normal(2 * QKVZ, seed=seed)
    qkvz[QKVZ + 2 * H_K * S + 5 * S:QKVZ + 2 * H_K * S + 5 * S + 32] *= 1e4    # token 1: one v block x 1e4
    qkvz[CH + 7 * S:CH + 7 * S + 32] *= 1e4                                  # token 0: one z block x 1e4 (Q8_1 finite path)
    ab = orc.normal(2 * 2 * H_V, seed=seed + 1)                               # per token [beta 32 | alpha 32]
    conv_w = orc.normal(4 * CH, seed=seed + 2, std=0.5)
    hist = orc.normal(3 * CH, seed=seed + 3, std=0.5)
    state = orc.normal(S * H_V * S, seed=seed + 4, std=0.05)
    dt = np.zeros(H_V, np.float32)
    ssm_a = (-np.exp(orc.normal(H_V, seed=seed + 5, std=0.5))).astype(np.float32)
    gamma = (1 + orc.normal(S, seed=seed + 6, std=0.1)).astype(np.float32)
    return qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma


def expand_hist(h):
    """[channels][3] conv history -> per value head [h_v][q | k | v][128][3] (head h sees k-head h % h_k)"""
    h = np.asarray(h, np.float32).reshape(CH, 3)
    out = np.empty((H_V, 3, S, 3), np.float32)
    for head in range(H_V):
        qh = head % H_K
        out[head, 0] = h[qh * S:(qh + 1) * S]
        out[head, 1] = h[(H_K + qh) * S:(H_K + qh + 1) * S]
        out[head, 2] = h[(2 * H_K + head) * S:(2 * H_K + head + 1) * S]
    return out.reshape(-1)


def oracle_chain(orc, qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma, ntok=2):
    st = state.astype(np.float64)
    hs = hist.copy()
    ys, states, hists, convs = [], [], [], []
    for t in range(ntok):
        x = qkvz[t * QKVZ:(t + 1) * QKVZ]
        h, hs = orc.gdn_conv_l2(hs, x[:CH], conv_w, 2 * H_K, EPS)
        b, g = orc.beta_gate(ab[t * 2 * H_V:t * 2 * H_V + H_V], ab[t * 2 * H_V + H_V:(t + 1) * 2 * H_V], dt, ssm_a)
        y, st = orc.gdn_step_norm(st, h[:H_K * S], h[H_K * S:2 * H_K * S], h[2 * H_K * S:], g, b, x[CH:], gamma, EPS,
                                  H_K, H_V)
        ys.append(y); states.append(st.copy()); hists.append(hs.copy()); convs.append(h)
    return ys, states, hists, convs


def run_layer(rmi, qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma, ntok, sel_val=0, split=False):
    """hist in the per-value-head layout (expand_hist); split: the engine's entry point (1 / 2-token launches on four
    workgroups per value head, with a fresh zeroed exchange buffer)"""
    t = torch()
    st_live, st_other = dev(state), t.zeros(S * H_V * S, device="cuda:0")
    hi_live, hi_other = dev(hist), t.zeros(H_V * 3 * S * 3, device="cuda:0")
    sel = dev(np.array([sel_val], np.int32))
    bufs = (st_live, st_other, hi_live, hi_other) if sel_val == 0 else (st_other, st_live, hi_other, hi_live)
    dq = dev(qkvz[:ntok * QKVZ])
    y = empty(ntok * H_V * S)
    q8 = empty(ntok * H_V * S // 32 * 36, "uint8")
    args = (bufs[0], bufs[1], bufs[2], bufs[3], sel, dq, QKVZ, dev(ab[:ntok * 2 * H_V]), 2 * H_V, dev(conv_w), dev(dt),
            dev(ssm_a), dev(gamma), EPS, y, H_V * S, q8, H_V * S // 32 * 36, H_K, H_V, ntok)
    if split:
        xch = t.zeros(rmi.gdn_exchange_bytes(H_V), dtype=t.uint8, device="cuda:0")
        rmi.gdn_layer_tokens_x(*args, xch)
    else:
        rmi.gdn_layer_tokens(*args)
    return dict(y=host(y), q8=host(q8), conv=host(dq), state=host(st_live), snap=host(st_other), hist=host(hi_live),
                hsnap=host(hi_other))


@pytest.mark.parametrize("split", [False, True])
def test_gdn_two_tokens_match_oracle(orc, rmi, split):
    inp = make_inputs(orc)
    qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma = inp
    r = run_layer(rmi, qkvz, ab, conv_w, expand_hist(hist), state, dt, ssm_a, gamma, ntok=2, split=split)
    assert np.array_equal(r["conv"], qkvz[:2 * QKVZ]), "the layer call reads q|k|v|z only"
    ys, states, hists, convs = oracle_chain(orc, *inp)
    for t in range(2):
        assert_close_rel(r["y"][t * H_V * S:(t + 1) * H_V * S], ys[t], rtol=1e-3, atol_frac=1e-5, what=f"y t{t}")
        blk = H_V * S // 32 * 36
        deq = orc.dequantize_q8_1(r["q8"][t * blk:(t + 1) * blk], H_V * S).reshape(-1, 32).astype(np.float64)
        ref = ys[t].reshape(-1, 32)
        amax = np.abs(ref).max(1, keepdims=True)
        assert (np.abs(deq - ref) <= 0.5 * amax / 127 * 1.001 + 1e-3 * amax + 1e-30).all(), f"q8 t{t}"
        d, s, _ = orc.q8_1_fields(r["q8"][t * blk:(t + 1) * blk])
        assert np.isfinite(d.view(np.float16)).all() and np.isfinite(s.view(np.float16)).all()
    assert np.abs(r["snap"] - states[0]).max() < 2e-3, "state after token 0 (rollback buffer)"
    assert np.abs(r["state"] - states[1]).max() < 2e-3, "state after token 1"
    assert np.array_equal(r["hsnap"], expand_hist(hists[0]))
    assert np.array_equal(r["hist"], expand_hist(hists[1]))


@pytest.mark.parametrize("split", [False, True])
@pytest.mark.parametrize("sel_val", [0, 1])
def test_gdn_two_tokens_bitwise_equal_sequential(orc, rmi, sel_val, split):
    inp = make_inputs(orc, seed=400)
    qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma = inp
    hist = expand_hist(hist)
    r2 = run_layer(rmi, qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma, ntok=2, sel_val=sel_val, split=split)
    a = run_layer(rmi, qkvz[:QKVZ], ab[:2 * H_V], conv_w, hist, state, dt, ssm_a, gamma, ntok=1, sel_val=sel_val,
                  split=split)
    b = run_layer(rmi, qkvz[QKVZ:], ab[2 * H_V:], conv_w, a["hist"], a["state"], dt, ssm_a, gamma, ntok=1,
                  sel_val=sel_val, split=split)
    u = lambda v: np.asarray(v).view(np.uint32)  # noqa: E731
    assert np.array_equal(u(r2["y"][:H_V * S]), u(a["y"])) and np.array_equal(u(r2["y"][H_V * S:]), u(b["y"]))
    blk = H_V * S // 32 * 36
    assert np.array_equal(r2["q8"][:blk], a["q8"]) and np.array_equal(r2["q8"][blk:], b["q8"])
    assert np.array_equal(u(r2["snap"]), u(a["state"])), "rollback state != 1-token state"
    assert np.array_equal(u(r2["state"]), u(b["state"]))
    assert np.array_equal(u(r2["hsnap"]), u(a["hist"])) and np.array_equal(u(r2["hist"]), u(b["hist"]))


def test_gdn_split_kernel_bitwise_equal_one_workgroup_kernel(orc, rmi):
    """The engine's decode / verify launches (1 and 2 tokens, gdn_layer_tokens_x) run four workgroups per value head;
    a 3-token launch runs the one-workgroup-per-head kernel the ingest chunks use.  Token by token the two give the same
    bits: y, Q8_1, the final state and history.  No exchange between a head's workgroups ran out of its bounded wait,
    including on a buffer reused across launches of both token counts."""
    qkvz3 = orc.normal(3 * QKVZ, seed=700)
    ab3 = orc.normal(3 * 2 * H_V, seed=701)
    _, _, conv_w, hist, state, dt, ssm_a, gamma = make_inputs(orc, seed=702)
    hist = expand_hist(hist)
    before = rmi.gdn_exchange_timeouts()
    r3 = run_layer(rmi, qkvz3, ab3, conv_w, hist, state, dt, ssm_a, gamma, ntok=3)
    a = run_layer(rmi, qkvz3[:2 * QKVZ], ab3[:4 * H_V], conv_w, hist, state, dt, ssm_a, gamma, ntok=2, split=True)
    b = run_layer(rmi, qkvz3[2 * QKVZ:], ab3[4 * H_V:], conv_w, a["hist"], a["state"], dt, ssm_a, gamma, ntok=1,
                  split=True)
    u = lambda v: np.asarray(v).view(np.uint32)  # noqa: E731
    n = H_V * S
    assert np.array_equal(u(r3["y"][:2 * n]), u(a["y"])) and np.array_equal(u(r3["y"][2 * n:]), u(b["y"]))
    blk = n // 32 * 36
    assert np.array_equal(r3["q8"][:2 * blk], a["q8"]) and np.array_equal(r3["q8"][2 * blk:], b["q8"])
    assert np.array_equal(u(r3["state"]), u(b["state"])) and np.array_equal(u(r3["hist"]), u(b["hist"]))
    # one exchange buffer across launches of 1 and 2 tokens (the engine's use): epochs stay in step
    t = torch()
    xch = t.zeros(rmi.gdn_exchange_bytes(H_V), dtype=t.uint8, device="cuda:0")
    st = [dev(state), t.zeros(S * H_V * S, device="cuda:0")]
    hi = [dev(hist), t.zeros(H_V * 3 * S * 3, device="cuda:0")]
    sel = dev(np.array([0], np.int32))
    y = empty(2 * H_V * S)
    q8 = empty(2 * H_V * S // 32 * 36, "uint8")
    for ntok in (2, 1, 1, 2, 2, 1):
        rmi.gdn_layer_tokens_x(st[0], st[1], hi[0], hi[1], sel, dev(qkvz3[:ntok * QKVZ]), QKVZ,
                               dev(ab3[:ntok * 2 * H_V]), 2 * H_V, dev(conv_w), dev(dt), dev(ssm_a), dev(gamma), EPS, y,
                               H_V * S, q8, H_V * S // 32 * 36, H_K, H_V, ntok, xch)
    t.cuda.synchronize()
    assert rmi.gdn_exchange_timeouts() == before   # none during this test (a forced-timeout test may have run)


def test_reference_surface_entry_points(orc, rmi):
    """fused_gdn_conv_l2 + beta_gate + fused_gdn_step_norm_silu_q8 (the reference's 3-launch chain) == layer call."""
    inp = make_inputs(orc, seed=500)
    qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma = inp
    ref = run_layer(rmi, qkvz[:QKVZ], ab[:2 * H_V], conv_w, expand_hist(hist), state, dt, ssm_a, gamma, ntok=1)
    _, _, _, convs = oracle_chain(orc, *inp, ntok=1)
    dh, dq = dev(hist), dev(qkvz[:QKVZ])
    rmi.fused_gdn_conv_l2(dh, dq, dev(conv_w), dq, CH, 2 * H_K, EPS)
    dab, gg = dev(ab[:2 * H_V]), empty(H_V)
    rmi.beta_gate(dab, dev(dt), dev(ssm_a), gg, H_V)
    st, y, q8 = dev(state), empty(H_V * S), empty(H_V * S // 32 * 36, "uint8")
    rmi.fused_gdn_step_norm_silu_q8(st, dq, dq[H_K * S:], dq[2 * H_K * S:], gg, dab, dq[CH:], dev(gamma), EPS, y, q8,
                                    H_K, H_V)
    assert_close_rel(host(dq)[:CH], convs[0], rtol=1e-3, atol_frac=1e-6, what="conv")
    assert np.array_equal(expand_hist(host(dh)), ref["hist"])
    # the prepared-gate path computes exp(gate) from a stored logit: same math, last-bit differences allowed
    assert_close_rel(host(y), ref["y"], rtol=1e-5, atol_frac=1e-6, what="step y")
    assert np.abs(host(st) - ref["state"]).max() < 1e-5


def make_chunk_inputs(orc, ntok, seed):
    qkvz = orc.normal(ntok * QKVZ, seed=seed)
    qkvz[CH + 3 * S:CH + 3 * S + 32] *= 1e4                                  # token 0: one z block x 1e4
    ab = orc.normal(ntok * 2 * H_V, seed=seed + 1)
    conv_w = orc.normal(4 * CH, seed=seed + 2, std=0.5)
    hist = orc.normal(3 * CH, seed=seed + 3, std=0.5)
    state = orc.normal(S * H_V * S, seed=seed + 4, std=0.05)
    dt = np.zeros(H_V, np.float32)
    ssm_a = (-np.exp(orc.normal(H_V, seed=seed + 5, std=0.5))).astype(np.float32)
    gamma = (1 + orc.normal(S, seed=seed + 6, std=0.1)).astype(np.float32)
    return qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma


@pytest.mark.parametrize("ntok", [3, 7, 16])
def test_gdn_ingest_chunk_bitwise_equal_sequential(orc, rmi, ntok):
    """an ingest chunk (3..16 tokens in one launch, the row-batched step of src/qwythos_ingest.cu) leaves the state,
    history, y and Q8_1 of ntok sequential 1-token steps, bit for bit, and updates the live buffers in place"""
    qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma = make_chunk_inputs(orc, ntok, seed=600 + ntok)
    hist = expand_hist(hist)
    r = run_layer(rmi, qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma, ntok=ntok)
    assert not r["snap"].any() and not r["hsnap"].any(), "a chunk writes no rollback buffer"
    u = lambda v: np.asarray(v).view(np.uint32)  # noqa: E731
    st, hs = state, hist
    blk = H_V * S // 32 * 36
    for t in range(ntok):
        a = run_layer(rmi, qkvz[t * QKVZ:(t + 1) * QKVZ], ab[t * 2 * H_V:(t + 1) * 2 * H_V], conv_w, hs, st, dt, ssm_a,
                      gamma, ntok=1)
        assert np.array_equal(u(r["y"][t * H_V * S:(t + 1) * H_V * S]), u(a["y"])), f"y token {t}"
        assert np.array_equal(r["q8"][t * blk:(t + 1) * blk], a["q8"]), f"q8 token {t}"
        st, hs = a["state"], a["hist"]
    assert np.array_equal(u(r["state"]), u(st)) and np.array_equal(u(r["hist"]), u(hs))


def test_gdn_ingest_chunk_matches_oracle(orc, rmi):
    ntok = 16
    inp = make_chunk_inputs(orc, ntok, seed=700)
    qkvz, ab, conv_w, hist, state, dt, ssm_a, gamma = inp
    r = run_layer(rmi, qkvz, ab, conv_w, expand_hist(hist), state, dt, ssm_a, gamma, ntok=ntok)
    ys, states, hists, _ = oracle_chain(orc, *inp, ntok=ntok)
    for t in range(ntok):
        assert_close_rel(r["y"][t * H_V * S:(t + 1) * H_V * S], ys[t], rtol=1e-3, atol_frac=1e-5, what=f"y t{t}")
    assert np.abs(r["state"] - states[-1]).max() < 2e-3
    assert np.array_equal(r["hist"], expand_hist(hists[-1]))
