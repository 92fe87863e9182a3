"""Batched ingest (prefill in chunks of 2..16 tokens, one weight pass per chunk) leaves exactly the state of the
token-by-token path: first token, position, every GDN layer's state and conv history, the K/V rows of every trunk
attention layer and of the draft block, and the hidden the first draft reads, all bit for bit; the greedy stream
that follows is therefore the same.  Reference: README.md:52-55 ("8-wide Q8 GEMV prefill (16-wide is QWYTHOS_BN=16,
same ids) ... Greedy ids match the per-token path"), serve_ingest_kernels src/qwythos.cpp:2192-2502 and the batch
loop 2658-2722, src/qwythos_ingest.cu:1-9 (bit-equal to the per-column path by construction)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def E():
    import rapier_amd.engine as eng
    from tests.gpu_util import torch
    torch()
    return eng


def snapshot(E, eng, n):
    """every buffer the prompt leaves behind, as bytes"""
    c = eng.cfg
    out = {"state": eng.state()}
    st_bytes = 4 * 128 * c.ssm_h_v * 128
    hist_bytes = 4 * c.ssm_h_v * 3 * 128 * 3
    kv_row = 2 * c.n_kv * c.head_dim
    for il in range(c.n_layer + 1):
        attn = il == c.n_layer or (il + 1) % 4 == 0
        if attn:
            out[f"k{il}"] = eng.read(E.BUF_K_CACHE, il, n * kv_row)
            out[f"v{il}"] = eng.read(E.BUF_V_CACHE, il, n * kv_row)
        else:
            out[f"s{il}"] = eng.read(E.BUF_GDN_STATE, il, st_bytes)
            out[f"h{il}"] = eng.read(E.BUF_GDN_HIST, il, hist_bytes)
    out["hidden"] = eng.read(E.BUF_HIDDEN, 0, 4 * c.n_embd)
    return out


def assert_same(a, b, what):
    assert a["state"] == b["state"], f"{what}: (pos, token) {a['state']} != {b['state']}"
    for k in a:
        if k == "state":
            continue
        if not np.array_equal(a[k], b[k]):
            nd = int(np.count_nonzero(a[k] != b[k]))
            raise AssertionError(f"{what}: buffer {k} differs in {nd} of {a[k].size} bytes")


@pytest.mark.parametrize("n", [37, 16, 5])
def test_small_model_chunked_prefill_equals_per_token(E, n):
    eng = E.Engine(E.small_config(), seed=5, max_ctx=256)
    rng = np.random.default_rng(n)
    prompt = [int(t) for t in rng.integers(0, 5000, size=n)]
    first1 = eng.prefill(prompt, batch=1)
    ref = snapshot(E, eng, n)
    assert ref["state"] == (n, first1)
    assert np.any(ref["k3"] != 0) and np.any(ref[f"k{eng.cfg.n_layer}"] != 0)
    greedy_ref, _ = eng.generate(12, mode=E.GREEDY)
    for batch in (16, 8, 3, 2):
        first = eng.prefill(prompt, batch=batch)
        assert first == first1, f"batch {batch}: first token {first} != {first1}"
        assert_same(snapshot(E, eng, n), ref, f"batch {batch}")
        toks, _ = eng.generate(12, mode=E.GREEDY)
        assert toks == greedy_ref, f"batch {batch}: greedy stream differs"
    eng.close()


def test_small_model_chunked_prefill_then_mtp(E):
    """MTP after a chunked prefill reproduces greedy (the draft KV the chunks wrote is the draft's context)"""
    eng = E.Engine(E.small_config(), seed=12, max_ctx=256)
    prompt = list(range(100, 141))
    eng.prefill(prompt, batch=16)
    pos0, cur0 = eng.state()
    eng.save_state()
    ref, _ = eng.generate(32, mode=E.GREEDY)
    eng.restore_state(pos0, cur0)
    toks, st = eng.generate(32, mode=E.MTP)
    assert toks == ref
    eng.close()


def test_qwen35_9b_chunked_prefill_equals_per_token(E):
    """the 9B-class shapes (packed GEMVs at 16 columns, 32 GDN value heads, 16 query heads in pairs of columns)"""
    eng = E.Engine(E.qwen35_9b_config(), seed=2024, max_ctx=512)
    rng = np.random.default_rng(1)
    n = 41
    prompt = [int(t) for t in rng.integers(0, 248320, size=n)]
    first1 = eng.prefill(prompt, batch=1)
    ref = snapshot(E, eng, n)
    first16 = eng.prefill(prompt, batch=16)
    assert first16 == first1
    assert_same(snapshot(E, eng, n), ref, "batch 16")
    first8 = eng.prefill(prompt, batch=8)
    assert first8 == first1
    assert_same(snapshot(E, eng, n), ref, "batch 8")
    eng.close()
