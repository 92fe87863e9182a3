"""End-to-end invariant of the exact-verify MTP round (config 5 and a small member of the same family): the greedy
token stream with MTP is bit-identical to greedy decoding without MTP on the same engine, at forced draft
acceptance 0, 0.5 and 1.0 and with the natural draft; rollback restores the GDN state exactly (a rejected round
leaves the same state as a 1-token step).  Reference behaviour: README.md:80-82, bench/RESULTS.md:81-82,
src/qwythos.cpp:3182-3241."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def eng_mod():
    import rapier_amd.engine as E
    from tests.gpu_util import torch
    torch()
    return E


PATTERNS = {"accept0": [0], "accept05": [1, 0], "accept1": [1]}


def streams_agree(E, eng, pos0, cur0, n, natural=True):
    eng.save_state()
    ref, st_g = eng.generate(n, mode=E.GREEDY)
    results = {"greedy": st_g}
    for name, pat in PATTERNS.items():
        eng.restore_state(pos0, cur0)
        toks, st = eng.generate(n, mode=E.MTP_FORCED, ref_tokens=ref, ref_base=pos0 + 1, pattern=pat)
        assert toks == ref, f"MTP stream differs from greedy ({name}) at {next(i for i in range(n) if toks[i] != ref[i])}"
        results[name] = st
    if natural:
        eng.restore_state(pos0, cur0)
        toks, st = eng.generate(n, mode=E.MTP)
        assert toks == ref, "MTP stream (natural draft) differs from greedy"
        results["natural"] = st
    return ref, results


def test_small_model_prefill_and_mtp_streams(eng_mod):
    E = eng_mod
    eng = E.Engine(E.small_config(), seed=7, max_ctx=512)
    rng = np.random.default_rng(3)
    prompt = [int(t) for t in rng.integers(0, 5000, size=24)]
    first = eng.prefill(prompt)
    pos0, cur0 = eng.state()
    assert pos0 == len(prompt) and cur0 == first
    ref, res = streams_agree(E, eng, pos0, cur0, 48)
    assert len(set(ref)) > 3, "degenerate stream"
    assert res["accept1"]["accepted"] == res["accept1"]["rounds"]
    assert res["accept0"]["accepted"] == 0 and res["accept0"]["rounds"] == 48
    a05 = res["accept05"]
    assert a05["accepted"] == (a05["rounds"] + 1) // 2
    # the same prompt prefilled again reproduces the stream (no state leaks between runs)
    first2 = eng.prefill(prompt)
    toks, _ = eng.generate(48, mode=E.GREEDY)
    assert first2 == first and toks == ref
    eng.close()


def test_small_model_eager_equals_graph(eng_mod):
    E = eng_mod
    eng = E.Engine(E.small_config(), seed=9, max_ctx=256)
    eng.prefill([1, 2, 3, 4, 5])
    pos0, cur0 = eng.state()
    eng.save_state()
    g, _ = eng.generate(16, mode=E.MTP, use_graph=True)
    eng.restore_state(pos0, cur0)
    e, _ = eng.generate(16, mode=E.MTP, use_graph=False)
    assert g == e
    eng.close()


def test_qwen35_9b_mtp_stream_bit_identical_at_4k(eng_mod):
    """config 5 at full size: random-init 9B-class qwen35 (32 layers, 24 GDN + 8 GQA, hidden 4096, FFN 12288, vocab
    248320, nextn block), synthetic 4K context, the config's 400 generated tokens: greedy vs MTP at forced acceptance
    0 / 0.5 / 1.0 and with the natural draft (README.md:80-82, bench/RESULTS.md:81-82 diff 400-token streams)."""
    E = eng_mod
    eng = E.Engine(E.qwen35_9b_config(), seed=2024, max_ctx=4096 + 512)
    info = eng.info()
    assert info["gdn_layers"] == 24 and info["attn_layers"] == 8
    # one weight pass per round: trunk 5,675,335,680 + lm_head 834,355,200 + draft block 199,557,120 + lm_head
    assert info["trunk_weight_bytes"] == 5_675_335_680 and info["lm_head_bytes"] == 834_355_200
    assert info["round_weight_bytes"] == 7_543_603_200
    first = eng.synth_context(4096, seed=11, last_token=12345)
    pos0, cur0 = eng.state()
    assert pos0 == 4096 and cur0 == first
    ref, res = streams_agree(E, eng, pos0, cur0, 400, natural=True)
    assert len(set(ref)) > 3, "degenerate stream"
    assert res["accept1"]["rounds"] == 200 and res["accept0"]["rounds"] == 400
    assert res["accept05"]["accepted"] == (res["accept05"]["rounds"] + 1) // 2
    eng.close()


@pytest.fixture(scope="module")
def engine_64k(eng_mod):
    E = eng_mod
    eng = E.Engine(E.qwen35_9b_config(), seed=2025, max_ctx=65536)
    yield eng
    eng.close()


def test_qwen35_9b_mtp_stream_bit_identical_at_64k(eng_mod, engine_64k):
    """config 5 at ctx 65536: synthetic context of 64K positions (attention over 512-position chunks, 128 of them per
    query), the config's 400 generated tokens: greedy vs MTP at forced acceptance 0 / 0.5 / 1.0 and with the natural
    draft."""
    E, eng = eng_mod, engine_64k
    ctx = 65536 - 512
    first = eng.synth_context(ctx, seed=13, last_token=4321)
    pos0, cur0 = eng.state()
    assert pos0 == ctx and cur0 == first
    ref, res = streams_agree(E, eng, pos0, cur0, 400, natural=True)
    assert len(set(ref)) > 3, "degenerate stream"
    assert res["accept1"]["rounds"] == 200 and res["accept0"]["rounds"] == 400
    assert res["accept05"]["accepted"] == (res["accept05"]["rounds"] + 1) // 2


def test_qwen35_9b_mtp_after_ingest_past_32k(eng_mod, engine_64k):
    """a random prompt of 33,000 tokens ingested in 16-token chunks (every GEMV, GDN step and attention chunk of the
    batched path, the context past 32K), then MTP at forced acceptance 0 / 0.5 / 1.0 equals greedy"""
    E, eng = eng_mod, engine_64k
    prompt = [int(t) for t in np.random.default_rng(17).integers(0, 248320, size=33000)]
    first = eng.prefill(prompt, batch=16)
    pos0, cur0 = eng.state()
    assert pos0 == len(prompt) and cur0 == first
    ref, _ = streams_agree(E, eng, pos0, cur0, 48, natural=True)
    assert len(set(ref)) > 3, "degenerate stream"


def test_gdn_exchange_timeout_is_an_error(eng_mod):
    """a bounded wait of the GDN layer kernel that runs out makes the engine call fail (RMI_ERR_STATE) instead of
    returning tokens computed from stale sums.  The timeout is forced from the host (a 4-poll bound and every wait
    made to miss), so every kernel still ends normally; the normal bound then gives a clean call again."""
    import rapier_amd as rmi
    E = eng_mod
    eng = E.Engine(E.small_config(), seed=5, max_ctx=256)
    eng.prefill([1, 2, 3, 4])
    pos0, cur0 = eng.state()
    eng.save_state()
    ref, _ = eng.generate(8, mode=E.MTP)
    before = rmi.gdn_exchange_timeouts()
    eng.restore_state(pos0, cur0)
    try:
        rmi.gdn_exchange_test(4, True)
        with pytest.raises(rmi.RapierError, match="GDN exchange"):
            eng.generate(8, mode=E.MTP)
    finally:
        rmi.gdn_exchange_test(0, False)
    grown = rmi.gdn_exchange_timeouts() - before
    assert grown > 0
    eng.restore_state(pos0, cur0)
    toks, _ = eng.generate(8, mode=E.MTP)
    assert toks == ref and rmi.gdn_exchange_timeouts() - before == grown
    eng.close()
