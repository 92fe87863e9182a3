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
    248320, nextn block), synthetic 4K context, greedy vs MTP at forced acceptance 0 / 0.5 / 1.0."""
    E = eng_mod
    eng = E.Engine(E.qwen35_9b_config(), seed=2024, max_ctx=4096 + 256)
    info = eng.info()
    assert info["gdn_layers"] == 24 and info["attn_layers"] == 8
    assert info["norm_fold"] == 0   # the reference's norm order (RMI_NORM_FOLD=1 folds them)
    # one weight pass per round: trunk 5,675,335,680 + lm_head 834,355,200 + draft block 199,557,120 + lm_head
    assert info["trunk_weight_bytes"] == 5_675_335_680 and info["lm_head_bytes"] == 834_355_200
    assert info["round_weight_bytes"] == 7_543_603_200
    first = eng.synth_context(4096, seed=11, last_token=12345)
    pos0, cur0 = eng.state()
    assert pos0 == 4096 and cur0 == first
    ref, res = streams_agree(E, eng, pos0, cur0, 64, natural=False)
    assert res["accept1"]["rounds"] == 32 and res["accept0"]["rounds"] == 64
    eng.close()


@pytest.fixture(scope="module")
def engine_64k(eng_mod):
    E = eng_mod
    eng = E.Engine(E.qwen35_9b_config(), seed=2025, max_ctx=65536)
    yield eng
    eng.close()


def test_qwen35_9b_mtp_stream_bit_identical_at_64k(eng_mod, engine_64k):
    """config 5 at ctx 65536: synthetic context of 64K positions (attention over 512-position chunks, 128 of them per
    query), greedy vs MTP at forced acceptance 0 / 0.5 / 1.0 for 64 tokens, then the config's 400 generated tokens at
    acceptance 0.5 and with the natural draft."""
    E, eng = eng_mod, engine_64k
    ctx = 65536 - 512
    first = eng.synth_context(ctx, seed=13, last_token=4321)
    pos0, cur0 = eng.state()
    assert pos0 == ctx and cur0 == first
    ref, res = streams_agree(E, eng, pos0, cur0, 64, natural=False)
    assert res["accept1"]["rounds"] == 32 and res["accept0"]["rounds"] == 64
    # 400 generated tokens (bench/RESULTS.md:81-82 diff the 400-token stream against greedy)
    eng.restore_state(pos0, cur0)
    long_ref, _ = eng.generate(400, mode=E.GREEDY)
    assert long_ref[:64] == ref
    eng.restore_state(pos0, cur0)
    toks, st = eng.generate(400, mode=E.MTP_FORCED, ref_tokens=long_ref, ref_base=pos0 + 1, pattern=[1, 0])
    assert toks == long_ref, f"400-token MTP stream differs at {next(i for i in range(400) if toks[i] != long_ref[i])}"
    assert st["accepted"] == (st["rounds"] + 1) // 2
    eng.restore_state(pos0, cur0)
    toks, _ = eng.generate(400, mode=E.MTP)
    assert toks == long_ref, "400-token MTP stream (natural draft) differs from greedy"


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


def test_small_model_folded_norms_follow_the_unfolded_engine(eng_mod, monkeypatch):
    """the folded norms (RMI_NORM_FOLD=1: Q8_1(x * w) into a GEMV that scales by inv) against the same seeded model
    with the default rms_quant_apply (the reference's rounding order).  The two round a few activations to
    neighbouring Q8_1 codes, and the GDN state carries each such flip to later tokens, so the bar is the multi-layer one
    of tests/test_gpu_gguf.py: after a 7-token prompt through 4 layers, logits and hidden within 5e-2 of max|.| and
    correlated > 0.999.  The folded engine's MTP stream equals its own greedy stream."""
    E = eng_mod
    monkeypatch.delenv("RMI_NORM_FOLD", raising=False)
    ref = E.Engine(E.small_config(), seed=21, max_ctx=256)
    monkeypatch.setenv("RMI_NORM_FOLD", "1")
    fold = E.Engine(E.small_config(), seed=21, max_ctx=256)
    monkeypatch.delenv("RMI_NORM_FOLD")
    assert ref.info()["norm_fold"] == 0 and fold.info()["norm_fold"] == 1
    prompt = [int(t) for t in np.random.default_rng(8).integers(0, 5000, size=7)]
    f_ref, f_fold = ref.prefill(prompt, batch=1), fold.prefill(prompt, batch=16)
    n_v, n_e = 5000, 2048
    lr = ref.read(E.BUF_LOGITS, 0, 4 * n_v).view(np.float32).astype(np.float64)
    lf = fold.read(E.BUF_LOGITS, 0, 4 * n_v).view(np.float32).astype(np.float64)
    assert np.abs(lf - lr).max() <= 5e-2 * np.abs(lr).max()
    assert np.corrcoef(lf, lr)[0, 1] > 0.999
    hr = ref.read(E.BUF_HIDDEN, 0, 4 * n_e).view(np.float32).astype(np.float64)
    hf = fold.read(E.BUF_HIDDEN, 0, 4 * n_e).view(np.float32).astype(np.float64)
    assert np.abs(hf - hr).max() <= 5e-2 * np.abs(hr).max()
    top = np.sort(lr)[-2:]
    if top[1] - top[0] > 1e-1 * np.abs(lr).max():
        assert f_fold == f_ref
    pos0, cur0 = fold.state()
    streams_agree(E, fold, pos0, cur0, 24)
    ref.close()
    fold.close()
