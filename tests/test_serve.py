"""CPU checks of the serve protocol (rmi_serve_fd, the loop behind `rmi_engine --serve`; serve_loop qw:2593-2813) and
of the oracle's top-k list (topk_out, qw:2513-2531).

The C loop runs over a deterministic stand-in engine (tests/serve_fake.py) through rmi_serve_backend callbacks; the
oracle's restatement of the reference loop (oracle/serve.py) runs over an identical instance; the response lines must
be identical, byte for byte.  The GPU tests run the same comparison over the real engine."""
import json

import numpy as np
import pytest

import oracle
from oracle import serve as oserve
from tests.serve_fake import RMI_ERR_LAUNCH, FakeModel, run_c_loop


def req(**kw):
    return json.dumps(kw, separators=(",", ":"))   # the compact JSON the reference's server sends


def both(lines, eos=7, topk=40, tmp_path=None, **model_kw):
    rc, got = run_c_loop(FakeModel(eos=eos, **model_kw), lines, eos=eos, topk=topk, tmp_path=tmp_path)
    want = oserve.serve(FakeModel(eos=eos, **model_kw), lines, eos=eos, topk=topk)
    return rc, got, want


# ---- the oracle's top-k list ----

@pytest.mark.parametrize("seed", [0, 1, 2])
def test_oracle_topk_scan_equals_full_sort(seed):
    """the restated streaming scan against a full sort (logit desc, id asc): many equal logits, -0 and +0"""
    rng = np.random.default_rng(seed)
    l = (rng.integers(-20, 20, 5000) / 4.0).astype(np.float32)
    l[rng.integers(0, 5000, 50)] = -0.0
    for k in (1, 2, 40, 64):
        assert oracle.topk(l, k) == oracle.topk_sorted(l, k)


def test_oracle_topk_known_answers():
    l = np.array([1, 3, 3, 2, 5, -0.0, 0.0, 3], np.float32)
    assert oracle.topk(l, 4) == [(4, 5.0), (1, 3.0), (2, 3.0), (7, 3.0)]
    assert [i for i, _ in oracle.topk(l, 8)] == [4, 1, 2, 7, 3, 0, 5, 6]
    assert oracle.topk(l, 1) == [(4, 5.0)]
    # fewer logits than k: the reference never sorts the partial list
    assert oracle.topk(np.array([1, 2], np.float32), 3) == [(0, 1.0), (1, 2.0)]


def test_token_line_format():
    assert oserve.token_line(12, [(3, 2.5), (9, -0.125)]) == '{"id":12,"top":[[3,2.50000],[9,-0.12500]]}'
    assert oserve.token_line(5, []) == '{"id":5,"top":[]}'


# ---- the C loop against the oracle's loop ----

def test_serve_loop_matches_reference_loop(tmp_path):
    lines = [req(op="reset"),
             req(op="run", tokens=[11, 12, 13], gen=10, mtp=False),
             req(op="run", tokens=[20], gen=12, mtp=True),          # continues the context
             req(op="run", tokens=[21, 22], gen=1, mtp=True),
             req(op="run", tokens=[23], gen=1, mtp=False),
             req(op="run", tokens=[24, 25, 26, 27], gen=30, mtp=True, topk=3),
             req(op="run", tokens=[28], gen=6, mtp=False, topk=0),
             "",
             req(op="reset"),
             req(op="run", tokens=list(range(30, 70)), gen=40, mtp=True),
             req(op="run", tokens=[1, 2], gen=25, mtp=False, topk=64)]
    rc, got, want = both(lines, tmp_path=tmp_path)
    assert rc == 0
    assert got == want
    kinds = [json.loads(x) for x in got]
    assert sum("done" in o for o in kinds) == 8 and sum("ok" in o for o in kinds) == 2
    # the stream is stopped by the end-of-sequence id in both modes
    assert any(o.get("id") == 7 for o in kinds)


@pytest.mark.parametrize("seed", range(6))
def test_serve_loop_matches_reference_loop_random(tmp_path, seed):
    rng = np.random.default_rng(seed)
    lines = [req(op="reset")]
    for _ in range(12):
        if rng.random() < 0.1:
            lines.append(req(op="reset"))
            continue
        n = int(rng.integers(1, 20))
        lines.append(req(op="run", tokens=rng.integers(0, 300, n).tolist(), gen=int(rng.integers(1, 30)),
                         mtp=bool(rng.random() < 0.6)))
    rc, got, want = both(lines, tmp_path=tmp_path, seed=seed, max_ctx=300)
    assert rc == 0 and got == want


def test_serve_errors_match_reference_loop(tmp_path):
    lines = [req(op="run", gen=5),                                  # no tokens
             req(op="run", tokens=[1, 2]),                          # no gen
             req(op="run", tokens=[1, 2], gen=0),
             req(op="run", tokens=[], gen=3),
             req(op="run", tokens=[1] * 50, gen=350),               # does not fit max_ctx 400
             req(op="run", tokens=[3, 4], gen=3, mtp=True)]         # still serves after the errors
    rc, got, want = both(lines, tmp_path=tmp_path)
    assert rc == 0 and got == want
    assert got[:5] == ['{"error":"need tokens and gen"}'] * 4 + ['{"error":"context full; send op reset"}']


def test_serve_request_checks(tmp_path):
    """requests the reference does not define: reported, and the loop goes on"""
    lines = ['{"op":"run","tokens":[1,2,',                              # malformed
             '{"op":"run","tokens":[1.5],"gen":2}',
             req(op="run", tokens=[1, 999], gen=2),                     # id outside the vocabulary
             req(op="run", tokens=[1], gen=2, topk=65),
             '  {"op" : "run", "tokens" : [ 4 , 5 ] , "gen" : 2 , "mtp" : false }  ',
             req(op="run", tokens=[6], gen=2, extra={"nested": [1, {"a": None}]})]
    rc, got = run_c_loop(FakeModel(), lines, eos=7, tmp_path=tmp_path)
    assert rc == 0
    assert got[0].startswith('{"error":"bad request:') and got[1].startswith('{"error":"bad request:')
    assert got[2] == '{"error":"rmi_engine_ingest: bad token id"}'
    assert got[3] == '{"error":"topk must be 0..64"}'
    ok = [json.loads(x) for x in got[4:]]
    # both well-formed requests are served: ids, then done (the second stops at the end-of-sequence id)
    assert [("id" in o, "done" in o) for o in ok] == [(True, False), (True, False), (False, True),
                                                      (True, False), (False, True)]
    assert ok[3]["id"] == 7


def test_serve_device_failure_ends_the_loop(tmp_path):
    lines = [req(op="run", tokens=[1, 2], gen=5), req(op="run", tokens=[3], gen=2)]
    rc, got = run_c_loop(FakeModel(fail_at=("gen_step", 2)), lines, eos=7, tmp_path=tmp_path)
    assert rc == RMI_ERR_LAUNCH
    assert got[-1] == '{"error":"fake device failure"}' and len(got) == 3   # two tokens, then the error; no more


def test_serve_last_line_without_newline(tmp_path):
    import os

    from rapier_amd import engine as E
    src, dst = tmp_path / "in", tmp_path / "out"
    src.write_bytes((req(op="reset") + "\r\n" + req(op="run", tokens=[5], gen=2)).encode())
    fi, fo = os.open(src, os.O_RDONLY), os.open(dst, os.O_WRONLY | os.O_CREAT)
    m = FakeModel()
    try:
        assert E.serve_fd(m.backend(), fi, fo, eos=7) == 0
    finally:
        os.close(fi)
        os.close(fo)
    out = dst.read_text().splitlines()
    assert out[0] == '{"ok":true,"op":"reset"}' and out[-1] == '{"done":true,"pos":3}' and len(out) == 4
