"""The serving path on the GPU (serve_loop qw:2593-2813): the engine's continuing context (rmi_engine_reset / ingest /
gen_begin / gen_step / topk) and the `rmi_engine --serve` executable.

- Ingest continues a context exactly: prefill(A), generate (greedy or MTP, with accepts and rejects), then ingest(B)
  leaves the state of one prefill of everything fed, bit for bit (GDN state and history, trunk and draft K/V rows,
  hidden, position, first token).
- The executable's response lines equal, byte for byte, the oracle's restatement of the reference loop
  (oracle/serve.py) run over the same engine in this process, whose lists come from the oracle's top-k of the logits
  read back from the device.  MTP ids equal greedy ids; the end-of-sequence id stops a run; QWYTHOS_BN /
  QWYTHOS_NOBATCH ingest gives the same lines."""
import json
import os
import subprocess

import numpy as np
import pytest

from oracle import serve as oserve
from tests.test_gpu_gguf import N_VOCAB, build_model, write

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "rapier_amd", "rmi_engine")
MAX_CTX = 1024
PATTERN = (0, 0, 0, 1)   # three GDN layers, one attention layer


@pytest.fixture(scope="module")
def E():
    import rapier_amd.engine as eng
    from tests.gpu_util import torch
    torch()
    return eng


@pytest.fixture(scope="module")
def model_path(orc, tmp_path_factory):
    t, meta = build_model(orc, seed=11, pattern=PATTERN)
    return str(write(t, meta, tmp_path_factory.mktemp("serve") / "m.gguf"))


def snapshot(E, eng, upto, draft_skip=(0, 0)):
    """everything a later token reads, for positions [0, upto); draft K/V rows [lo, hi) of draft_skip left out"""
    c = eng.cfg
    out = {"state": eng.state(), "hidden": eng.read(E.BUF_HIDDEN, 0, 4 * c.n_embd)}
    row = c.n_kv * c.head_dim * 2
    for il in range(c.n_layer + 1):
        if il < c.n_layer and not PATTERN[il]:
            out[f"s{il}"] = eng.read(E.BUF_GDN_STATE, il, 4 * 128 * c.ssm_h_v * 128)
            out[f"h{il}"] = eng.read(E.BUF_GDN_HIST, il, 4 * c.ssm_h_v * 3 * 128 * 3)
        else:                                         # attention layers and the draft block (layer n_layer)
            keep = np.ones(upto * row, bool)
            if il == c.n_layer:
                keep[draft_skip[0] * row:draft_skip[1] * row] = False
            out[f"k{il}"] = eng.read(E.BUF_K_CACHE, il, upto * row)[keep]
            out[f"v{il}"] = eng.read(E.BUF_V_CACHE, il, upto * row)[keep]
    return out


def assert_same(a, b):
    assert a.keys() == b.keys()
    for key in a:
        if isinstance(a[key], tuple):
            assert a[key] == b[key], key
        else:
            assert np.array_equal(a[key], b[key]), key


@pytest.mark.parametrize("mode,batch", [(0, 16), (2, 16), (2, 1), (0, 5), (1, 16)])
def test_ingest_continues_the_context(E, model_path, mode, batch):
    """mode 0 greedy, 1 MTP with the model's own drafts, 2 MTP with forced accepts and rejects.  A greedy generation
    runs no draft, so the draft K/V rows of the positions it fed stay unwritten (as in the reference, whose
    forward_token writes none either): those rows are left out after mode 0, every row is compared after MTP."""
    eng = E.Engine.from_gguf(model_path, max_ctx=MAX_CTX)
    rng = np.random.default_rng(mode * 10 + batch)
    a, b = rng.integers(0, N_VOCAB, 37).tolist(), rng.integers(0, N_VOCAB, 21).tolist()
    first = eng.prefill(a, batch=batch)
    if mode == 2:
        ref, _ = eng.generate(14, mode=E.GREEDY)
        first = eng.prefill(a, batch=batch)
        gen, st = eng.generate(12, mode=E.MTP_FORCED, ref_tokens=[first] + ref, ref_base=len(a),
                               pattern=[1, 0, 1, 1, 0])
        assert 0 < st["accepted"] < st["rounds"], st  # the round's hidden hand-over runs both ways
    else:
        gen, st = eng.generate(12, mode=mode)
    pos, _ = eng.state()
    stream = [first] + gen
    fed = a + stream[:pos - len(a)]                  # the tokens now in the context
    nxt = eng.ingest(b, batch=batch)
    skip = (len(a), pos) if mode == 0 else (0, 0)
    got = snapshot(E, eng, pos + len(b), skip)
    ref_first = eng.prefill(fed + b, batch=batch)
    assert nxt == ref_first
    assert_same(got, snapshot(E, eng, pos + len(b), skip))
    eng.close()


class EngineAdapter:
    """the oracle loop's engine interface over rapier_amd.engine.Engine; lists from the oracle's top-k of the logits
    read back from the device"""

    def __init__(self, E, eng, orc):
        self.E, self.eng, self.orc = E, eng, orc
        self.max_ctx = eng.info()["max_ctx"]
        self.mode = None

    def reset(self):
        self.eng.reset()
        self.mode = None

    def position(self):
        return self.eng.state()[0]

    def ingest(self, tokens):
        self.mode = None
        return self.eng.ingest(tokens, batch=16)

    def top(self, k):
        logits = self.eng.read(self.E.BUF_LOGITS, 0, 4 * N_VOCAB).view(np.float32)
        got = self.eng.topk(k)
        ref = self.orc.topk(logits, k)
        assert got == ref
        return ref

    def greedy_step(self):
        if self.mode != 0:
            self.eng.gen_begin(0)
            self.mode = 0
        return self.eng.gen_step()[0]

    def mtp_begin(self):
        self.eng.gen_begin(1)
        self.mode = 1

    def mtp_round(self):
        out = self.eng.gen_step()
        return out[0], out[1] if len(out) > 1 else -1, len(out) == 2


def run_bin(model_path, lines, eos=None, env=None, timeout=240):
    cmd = [BIN, "--model", model_path, "--serve"] + (["--eos", str(eos)] if eos is not None else [])
    e = dict(os.environ, QWYTHOS_MAXCTX=str(MAX_CTX), **(env or {}))
    print("serve executable:", " ".join(cmd), env or "", flush=True)
    p = subprocess.run(cmd, input="".join(x + "\n" for x in lines), capture_output=True, text=True, env=e,
                       timeout=timeout)
    assert p.returncode == 0, p.stderr[-2000:]
    assert "rapier serve: ready" in p.stderr
    return p.stdout.splitlines()


def req(**kw):
    return json.dumps(kw, separators=(",", ":"))


def requests(rng):
    return [req(op="reset"),
            req(op="run", tokens=rng.integers(0, N_VOCAB, 40).tolist(), gen=24, mtp=False),
            req(op="run", tokens=rng.integers(0, N_VOCAB, 5).tolist(), gen=30, mtp=True),
            req(op="run", tokens=[17], gen=1, mtp=True),
            req(op="run", tokens=[18, 19], gen=9, mtp=False, topk=5),
            req(op="run", gen=3),
            req(op="run", tokens=[1] * 20, gen=2000),
            req(op="reset"),
            req(op="run", tokens=rng.integers(0, N_VOCAB, 19).tolist(), gen=40, mtp=True)]


def test_serve_executable_matches_reference_loop(E, orc, model_path):
    assert os.path.exists(BIN), "build the engine executable first"
    lines = requests(np.random.default_rng(5))
    got = run_bin(model_path, lines)
    eng = E.Engine.from_gguf(model_path, max_ctx=MAX_CTX)
    want = oserve.serve(EngineAdapter(E, eng, orc), lines, eos=248046)
    eng.close()
    assert got == want
    assert sum('"done"' in x for x in got) == 5
    for x in got:
        json.loads(x)


def test_serve_in_process_and_batches_agree(E, model_path, tmp_path):
    lines = requests(np.random.default_rng(6))
    ref = run_bin(model_path, lines)
    for env in ({"QWYTHOS_BN": "8"}, {"QWYTHOS_NOBATCH": "1"}):
        assert run_bin(model_path, lines, env=env) == ref, env
    eng = E.Engine.from_gguf(model_path, max_ctx=MAX_CTX)
    src, dst = tmp_path / "in.jsonl", tmp_path / "out.jsonl"
    src.write_text("".join(x + "\n" for x in lines))
    fi, fo = os.open(src, os.O_RDONLY), os.open(dst, os.O_WRONLY | os.O_CREAT)
    try:
        eng.serve_fd(fi, fo)
    finally:
        os.close(fi)
        os.close(fo)
    eng.close()
    assert dst.read_text().splitlines() == ref


def ids_of(lines):
    runs, cur = [], []
    for x in lines:
        o = json.loads(x)
        if "id" in o:
            cur.append(o["id"])
        elif "done" in o:
            runs.append(cur)
            cur = []
    return runs


def test_serve_mtp_ids_equal_greedy_and_eos_stops(model_path):
    prompt = list(range(100, 140))
    greedy = ids_of(run_bin(model_path, [req(op="run", tokens=prompt, gen=48, mtp=False)]))[0]
    mtp = ids_of(run_bin(model_path, [req(op="run", tokens=prompt, gen=48, mtp=True)]))[0]
    assert mtp == greedy and len(greedy) == 48
    eos = greedy[6]
    stop = greedy.index(eos) + 1
    for mtp_flag in (False, True):
        out = run_bin(model_path, [req(op="run", tokens=prompt, gen=48, mtp=mtp_flag)], eos=eos)
        got = ids_of(out)[0]
        assert got[:stop] == greedy[:stop]
        if not mtp_flag:
            assert got == greedy[:stop]            # greedy ends right after the id (qw:2752)
            assert json.loads(out[-1]) == {"done": True, "pos": len(prompt) + stop - 1}


def test_executable_cli_generates_the_greedy_stream(model_path):
    prompt = list(range(100, 140))
    greedy = ids_of(run_bin(model_path, [req(op="run", tokens=prompt, gen=20, mtp=False)]))[0]
    p = subprocess.run([BIN, "--model", model_path, "--tokens", ",".join(map(str, prompt)), "--n", "20"],
                       capture_output=True, text=True, env=dict(os.environ, QWYTHOS_MAXCTX=str(MAX_CTX)), timeout=240)
    assert p.returncode == 0, p.stderr[-2000:]
    assert json.loads(p.stdout.splitlines()[-1])["tokens"] == greedy
    bad = subprocess.run([BIN, "--model", model_path, "--split", "0.3", "--serve"], capture_output=True, text=True,
                         timeout=60)
    assert bad.returncode == 2 and "split" in bad.stderr

