"""GPU parity of rmi_topk (the serve protocol's per-token list; topk_out, qw:2513-2531) against the oracle's
restatement of the reference's scan: ids equal and logits bitwise equal, on the qwen35 vocabulary and on the shapes
where the kernel changes its lane width (8 / 16 / 32 logits per lane), with many equal logits and -0 / +0."""
import numpy as np
import pytest

from tests.gpu_util import dev, empty, host

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rmi():
    import rapier_amd
    rapier_amd.lib()
    return rapier_amd


def run(rmi, l, k):
    n = l.size
    ws = empty(max(rmi.topk_workspace_bytes(n), 8) // 4)
    ids, vals = empty(k, "int32"), empty(k)
    rmi.topk(dev(l), n, k, ids, vals, ws)
    return list(zip(host(ids).tolist(), host(vals).tolist()))


@pytest.mark.parametrize("n", [248320, 1, 100, 1000, 262144, 262145, 524289, 1048576])
def test_topk_matches_oracle(orc, rmi, n):
    rng = np.random.default_rng(n)
    l = (rng.standard_normal(n) * 3).astype(np.float32)
    for k in sorted({1, min(n, 40), min(n, 64)}):
        got = run(rmi, l, k)
        assert got == orc.topk(l, k), (n, k)


@pytest.mark.parametrize("n", [248320, 5000])
def test_topk_ties_and_signed_zero(orc, rmi, n):
    rng = np.random.default_rng(7)
    l = (rng.integers(-30, 12, n) / 4.0).astype(np.float32)     # hundreds of logits share each value
    l[rng.integers(0, n, 200)] = -0.0
    for k in (1, 40, 64):
        got = run(rmi, l, k)
        assert got == orc.topk(l, k) == orc.topk_sorted(l, k), k
    z = np.zeros(n, np.float32)
    z[::3] = -0.0                                                 # all equal: the k lowest ids
    assert [i for i, _ in run(rmi, z, 40)] == list(range(40))


def test_topk_concentrated_and_extremes(orc, rmi):
    """every winner in one wave's slice (the merge pops one list repeatedly), and infinities"""
    n = 248320
    l = np.full(n, -1.0, np.float32)
    l[1000:1064] = np.arange(64, dtype=np.float32)
    l[5] = np.inf
    l[7] = -np.inf
    assert run(rmi, l, 64) == orc.topk(l, 64)
    l2 = np.full(n, -np.inf, np.float32)
    l2[n - 1] = 0.0
    assert run(rmi, l2, 3) == orc.topk(l2, 3)


def test_topk_rejects_bad_shapes(rmi):
    ws = empty(1024)
    ids, vals = empty(64, "int32"), empty(64)
    x = empty(100)
    for n, k in [(100, 0), (100, 65), (10, 11), (0, 1), (1048577, 1)]:
        with pytest.raises(ValueError):
            rmi.topk(x, n, k, ids, vals, ws)
