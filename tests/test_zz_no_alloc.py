"""rmi_gqa_flash_decode_noalloc (the allocation-free attention entry point; its records live in the library's
per-GPU scratch array) against rmi_gqa_flash_decode with a caller workspace, bit for bit, on two calls in a row: the
config-4 verify pair at ctx 65536, then a smaller call (one query at ctx 4096) that reuses the array; plus the size
check that rejects records beyond the array before any device work."""
import numpy as np
import pytest

from tests.gpu_util import dev, empty, host

pytestmark = pytest.mark.gpu

NH, NKV, HD = 16, 4, 256
Q3 = NH * 2 * HD + 2 * NKV * HD
SCALE = 1.0 / 16.0


@pytest.fixture(scope="module")
def rmi():
    import rapier_amd
    rapier_amd.lib()
    return rapier_amd


def run(rmi, fn, q, kc, vc, p0, gate, ntok, max_ctx, nsub):
    y = empty(ntok * NH * HD)
    q8 = empty(ntok * NH * HD // 32 * 36, "uint8")
    args = (q, kc, vc, dev(np.array([p0], np.int32)), gate, Q3, y, NH * HD, q8, NH * HD // 32 * 36)
    if fn == "ws":
        ws = empty(rmi.gqa_workspace_bytes(max_ctx, NKV, nsub), "uint8")
        rmi.gqa_flash_decode(*args, ws, NH, NKV, HD, ntok, max_ctx, nsub, SCALE)
    else:
        rmi.gqa_flash_decode_noalloc(*args, NH, NKV, HD, ntok, max_ctx, nsub, SCALE)
    return host(y), host(q8)


def test_noalloc_equals_workspace_entry(orc, rmi):
    assert rmi.lib().rmi_gqa_noalloc_scratch_max() == 16 << 20
    for ctx, nsub, ntok, seed in ((65536, 8, 2, 1), (4096, 2, 1, 2)):   # the second call is the smaller one
        print(f"noalloc: ctx {ctx} nsub {nsub} ntok {ntok}", flush=True)
        assert rmi.lib().rmi_gqa_noalloc_scratch_bytes(ctx, NKV, nsub, ntok * NH // NKV) <= 16 << 20
        k = orc.normal(ctx * NKV * HD, seed=seed).astype(np.float16).view(np.uint16)
        v = orc.normal(ctx * NKV * HD, seed=seed + 10).astype(np.float16).view(np.uint16)
        q = orc.normal(ntok * NH * HD, seed=seed + 20)
        g = orc.normal(ntok * Q3, seed=seed + 30)
        dk, dv, dq, dg = dev(k), dev(v), dev(q), dev(g)
        p0 = ctx - ntok - 5
        y_ws, q8_ws = run(rmi, "ws", dq, dk, dv, p0, dg, ntok, ctx, nsub)
        y_na, q8_na = run(rmi, "noalloc", dq, dk, dv, p0, dg, ntok, ctx, nsub)
        assert np.array_equal(y_na.view(np.uint32), y_ws.view(np.uint32)), f"y at ctx {ctx}"
        assert np.array_equal(q8_na, q8_ws), f"q8 at ctx {ctx}"


def test_noalloc_rejects_records_beyond_the_scratch(rmi):
    # a 16-token ingest chunk at ctx 65536 with nsub 2: 512 chunks x 4 heads x 64 slots of 1040 B = 136 MB
    fake = empty(64, "uint8")
    assert rmi.lib().rmi_gqa_noalloc_scratch_bytes(65536, NKV, 2, 64) > 16 << 20
    with pytest.raises(ValueError, match="scratch"):
        rmi.gqa_flash_decode_noalloc(fake, fake, fake, fake, fake, Q3, fake, NH * HD, fake, 0, NH, NKV, HD, 16, 65536,
                                     2, SCALE)
