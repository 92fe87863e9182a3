"""The divide-free rounding of the GEMV kernels that quantize a normed vector in their own activation stage
(q8_round in rapier_amd/csrc/rmi_common.h): roundf(v * (1 / d)) equals roundf(v / d), the norm kernels' quantizer, for
every float v with |v| <= 128 d, except within 2^-14 of a half-integer, where the kernel takes the true divide.
Checked exhaustively (all ~2^31 such v) for a spread of block scales by tests/cpp/q8_round_check.c, which performs the
device's operations in IEEE single precision.  A variant without the fallback window must show mismatches, so the
check can fail."""
import os
import struct
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))


def bits(f):
    return "%08x" % struct.unpack("<I", struct.pack("<f", f))[0]


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    out = tmp_path_factory.mktemp("q8r")
    src = os.path.join(HERE, "cpp", "q8_round_check.c")
    exe, nofb = str(out / "check"), str(out / "check_nofb")
    flags = ["-O2", "-ffp-contract=off", "-fopenmp"]
    subprocess.run(["gcc", *flags, "-o", exe, src, "-lm"], check=True)
    text = open(src).read().replace("0x1p-14f) ||", "0x0p0f) ||")
    nsrc = out / "nofb.c"
    nsrc.write_text(text)
    subprocess.run(["gcc", *flags, "-o", nofb, str(nsrc), "-lm"], check=True)
    return exe, nofb


def run(exe, ds):
    r = subprocess.run([exe] + [bits(d) for d in ds], capture_output=True, text=True, timeout=300)
    rows = [dict(kv.split("=") for kv in line.split()) for line in r.stdout.splitlines()]
    return r.returncode, rows


def test_fast_rounding_equals_divide_exhaustively(checker):
    # block scales of amax 1, 3.7, 1e-3 and 1e4 (d = amax / 127): every |v| <= 128 d, both signs
    rc, rows = run(checker[0], [1.0 / 127, 3.7 / 127, 1e-3 / 127, 1e4 / 127])
    assert rc == 0 and len(rows) == 4
    for r in rows:
        assert int(r["mismatches"]) == 0
        assert int(r["checked"]) > 1_900_000_000
        assert int(r["divide"]) < 1e-4 * int(r["checked"])   # the true divide is the rare path


def test_without_the_fallback_window_the_check_fails(checker):
    rc, rows = run(checker[1], [1.0 / 127])
    assert rc == 1 and int(rows[0]["mismatches"]) > 0
