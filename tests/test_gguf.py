"""CPU checks of the GGUF reader (rmi_gguf_*, the engine's loader front end; the role strata::GgufFile plays at
qw:945-957, 1978-2134): files written by tests/gguf_writer.py from the published GGUF layout read back with every
metadata type, tensor type, shape, offset and alignment intact; malformed files are errors, never crashes."""
import os

import numpy as np
import pytest

from tests.gguf_writer import (ARR, BOOL, F32, F64, I8, I16, I32, I64, STR, U8, U16, U32, U64, tensor_bytes,
                               write_gguf)


@pytest.fixture(scope="module")
def E():
    import rapier_amd.engine as eng
    return eng


def sample(tmp_path, alignment=32):
    rng = np.random.default_rng(5)
    meta = [("general.architecture", STR, "qwen35"), ("general.alignment", U32, alignment),
            ("a.u8", U8, 200), ("a.i8", I8, -7), ("a.u16", U16, 65000), ("a.i16", I16, -300), ("a.i32", I32, -123456),
            ("a.u64", U64, 2 ** 40 + 3), ("a.i64", I64, -(2 ** 41)), ("a.f32", F32, 0.25), ("a.f64", F64, 1e-6),
            ("a.bool", BOOL, True), ("tok", ARR, (STR, ["<|im_end|>", "Ġthe", ""])), ("ids", ARR, (I32, [3, -1, 7]))]
    tensors = [("w.q6", "Q6_K", (512, 3), rng.integers(0, 256, tensor_bytes("Q6_K", (512, 3)), dtype=np.uint8)),
               ("v.f32", "F32", (7,), rng.normal(size=7).astype(np.float32)),
               ("w.q8", "Q8_0", (64, 5), rng.integers(0, 256, tensor_bytes("Q8_0", (64, 5)), dtype=np.uint8)),
               ("w.q5", "Q5_K", (256, 2), rng.integers(0, 256, tensor_bytes("Q5_K", (256, 2)), dtype=np.uint8)),
               ("w.q4", "Q4_K", (256, 1, 2), rng.integers(0, 256, tensor_bytes("Q4_K", (256, 1, 2)), dtype=np.uint8))]
    path = write_gguf(str(tmp_path / f"s{alignment}.gguf"), meta, tensors, alignment=alignment)
    return path, meta, tensors


@pytest.mark.parametrize("alignment", [32, 64])
def test_reader_round_trip(E, tmp_path, alignment):
    path, meta, tensors = sample(tmp_path, alignment)
    g = E.GgufFile(path)
    assert len(g) == len(tensors)
    assert g.str("general.architecture") == "qwen35"
    for k, t, v in meta:
        if t == STR:
            assert g.str(k) == v
        elif t == ARR:
            assert g.array(k) == list(v[1])
        elif t == F32:
            assert g.num(k) == np.float32(v)
        else:
            assert g.num(k) == float(v), k
    types = {"Q6_K": 14, "F32": 0, "Q8_0": 8, "Q5_K": 13, "Q4_K": 12}
    for i, (name, tname, dims, data) in enumerate(tensors):
        assert g.find(name) == i
        n, t, d, arr = g.tensor(i)
        assert (n, t, d) == (name, types[tname], tuple(dims))
        assert np.array_equal(arr, np.ascontiguousarray(data).view(np.uint8).reshape(-1))
    assert g.find("nope") == -1 and g.num("tok") is None and g.str("a.u8") is None
    g.close()


def test_reader_rejects_malformed(E, tmp_path):
    path, _, _ = sample(tmp_path)
    blob = open(path, "rb").read()
    cases = {"magic": b"GGUX" + blob[4:], "version": blob[:4] + b"\x07\0\0\0" + blob[8:],
             "truncated meta": blob[:60], "truncated data": blob[:-100], "empty": b"",
             # a 16M tensor count in a file of a few hundred bytes: rejected before the table is sized by it
             "tensor count": blob[:8] + (1 << 24).to_bytes(8, "little") + blob[16:]}
    for what, data in cases.items():
        p = tmp_path / f"bad_{what.replace(' ', '_')}.gguf"
        p.write_bytes(data)
        with pytest.raises((ValueError, RuntimeError)):
            E.GgufFile(str(p))
    with pytest.raises((ValueError, RuntimeError)):
        E.GgufFile(str(tmp_path / "missing.gguf"))


def test_engine_create_gguf_rejects_non_qwen35(E, tmp_path):
    """architecture check before any device work (load_model, qw:1979-1983)"""
    import ctypes
    path = write_gguf(str(tmp_path / "llama.gguf"), [("general.architecture", STR, "llama")], [])
    E._bind()
    h = ctypes.c_void_p()
    rc = E.lib().rmi_engine_create_gguf(os.fsencode(path), 4096, None, ctypes.byref(h))
    assert rc != 0 and not h.value
    assert b"qwen35" in E.lib().rmi_last_error()
