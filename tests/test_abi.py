"""CPU-side checks of the C ABI (no GPU needed): librapier_mi.so loads and exports every entry point
include/rapier_mi.h declares; argument validation rejects bad calls before any device work, with the reference's
messages and exception types (mmvq:2312-2331: std::invalid_argument -> ValueError)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


@pytest.fixture(scope="module")
def rmi():
    import rapier_amd
    rapier_amd.lib()
    return rapier_amd


def declared(headers=("rapier_mi.h",)):
    hdr = "".join(open(os.path.join(ROOT, "include", h)).read() for h in headers)
    return sorted(set(re.findall(r"\b(rmi_\w+)\s*\(", hdr)))


def test_every_declared_symbol_is_exported(rmi):
    names = declared(("rapier_mi.h", "rapier_mi_engine.h"))
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(rmi.lib(), n)]
    assert not missing, missing


def test_python_mirror_covers_the_header(rmi):
    assert set(rmi.SIGNATURES) <= set(declared())


def test_version(rmi):
    assert b"gfx950" in rmi.lib().rmi_version()


FAKE = ctypes.c_void_p(1 << 20)   # aligned, never dereferenced: validation fails first


@pytest.mark.parametrize("n_in,n_out,ncols,msg", [
    (100, 4, 1, "divisible"), (256, 4, 0, "ncols"), (256, 4, 17, "ncols"), (256, 0, 1, "n_out")])
def test_gemv_shape_validation(rmi, n_in, n_out, ncols, msg):
    with pytest.raises(ValueError, match=msg):
        rmi._call("rmi_native_q6_k_mmvq", FAKE, FAKE, FAKE, n_in, n_out, ncols, FAKE)


def test_gemv_pointer_and_stream_validation(rmi):
    with pytest.raises(ValueError, match="aligned"):
        rmi._call("rmi_native_q6_k_mmvq", ctypes.c_void_p((1 << 20) + 2), FAKE, FAKE, 256, 4, 1, FAKE)
    with pytest.raises(ValueError, match="aligned"):
        rmi._call("rmi_native_q6_k_mmvq", None, FAKE, FAKE, 256, 4, 1, FAKE)
    with pytest.raises(ValueError, match="stream"):
        rmi._call("rmi_native_q6_k_mmvq", FAKE, FAKE, FAKE, 256, 4, 1, None)


def test_type_dispatch(rmi):
    L = rmi.lib()
    for t in (14, 13, 12, 8):
        assert L.rmi_native_mmvq_supported(t)
    assert not L.rmi_native_mmvq_supported(11) and not L.rmi_native_mmvq_supported(23)   # Q3_K, IQ4_XS
    with pytest.raises(ValueError, match="unsupported"):
        rmi._call("rmi_native_mmvq", 11, FAKE, FAKE, FAKE, 256, 4, 1, FAKE)
    L.rmi_native_mmvq_weight_bytes.restype = ctypes.c_size_t
    L.rmi_native_mmvq_weight_bytes.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    assert L.rmi_native_mmvq_weight_bytes(14, 4096, 12288) == 41_287_680
    assert L.rmi_native_mmvq_weight_bytes(8, 4096, 10) == 10 * 128 * 34
    assert L.rmi_native_mmvq_weight_bytes(13, 4096, 10) == 10 * 16 * 176
    assert L.rmi_native_mmvq_weight_bytes(12, 4096, 10) == 10 * 16 * 144
    assert L.rmi_native_mmvq_weight_bytes(14, 100, 10) == 0


def test_q8_1_bytes(rmi):
    assert rmi.native_q8_1_bytes(4096, 2) == 9216
    with pytest.raises(ValueError):
        rmi.native_q8_1_bytes(31, 1)


def test_kernel_argument_validation(rmi):
    with pytest.raises(ValueError, match="invalid"):
        rmi._call("rmi_fused_gdn_conv_l2", FAKE, FAKE, FAKE, FAKE, 100, 0, ctypes.c_float(1e-6), FAKE)
    with pytest.raises(ValueError, match="invalid"):
        rmi._call("rmi_fused_gdn_step_norm_silu_q8", *([FAKE] * 8), ctypes.c_float(1e-6), FAKE, None, 16, 30, FAKE)
    with pytest.raises(ValueError, match="invalid"):
        rmi._call("rmi_gqa_flash_decode", *([FAKE] * 5), 0, FAKE, 0, None, 0, FAKE, 16, 4, 128, 1, 4096, 1,
                  ctypes.c_float(0.0625), FAKE)
    with pytest.raises(ValueError, match="bad shape"):
        rmi._call("rmi_argmax", FAKE, 0, 1, 0, FAKE, FAKE, FAKE)
