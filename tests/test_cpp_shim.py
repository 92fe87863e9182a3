"""CPU-side check of include/rapier_mi.hpp: a C++ caller written against the reference's strata::kernels surface
compiles against the shim, links librapier_mi.so, and gets the reference's exception types for bad arguments
(std::invalid_argument, mmvq:2312-2325) before any device work."""
import os
import shutil
import subprocess
import textwrap

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

PROGRAM = textwrap.dedent(r"""
    #include "rapier_mi.hpp"
    #include "rapier_mi_engine.h"
    #include <cstdio>
    #include <cstring>
    int main() {
        void* fake = reinterpret_cast<void*>(uintptr_t(1) << 20);
        int caught = 0;
        try { strata::kernels::native_q6_k_mmvq(fake, fake, (float*) fake, 100, 4, 1, fake); }
        catch (const std::invalid_argument& e) { caught += std::strstr(e.what(), "divisible") != nullptr; }
        try { strata::kernels::native_q6_k_mmvq(fake, fake, (float*) fake, 256, 4, 1, nullptr); }
        catch (const std::invalid_argument& e) { caught += std::strstr(e.what(), "stream") != nullptr; }
        try { strata::kernels::native_mmvq(11, fake, fake, (float*) fake, 256, 4, 1, fake); }
        catch (const std::invalid_argument& e) { caught += std::strstr(e.what(), "unsupported") != nullptr; }
        try { (void) strata::kernels::native_q8_1_bytes(31, 1); }
        catch (const std::invalid_argument&) { caught += 1; }
        try { strata::kernels::native_q5_k_mmvq(fake, fake, (float*) fake, 100, 4, 1, fake); }
        catch (const std::invalid_argument& e) { caught += std::strstr(e.what(), "divisible") != nullptr; }
        // the attention glue and --split names (qw:971-975, 1542-1544, 1002-1068), validated before device work
        strata::kernels::RopeScaling rope;
        rope.type = strata::kernels::RopeScalingType::YaRN;
        rope.freq_base = 1e7;
        rope.factor = 4.0;
        try { strata::kernels::native_rope_apply((float*) fake, (float*) fake, 16, 256, 63, rope, (int*) fake, fake); }
        catch (const std::invalid_argument&) { caught += 1; }
        try { strata::kernels::rms_norm_weighted((float*) fake, (float*) fake, 16, 0, 1e-6f, fake); }
        catch (const std::invalid_argument&) { caught += 1; }
        try { strata::kernels::add_inplace(nullptr, (float*) fake, 16, fake); }
        catch (const std::invalid_argument&) { caught += 1; }
        try { strata::kernels::scale_inplace(nullptr, 16, 0.5f, fake); }
        catch (const std::invalid_argument&) { caught += 1; }
        try { strata::kernels::silu_inplace(nullptr, 16, fake); }
        catch (const std::invalid_argument&) { caught += 1; }
        const bool ok = strata::kernels::native_q8_1_bytes(4096, 2) == 9216 &&
                        strata::kernels::native_mmvq_weight_bytes(14, 4096, 12288) == 41287680u &&
                        rmi_qwen35_9b_config().n_vocab == 248320;
        std::printf("%d %d\n", caught, ok ? 1 : 0);
        return caught == 10 && ok ? 0 : 1;
    }
""")


@pytest.mark.skipif(shutil.which("g++") is None, reason="g++ not available")
def test_cpp_shim_compiles_and_throws(tmp_path):
    lib = os.path.join(ROOT, "rapier_amd", "librapier_mi.so")
    if not os.path.exists(lib):
        pytest.skip("librapier_mi.so not built")
    src = tmp_path / "shim.cpp"
    src.write_text(PROGRAM)
    exe = tmp_path / "shim"
    subprocess.run(["g++", "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), str(src), lib,
                    f"-Wl,-rpath,{os.path.dirname(lib)}", "-o", str(exe)], check=True)
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=60)
    assert r.returncode == 0, r.stdout + r.stderr
    assert r.stdout.split() == ["10", "1"]


Q8_1_PROGRAM = textwrap.dedent(r"""
    // the reference's own quantize kernels (qw:650-653, 684-688) use q8_1_finite / q8_1_quant / q8_1_ds; the helpers
    // are __host__ __device__, so their host form is checked here against the library's quantizer policy
    #include "rapier_mi_q8_1.hpp"
    #include <cmath>
    #include <cstdio>
    #include <cstring>
    int main(int argc, char** argv) {
        float x[32];
        FILE* f = std::fopen(argv[1], "rb");
        for (int b = 0; std::fread(x, 4, 32, f) == 32; ++b) {
            float amax = 0.0f, sum = 0.0f;
            for (int i = 0; i < 32; ++i) amax = std::fmax(amax, std::fabs(x[i]));
            // the 32-lane xor tree of the block sum (offsets 16, 8, 4, 2, 1)
            float t[32];
            std::memcpy(t, x, sizeof t);
            for (int o = 16; o >= 1; o /= 2) {
                float u[32];
                for (int i = 0; i < 32; ++i) u[i] = t[i] + t[i ^ o];
                std::memcpy(t, u, sizeof t);
            }
            sum = t[0];
            const float d = strata::kernels::q8_1_finite(amax / 127.0f);
            const __half2 ds = strata::kernels::q8_1_ds(d, sum);
            unsigned short h[2];
            std::memcpy(h, &ds, 4);
            std::printf("%u %u", h[0], h[1]);
            for (int i = 0; i < 32; ++i) std::printf(" %d", (int) strata::kernels::q8_1_quant(x[i], d, amax));
            std::printf("\n");
        }
        std::fclose(f);
        return 0;
    }
""")


def test_q8_1_helpers_match_the_quantizer(orc, tmp_path):
    """q8_1_finite / q8_1_quant / q8_1_ds (rapier_mi_q8_1.hpp) give the oracle quantizer's bytes: ordinary blocks, an
    all-zero block, exact .5 ties, a x1e4 block whose sum saturates fp16, and a block whose d saturates"""
    import numpy as np
    hipcc = "/opt/rocm/bin/hipcc"
    if not os.path.exists(hipcc):
        pytest.skip("hipcc not available")
    x = orc.normal(32 * 6, seed=77)
    x[32:64] = 0.0
    x[64:96] = np.arange(32, dtype=np.float32) - 15.5          # d = 16.5 / 127: codes land on ties only by chance
    x[96:128] = np.float32(127.0) * np.array([(-1) ** i * (i / 2) for i in range(32)], np.float32)
    x[128:160] *= np.float32(1e4)
    x[160:192] = np.float32(1e7)
    src, exe, data = tmp_path / "q81.cpp", tmp_path / "q81", tmp_path / "x.bin"
    src.write_text(Q8_1_PROGRAM)
    x.tofile(data)
    subprocess.run([hipcc, "-std=c++17", "-O1", "-I", os.path.join(ROOT, "include"), str(src), "-o", str(exe)],
                   check=True, capture_output=True)
    out = subprocess.run([str(exe), str(data)], capture_output=True, text=True, timeout=60, check=True).stdout
    rows = [list(map(int, line.split())) for line in out.strip().splitlines()]
    assert len(rows) == 6
    ref = orc.quantize_q8_1(x, 32 * 6).reshape(6, 36)
    for b, row in enumerate(rows):
        ds = ref[b, :4].view(np.uint16)
        codes = ref[b, 4:].view(np.int8)
        assert row[:2] == [int(ds[0]), int(ds[1])], f"block {b} ds"
        assert row[2:] == codes.tolist(), f"block {b} codes"
