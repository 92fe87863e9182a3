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
        const bool ok = strata::kernels::native_q8_1_bytes(4096, 2) == 9216 &&
                        strata::kernels::native_mmvq_weight_bytes(14, 4096, 12288) == 41287680u &&
                        rmi_qwen35_9b_config().n_vocab == 248320;
        std::printf("%d %d\n", caught, ok ? 1 : 0);
        return caught == 5 && ok ? 0 : 1;
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
    assert r.stdout.split() == ["5", "1"]
