// shim_device - drives librapier_mi on the GPU through the reference-named C++ surface (include/rapier_mi.hpp), the
// way the reference engine calls strata::kernels, and checks the invariants the reference's own src/test_res.cpp
// checks on its kernels: the residual kernel equals the plain GEMV plus the residual, its partials are the 4-row
// sums of squares, and a 2-column call equals two 1-column calls.  Everything here is compared bit for bit; the
// numerical comparison against the CPU oracle is done by tests/test_gpu_shim.py on the files this program writes.
//
//   shim_device DIR    reads DIR/<name>.bin inputs, writes DIR/out_<name>.bin, prints one line per check,
//                      exits 0 when every check passed
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "rapier_mi.hpp"
#include "rapier_mi_engine.h"

namespace {

std::string g_dir;
int g_failures = 0;

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::printf("HIP error in %s: %s\n", what, hipGetErrorString(e));
        std::exit(2);
    }
}

std::vector<uint8_t> load(const char* name) {
    const std::string path = g_dir + "/" + name + ".bin";
    FILE* f = std::fopen(path.c_str(), "rb");
    if (!f) {
        std::printf("missing input %s\n", path.c_str());
        std::exit(2);
    }
    std::vector<uint8_t> v;
    uint8_t buf[1 << 16];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) v.insert(v.end(), buf, buf + n);
    std::fclose(f);
    return v;
}

void save(const char* name, const void* host, size_t bytes) {
    const std::string path = g_dir + "/out_" + name + ".bin";
    FILE* f = std::fopen(path.c_str(), "wb");
    if (!f || std::fwrite(host, 1, bytes, f) != bytes) {
        std::printf("cannot write %s\n", path.c_str());
        std::exit(2);
    }
    std::fclose(f);
}

// device buffer holding a copy of host bytes (or zeros)
struct Buf {
    void* p = nullptr;
    size_t n = 0;
    explicit Buf(size_t bytes) : n(bytes) {
        hip_ok(hipMalloc(&p, bytes), "hipMalloc");
        hip_ok(hipMemset(p, 0, bytes), "hipMemset");
    }
    explicit Buf(const std::vector<uint8_t>& h) : Buf(h.size()) {
        hip_ok(hipMemcpy(p, h.data(), h.size(), hipMemcpyHostToDevice), "upload");
    }
    ~Buf() { (void) hipFree(p); }
    Buf(const Buf&) = delete;
    Buf& operator=(const Buf&) = delete;
    float* f() const { return static_cast<float*>(p); }
    std::vector<uint8_t> host() const {
        std::vector<uint8_t> h(n);
        hip_ok(hipDeviceSynchronize(), "sync");
        hip_ok(hipMemcpy(h.data(), p, n, hipMemcpyDeviceToHost), "download");
        return h;
    }
};

void check(bool ok, const char* what) {
    std::printf("%s %s\n", ok ? "PASS" : "FAIL", what);
    if (!ok) ++g_failures;
}

bool same(const std::vector<uint8_t>& a, const std::vector<uint8_t>& b, size_t off_a, size_t off_b, size_t n) {
    return off_a + n <= a.size() && off_b + n <= b.size() && std::memcmp(a.data() + off_a, b.data() + off_b, n) == 0;
}

}  // namespace

int main(int argc, char** argv) {
    if (argc != 2) {
        std::printf("usage: shim_device DIR\n");
        return 2;
    }
    g_dir = argv[1];
    namespace sk = strata::kernels;
    hip_ok(hipSetDevice(0), "hipSetDevice");
    hipStream_t st;
    hip_ok(hipStreamCreate(&st), "hipStreamCreate");
    std::fflush(stdout);

    // ---- Q8_1 quantize, Q6_K GEMV at 1 and 2 columns, residual epilogue (config-2 down shape at 1024 rows) -------
    const int n_in = 4096, n_out = 1024;
    Buf w(load("w_q6k")), x(load("x")), res(load("res")), w8(load("w_q8_0"));
    Buf xq(sk::native_q8_1_bytes(n_in, 2));
    sk::native_quantize_q8_1(x.f(), xq.p, n_in, 2, st);
    const auto xq_h = xq.host();
    save("xq", xq_h.data(), xq_h.size());
    const size_t col_q8 = sk::native_q8_1_bytes(n_in, 1), col_y = sizeof(float) * n_out;

    Buf y2(2 * col_y), y1(2 * col_y);
    sk::native_q6_k_mmvq(w.p, xq.p, y2.f(), n_in, n_out, 2, st);
    sk::native_q6_k_mmvq(w.p, xq.p, y1.f(), n_in, n_out, 1, st);
    sk::native_q6_k_mmvq(w.p, static_cast<uint8_t*>(xq.p) + col_q8, y1.f() + n_out, n_in, n_out, 1, st);
    const auto y2_h = y2.host(), y1_h = y1.host();
    save("y", y2_h.data(), y2_h.size());
    check(same(y2_h, y1_h, 0, 0, 2 * col_y), "native_q6_k_mmvq: 2-column call == two 1-column calls (bitwise)");

    Buf yd(2 * col_y);
    sk::native_mmvq(14, w.p, xq.p, yd.f(), n_in, n_out, 2, st);
    check(same(yd.host(), y2_h, 0, 0, 2 * col_y), "native_mmvq(14) == native_q6_k_mmvq (bitwise)");

    Buf yr(res.host()), part((n_out / 4) * sizeof(float));
    sk::native_q6_k_mmvq_res(w.p, xq.p, yr.f(), yr.f(), part.f(), n_in, n_out, st);   // y aliases res (qw:843)
    const auto yr_h = yr.host(), part_h = part.host(), res_h = res.host();
    save("y_res", yr_h.data(), yr_h.size());
    save("partials", part_h.data(), part_h.size());
    {
        const float* yp = reinterpret_cast<const float*>(y2_h.data());
        const float* rp = reinterpret_cast<const float*>(res_h.data());
        const float* gp = reinterpret_cast<const float*>(yr_h.data());
        const float* pp = reinterpret_cast<const float*>(part_h.data());
        bool add_ok = true, part_ok = true;
        for (int r = 0; r < n_out; ++r) {
            const float want = yp[r] + rp[r];
            add_ok &= std::memcmp(&want, &gp[r], 4) == 0;
        }
        for (int g = 0; g < n_out / 4; ++g) {
            float s = gp[4 * g] * gp[4 * g];
            for (int r = 1; r < 4; ++r) s = gp[4 * g + r] * gp[4 * g + r] + s;
            const float d = s - pp[g];
            part_ok &= d <= 1e-6f * s && -d <= 1e-6f * s;
        }
        check(add_ok, "native_q6_k_mmvq_res == native_q6_k_mmvq + res (bitwise, y aliasing res)");
        check(part_ok, "native_q6_k_mmvq_res partials == 4-row sums of y^2 (1e-6 rel)");
    }

    // the registry-owned packed copy (native_q6_k_pack, mmvq:2930-2960): the same entry points, the same bits
    {
        const bool packed = sk::native_q6_k_pack(w.p, n_in, n_out, "test matrix");
        Buf yp(2 * col_y), yrp(res.host()), partp((n_out / 4) * sizeof(float));
        sk::native_q6_k_mmvq(w.p, xq.p, yp.f(), n_in, n_out, 2, st);
        sk::native_q6_k_mmvq_res(w.p, xq.p, yrp.f(), yrp.f(), partp.f(), n_in, n_out, st);
        sk::native_q6_k_unpack(w.p);
        check(packed && same(yp.host(), y2_h, 0, 0, 2 * col_y) && same(yrp.host(), yr_h, 0, 0, col_y) &&
                  same(partp.host(), part_h, 0, 0, (n_out / 4) * sizeof(float)),
              "native_q6_k_pack: native_q6_k_mmvq / _res on the packed copy == the GGUF-layout results (bitwise)");
    }

    Buf y8(col_y);
    sk::native_q8_0_mmvq(w8.p, xq.p, y8.f(), n_in, n_out, 1, st);
    const auto y8_h = y8.host();
    save("y_q8_0", y8_h.data(), y8_h.size());

    // error paths with live device buffers: the reference's exception types (mmvq:2312-2331)
    int caught = 0;
    try { sk::native_q6_k_mmvq(w.p, xq.p, y1.f(), n_in, n_out, 1, nullptr); }
    catch (const std::invalid_argument&) { ++caught; }
    try { sk::native_q6_k_mmvq(w.p, xq.p, y1.f(), n_in + 32, n_out, 1, st); }
    catch (const std::invalid_argument&) { ++caught; }
    try { sk::native_q6_k_mmvq(w.p, xq.p, y1.f(), n_in, n_out, 17, st); }
    catch (const std::invalid_argument&) { ++caught; }
    try { sk::rms_norm_weighted(y1.f(), y1.f(), 4, 100000, 1e-6f, st); }
    catch (const std::invalid_argument&) { ++caught; }
    check(caught == 4, "bad stream / n_in / ncols / cols throw std::invalid_argument");

    // ---- fused GDN: conv + SiLU + L2, then the delta-rule step + RMSNorm * SiLU(z) + Q8_1 (fgdn:167-225) ----------
    {
        const int h_k = 2, h_v = 4, S = 128, ch = (2 * h_k + h_v) * S;
        Buf hist(load("gdn_hist")), qkv(load("gdn_qkv")), cw(load("gdn_conv_w")), state(load("gdn_state"));
        Buf gate(load("gdn_gate")), beta(load("gdn_beta")), z(load("gdn_z")), gamma(load("gdn_gamma"));
        Buf h(sizeof(float) * ch), y(sizeof(float) * h_v * S), q8(sk::native_q8_1_bytes(h_v * S, 1));
        sk::fused_gdn_conv_l2(hist.f(), qkv.f(), cw.f(), h.f(), ch, 2 * h_k, 1e-6f, st);
        const float* hp = h.f();
        sk::fused_gdn_step_norm_silu_q8(state.f(), hp, hp + h_k * S, hp + 2 * h_k * S, gate.f(), beta.f(), z.f(),
                                        gamma.f(), 1e-6f, y.f(), static_cast<uint8_t*>(q8.p), h_k, h_v, st);
        const auto hh = h.host(), hi = hist.host(), sh = state.host(), yh = y.host(), qh = q8.host();
        save("gdn_h", hh.data(), hh.size());
        save("gdn_hist", hi.data(), hi.size());
        save("gdn_state", sh.data(), sh.size());
        save("gdn_y", yh.data(), yh.size());
        save("gdn_q8", qh.data(), qh.size());
        // the step's Q8_1 epilogue equals quantizing its fp32 output
        Buf q8b(sk::native_q8_1_bytes(h_v * S, 1));
        sk::native_quantize_q8_1(y.f(), q8b.p, h_v * S, 1, st);
        check(q8b.host() == qh, "fused_gdn_step_norm_silu_q8: Q8_1 epilogue == native_quantize_q8_1(y) (bitwise)");
    }

    // ---- attention glue: q/k per-head norm, then RoPE in place at per-head device positions (qw:1535-1544) --------
    {
        const int heads = 16, hd = 256, n_rot = 64;
        Buf q(load("rope_x")), qn(load("rope_w")), pos(load("rope_pos"));
        sk::rms_norm_weighted(q.f(), qn.f(), heads, hd, 1e-6f, st);
        const auto normed = q.host();
        save("norm", normed.data(), normed.size());
        sk::RopeScaling rope;
        rope.type = sk::RopeScalingType::YaRN;
        rope.freq_base = 1e7f;
        rope.factor = 4.0f;
        rope.orig_ctx = 65536.0f;
        rope.ext_factor = 1.0f;
        rope.attn_factor = 1.0f;
        rope.beta_fast = 32.0f;
        rope.beta_slow = 1.0f;
        Buf out(normed.size());
        sk::native_rope_apply(q.f(), out.f(), heads, hd, n_rot, rope, static_cast<const int*>(pos.p), st);
        sk::native_rope_apply(q.f(), q.f(), heads, hd, n_rot, rope, static_cast<const int*>(pos.p), st);
        const auto inplace = q.host();
        save("rope", inplace.data(), inplace.size());
        check(out.host() == inplace, "native_rope_apply: in place == out of place (bitwise)");
    }

    // ---- elementwise glue of the --split path ----------------------------------------------------------------------
    {
        const auto a = load("ew_a"), b = load("ew_b");
        const int n = static_cast<int>(a.size() / 4);
        Buf xa(a), xb(b);
        sk::add_inplace(xa.f(), xb.f(), n, st);
        sk::scale_inplace(xa.f(), n, 0.5f, st);
        sk::silu_inplace(xa.f(), n, st);
        const auto r = xa.host();
        save("ew", r.data(), r.size());
    }

    hip_ok(hipStreamSynchronize(st), "final sync");
    hip_ok(hipStreamDestroy(st), "hipStreamDestroy");
    std::printf("%s: %d failed checks\n", g_failures ? "FAILED" : "OK", g_failures);
    return g_failures ? 1 : 0;
}
