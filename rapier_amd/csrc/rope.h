// rope.h - NEOX rotary embedding with the YaRN ramp, shared by attn_prep (fused per-head norm + RoPE + KV store) and
// the standalone rmi_native_rope_apply, so both rotate a pair with the same operations and give the same bits.
//
// The reference configures YaRN for qwen35 (qw:1991-1999): freq_base, factor, orig_ctx, ext_factor 1, attn_factor 1,
// beta_fast 32, beta_slow 1.  Its rotation (strata's native_rope_apply) is absent from its tree; this is the published
// YaRN algorithm as ggml implements it.  Pair i of n_rot / 2 rotates dims i and i + n_rot / 2 by
//   theta_extrap = pos * base^(-2i / n_rot),  theta = theta_extrap / factor * (1 - ramp) + theta_extrap * ramp,
//   ramp = (1 - clamp((i - low) / max(0.001, high - low), 0, 1)) * ext_factor,
// with cos and sin scaled by mscale.  factor <= 1 is plain NEOX RoPE.
#pragma once

#include <cmath>

#include "rmi_common.h"

namespace rmi {

struct Yarn {
    int on;
    double factor, low, high, ext, mscale;
};

// Host side: the corr dims and magnitude scale of the ramp (fp64, once per call).  Returns false for parameters the
// ramp cannot use.
inline bool yarn_setup(const rmi_rope_params& r, int n_rot, Yarn* y) {
    *y = Yarn{};
    if (!(r.factor > 1.0f)) return true;
    if (!(r.orig_ctx > 0.0f) || !(r.beta_fast > 0.0f) || !(r.beta_slow > 0.0f)) return false;
    const double pi = 3.14159265358979323846, base = r.freq_base;
    const double cf = n_rot * std::log(r.orig_ctx / (r.beta_fast * 2.0 * pi)) / (2.0 * std::log(base));
    const double cs = n_rot * std::log(r.orig_ctx / (r.beta_slow * 2.0 * pi)) / (2.0 * std::log(base));
    y->on = 1;
    y->factor = r.factor;
    y->low = std::fmax(0.0, std::floor(cf));
    y->high = std::fmin(static_cast<double>(n_rot - 1), std::ceil(cs));
    y->ext = r.ext_factor;
    y->mscale = r.ext_factor != 0.0f ? r.attn_factor * (1.0 + 0.1 * std::log(static_cast<double>(r.factor)))
                                     : r.attn_factor;
    return true;
}

// the frequency of pair i (fp64): theta^(-2 i / n_rot), which does not depend on the position
__device__ __forceinline__ double rope_freq(int i, int n_rot, float theta) {
    return pow(static_cast<double>(theta), -2.0 * i / static_cast<double>(n_rot));
}

// cos and sin of pair i at position p from its frequency (angle in fp64, rounded to fp32 once)
__device__ __forceinline__ void rope_cos_sin_f(int p, double freq, int i, const Yarn& yarn, float* c, float* s) {
    double ang = static_cast<double>(p) * freq;
    double sn, cs;
    if (yarn.on) {
        const double y = (static_cast<double>(i) - yarn.low) / fmax(0.001, yarn.high - yarn.low);
        const double ramp = (1.0 - fmin(1.0, fmax(0.0, y))) * yarn.ext;
        ang = (ang / yarn.factor) * (1.0 - ramp) + ang * ramp;
        sincos(ang, &sn, &cs);
        sn *= yarn.mscale;
        cs *= yarn.mscale;
    } else {
        sincos(ang, &sn, &cs);
    }
    *c = static_cast<float>(cs);
    *s = static_cast<float>(sn);
}

__device__ __forceinline__ void rope_cos_sin(int p, int i, int n_rot, float theta, const Yarn& yarn, float* c,
                                             float* s) {
    rope_cos_sin_f(p, rope_freq(i, n_rot, theta), i, yarn, c, s);
}

// the rotated pair (a, b) = (dim i, dim i + n_rot / 2); explicit fmas, so contraction cannot change the bits
__device__ __forceinline__ float rope_lo(float a, float b, float c, float s) { return fmaf(a, c, -(b * s)); }
__device__ __forceinline__ float rope_hi(float a, float b, float c, float s) { return fmaf(a, s, b * c); }

}  // namespace rmi
