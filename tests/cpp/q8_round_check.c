/* Exhaustive CPU check of the divide-free Q8_1 rounding used by the GEMV kernels that quantize a normed vector in
 * their activation stage (rmi_common.h q8_round): for a block scale d = amax / 127 and every float v with |v| <= 128 d,
 * the fast path rint(v * (1 / d)) - taken unless the product lies within 2^-14 of a half-integer - must equal
 * roundf(v / d), the quantizer of the norm kernels.  The arithmetic below is the device's, operation for operation
 * (IEEE single, round to nearest, no contraction).
 *
 * usage: q8_round_check <d_bits_hex>...   (each d a float bit pattern); prints, per d, the values checked, the values
 * sent to the true divide and the mismatches of the fast path (must be 0).  Exit status 1 on any mismatch. */
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

static float f_of(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* the device's decision: 1 = the fast path's integer is taken */
static int fast_path(float v, float d, float inv_d, int* q) {
    const float y = v * inv_d;
    const float a = fabsf(y);
    const float fr = a - floorf(a);
    if (!(fabsf(fr - 0.5f) > 0x1p-14f) || !(d >= 0x1p-126f && d <= 0x1p126f)) return 0;
    *q = (int) rintf(y);   /* round half to even (the default mode): equal to roundf away from the ties */
    return 1;
}

int main(int argc, char** argv) {
    int bad_total = 0;
    for (int a = 1; a < argc; ++a) {
        const float d = f_of((uint32_t) strtoul(argv[a], NULL, 16));
        const float inv_d = 1.0f / d;
        const float lim = 128.0f * d;
        long long checked = 0, slow = 0, bad = 0;
        /* every non-negative float up to lim, and its negation */
        uint32_t top;
        memcpy(&top, &lim, 4);
#pragma omp parallel for reduction(+ : checked, slow, bad) schedule(static, 65536)
        for (long long u = 0; u <= (long long) top; ++u) {
            for (int s = 0; s < 2; ++s) {
                const float v = f_of((uint32_t) u | (s ? 0x80000000u : 0u));
                int q;
                const int ref = (int) roundf(v / d);
                if (fast_path(v, d, inv_d, &q)) {
                    if (q != ref) ++bad;
                } else {
                    ++slow;
                }
                ++checked;
            }
        }
        printf("d=%a checked=%lld divide=%lld mismatches=%lld\n", d, checked, slow, bad);
        fflush(stdout);
        if (bad) bad_total = 1;
    }
    return bad_total;
}
