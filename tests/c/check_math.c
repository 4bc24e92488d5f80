/* Host check of zllm_amd/csrc/zs_math.h: zs_expf against the host libm expf on
 * a strided sweep of all f32 bit patterns, and the exact-sum increment rule
 * against real f32 additions. Prints "ok" on success. */
#include "../../zllm_amd/csrc/zs_math.h"
#include <stdio.h>
#include <stdlib.h>

static uint64_t st = 88172645463325252ull;
static uint32_t rnd(void) { st ^= st << 13; st ^= st >> 7; st ^= st << 17; return (uint32_t)(st >> 11); }

int main(int argc, char** argv) {
    uint64_t stride = argc > 1 ? strtoull(argv[1], 0, 10) : 97;
    long long bad = 0, n = 0;
    for (uint64_t u = 0; u < 0x100000000ull; u += stride) {
        float x = zs_u2f((uint32_t)u), a = expf(x), b = zs_expf(x);
        n++;
        if (zs_f2u(a) != zs_f2u(b) && !(a != a && b != b)) {
            if (bad < 5) printf("expf mismatch x=%a libm=%a zs=%a\n", x, a, b);
            bad++;
        }
    }
    long long badi = 0, evs = 0;
    for (int it = 0; it < 4000000; it++) {
        float s = zs_u2f(rnd() & 0x7fffffff);
        if (s != s || s > 3e38f) continue;
        float t;
        if (rnd() & 1) t = zs_u2f(rnd() & 0x7fffffff);
        else t = ldexpf(s, -(int)(rnd() % 40)) * (1.0f + (rnd() % 1000) / 1000.0f);
        if (t != t || t > 3e38f) continue;
        int eg = zs_grid_exp(s);
        uint32_t k0 = zs_grid_k(s), tie;
        uint32_t inc = zs_seq_inc(t, eg, &tie);
        if (tie || k0 + inc >= ZS_BINADE) { evs++; continue; }
        if (zs_f2u(zs_grid_value(k0 + inc, eg)) != zs_f2u(s + t)) badi++;
    }
    printf("expf checked %lld mismatches %lld; increments mismatches %lld (events %lld)\n", n, bad, badi, evs);
    if (bad == 0 && badi == 0) printf("ok\n");
    return (bad || badi) ? 1 : 0;
}
