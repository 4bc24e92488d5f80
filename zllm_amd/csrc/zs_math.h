// zs_math.h -- scalar arithmetic shared by the HIP kernels and the host code.
//
// Everything here is exact integer or IEEE arithmetic with explicit fma(), so a
// function gives bit-identical results on the host (x86-64) and on gfx950.
#pragma once
#include <stdint.h>
#include <string.h>
#include <math.h>

#if defined(__HIPCC__)
#include <hip/hip_runtime.h>
#define ZS_HD __host__ __device__ __forceinline__
#else
#define ZS_HD static inline
#endif

ZS_HD uint32_t zs_f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
ZS_HD float zs_u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
ZS_HD uint64_t zs_d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
ZS_HD double zs_u2d(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

// ---------------------------------------------------------------------------
// expf exactly as glibc 2.35 computes it on x86-64 with FMA (the routine Rust's
// f32::exp resolves to on Linux, used by sampler.rs:68-69 and logprobs.rs:36).
// Algorithm: ARM optimized-routines expf (Szabolcs Nagy), EXP2F_TABLE_BITS=5:
//   x*32/ln2 = k + r,  exp(x) = 2^(k/32) * 2^(r/32),
//   2^(r/32) ~= 1 + C2 r + C1 r^2 + C0 r^3 evaluated in double,
// with the FMA-contracted reduction r = fma(32/ln2, x, -k). The table holds the
// correctly rounded doubles 2^(i/32) with i<<47 pre-subtracted from the bits.
// Checked against the host libm over every finite f32 input (tests/).
// ---------------------------------------------------------------------------
#define ZS_EXP2F_TAB                                                                     \
    {0x3ff0000000000000ull, 0x3fefd9b0d3158574ull, 0x3fefb5586cf9890full,                \
     0x3fef9301d0125b51ull, 0x3fef72b83c7d517bull, 0x3fef54873168b9aaull,                \
     0x3fef387a6e756238ull, 0x3fef1e9df51fdee1ull, 0x3fef06fe0a31b715ull,                \
     0x3feef1a7373aa9cbull, 0x3feedea64c123422ull, 0x3feece086061892dull,                \
     0x3feebfdad5362a27ull, 0x3feeb42b569d4f82ull, 0x3feeab07dd485429ull,                \
     0x3feea47eb03a5585ull, 0x3feea09e667f3bcdull, 0x3fee9f75e8ec5f74ull,                \
     0x3feea11473eb0187ull, 0x3feea589994cce13ull, 0x3feeace5422aa0dbull,                \
     0x3feeb737b0cdc5e5ull, 0x3feec49182a3f090ull, 0x3feed503b23e255dull,                \
     0x3feee89f995ad3adull, 0x3feeff76f2fb5e47ull, 0x3fef199bdd85529cull,                \
     0x3fef3720dcef9069ull, 0x3fef5818dcfba487ull, 0x3fef7c97337b9b5full,                \
     0x3fefa4afa2a490daull, 0x3fefd0765b6e4540ull}

#if defined(__HIP_DEVICE_COMPILE__)
__device__ __constant__ static const uint64_t zs_exp2f_tab_dev[32] = ZS_EXP2F_TAB;
#define ZS_EXP2F_TABLE zs_exp2f_tab_dev
#else
static const uint64_t zs_exp2f_tab_host[32] = ZS_EXP2F_TAB;
#define ZS_EXP2F_TABLE zs_exp2f_tab_host
#endif

// (the table is an argument so that a kernel can read it from LDS)
ZS_HD float zs_expf_tab(float x, const uint64_t* tab) {
    const double InvLn2N = 0x1.71547652b82fep+0 * 32;
    const double SHIFT = 0x1.8p+52;
    const double C0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double C1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double C2 = 0x1.62e42ff0c52d6p-1 / 32;
    uint32_t ux = zs_f2u(x);
    uint32_t abstop = (ux >> 20) & 0x7ffu;
    if (abstop >= 0x42bu) {              // |x| >= 88 or nan
        if (ux == 0xff800000u) return 0.0f;
        if (abstop >= 0x7f8u) return x + x;
        if (x > 0x1.62e42ep6f) return zs_u2f(0x7f800000u);
        if (x < -0x1.9fe368p6f) return 0.0f;
    }
    double xd = (double)x;
    double z = InvLn2N * xd;
    double kd = z + SHIFT;
    uint64_t ki = zs_d2u(kd);
    kd -= SHIFT;
    double r = fma(InvLn2N, xd, -kd);
    uint64_t t = tab[ki & 31] + (ki << 47);
    double s = zs_u2d(t);
    double zz = fma(C0, r, C1);
    double r2 = r * r;
    double y = fma(C2, r, 1.0);
    y = fma(zz, r2, y);
    y = y * s;
    return (float)y;
}
ZS_HD float zs_expf(float x) { return zs_expf_tab(x, ZS_EXP2F_TABLE); }

// Rust f32::total_cmp order as an unsigned key: ascending key == ascending
// total order (-NaN < -inf < ... < -0 < +0 < ... < +inf < +NaN).
ZS_HD uint32_t zs_total_key(float f) {
    uint32_t b = zs_f2u(f);
    uint32_t k = b ^ ((uint32_t)((int32_t)b >> 31) >> 1);
    return k ^ 0x80000000u;
}
ZS_HD float zs_key_to_float(uint32_t k) {
    uint32_t b = k ^ 0x80000000u;
    b ^= ((uint32_t)((int32_t)b >> 31) >> 1);
    return zs_u2f(b);
}

// ---------------------------------------------------------------------------
// Philox4x32-10 (Salmon et al., SC'11).
// ---------------------------------------------------------------------------
ZS_HD void zs_philox(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                     uint32_t k1, uint32_t out[4]) {
    for (int r = 0; r < 10; r++) {
        uint64_t p0 = (uint64_t)0xD2511F53u * c0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * c2;
        uint32_t y0 = (uint32_t)(p1 >> 32) ^ c1 ^ k0;
        uint32_t y2 = (uint32_t)(p0 >> 32) ^ c3 ^ k1;
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = y0;
        c2 = y2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}
// First output word for (seed, counter, tag).
ZS_HD uint32_t zs_philox_u32(uint64_t seed, uint64_t counter, uint32_t tag) {
    uint32_t o[4];
    zs_philox((uint32_t)counter, (uint32_t)(counter >> 32), tag, 0u, (uint32_t)seed,
              (uint32_t)(seed >> 32), o);
    return o[0];
}
// Uniform f32 in [0, 1) with rand 0.9's f32 mapping: top 23 bits of a u32.
ZS_HD float zs_philox_uniform(uint64_t seed, uint64_t counter, uint32_t tag) {
    return (float)(zs_philox_u32(seed, counter, tag) >> 9) * 0x1p-23f;
}

// ---------------------------------------------------------------------------
// Exact sequential f32 summation of non-negative terms.
//
// While a running sum s stays inside one binade its values lie on the grid
// g = ulp(s) = 2^(max(E_s,1)-150) and s = k*g with k < 2^24. Adding a term t
// then gives (k + round_half_even(t/g)) * g, so each term contributes an integer
// increment independent of s -- except when t/g has fraction exactly 1/2 (the
// tie goes to the even neighbour, which depends on k) or when k + inc reaches
// 2^24 (the sum leaves the binade). Those two cases are "events" that the
// kernels resolve with a real f32 add; everything else is an integer prefix
// sum, which parallelises exactly.
// ---------------------------------------------------------------------------
#define ZS_INC_CAP (1u << 26)
#define ZS_BINADE (1u << 24)

// Grid exponent of a non-negative float s: max(E_s, 1). k0 = s / g.
ZS_HD int zs_grid_exp(float s) {
    int E = (int)((zs_f2u(s) >> 23) & 0xffu);
    return E > 1 ? E : 1;
}
ZS_HD uint32_t zs_grid_k(float s) {
    uint32_t b = zs_f2u(s) & 0x7fffffffu;
    uint32_t E = b >> 23;
    return E ? ((b & 0x7fffffu) | 0x800000u) : b;
}
// Float value k * 2^(eg-150) for k < 2^25 (exact).
ZS_HD float zs_grid_value(uint32_t k, int eg) {
    return ldexpf((float)k, eg - 150);
}
// Increment round_half_even(t / 2^(eg-150)) saturated at ZS_INC_CAP, and the
// exact-half flag. t must be >= 0 (a -0.0 is treated as 0).
ZS_HD uint32_t zs_seq_inc(float t, int eg, uint32_t* tie) {
    uint32_t b = zs_f2u(t) & 0x7fffffffu;
    int E = (int)(b >> 23);
    uint32_t m = E ? ((b & 0x7fffffu) | 0x800000u) : (b & 0x7fffffu);
    int ee = E ? E : 1;
    int d = ee - eg;
    *tie = 0;
    if (d > 0) return m ? ZS_INC_CAP : 0u;
    if (d == 0) return m;
    int sh = -d;
    if (sh >= 26) return 0u;
    uint32_t q = m >> sh;
    uint32_t rem = m & ((1u << sh) - 1u);
    uint32_t half = 1u << (sh - 1);
    *tie = (rem == half) ? 1u : 0u;
    return q + (rem > half ? 1u : 0u);
}
ZS_HD uint32_t zs_sat_add(uint32_t a, uint32_t b) {
    uint32_t c = a + b;
    return c > ZS_INC_CAP ? ZS_INC_CAP : c;
}
// Smallest integer K with K * 2^(eg-150) >= thresh (thresh may be NaN/inf:
// returns a value above any reachable k, i.e. "never").
ZS_HD uint32_t zs_grid_thresh(float thresh, int eg) {
    if (!(thresh == thresh)) return 0xffffffffu;       // NaN: comparison never true
    if (thresh <= 0.0f) return 0u;
    double q = ldexp((double)thresh, 150 - eg);
    if (q > 1e9) return 0xffffffffu;
    double c = ceil(q);
    return (uint32_t)c;
}
