// zs_terms.h -- term functors for the exact sequential sums of zs_seq.h.
//
// A sequential sum only needs each term's increment round_half_even(t/g) on the
// current grid g. For the exponential terms a fast f32 exp (range reduction
// + v_exp_f32, relative error below ZS_EXP_EPS, calibrated over every input
// of its domain by tests/test_gpu_calib.py) decides the increment whenever the
// approximate t/g is farther than its error band from a half-integer; the
// remaining terms (a few per row) are recomputed exactly with the
// glibc-identical zs_expf. Event terms always use the exact value.
#pragma once
#include "zs_seq.h"

#define ZS_EXP_EPS 0x1p-21   // measured: 2^-23 over the whole domain (the sweep asserts below 2^-22)
#define ZS_EXP_FAST_MIN -87.0f   // below: subnormal results, use the exact path
#define ZS_EXP_ZERO -104.0f      // below: glibc expf returns 0

__device__ __forceinline__ float zs_exp_fast(float d) {
    const float L2E = 1.44269502162933349609375f;    // f32(log2 e)
    const float L2E_LO = 1.925963033500772e-8f;       // log2 e - L2E
    float t = d * L2E;
    float tl = fmaf(d, L2E, -t);
    tl = fmaf(d, L2E_LO, tl);
    float n = rintf(t);
    float f = (t - n) + tl;
    float y = __builtin_amdgcn_exp2f(f);
    return ldexpf(y, (int)n);
}

// A cheaper exp for approximate sums only (the grid predictions of the row
// sums, zs_k_sapx: a wrong prediction costs time, never exactness): 2^(d *
// f32(log2 e)) by v_exp_f32 alone, for d in [ZS_EXP_FAST_MIN, 1]. Its relative
// error against zs_expf (the argument's rounding, at most |d log2 e| 2^-24,
// dominates) is measured by tests/test_gpu_calib.py over every input.
#define ZS_EXP_HW_EPS 0x1p-16
__device__ __forceinline__ float zs_exp_hw(float d) {
    return __builtin_amdgcn_exp2f(d * 1.44269502162933349609375f);
}

// Certified increment of an approximate term a (|a - t| <= ZS_EXP_EPS * t).
__device__ __forceinline__ bool zs_cert_inc(float a, int eg, uint32_t* inc) {
    double q = ldexp((double)a, 150 - eg);
    if (q >= 8388608.0) return false;
    double fl = floor(q);
    double fr = q - fl;
    if (fabs(fr - 0.5) <= q * ZS_EXP_EPS + 1e-30) return false;
    *inc = (uint32_t)fl + (fr > 0.5 ? 1u : 0u);
    return true;
}

template <int EPT>
__device__ __forceinline__ float zs_pick(const float (&v)[EPT], int j) { return seq_pick_f(v, j); }

// term = expf(d) (softmax numerators: sampler.rs:68, logprobs.rs:36, hallucination.rs:135)
template <int EPT>
struct exp_terms {
    float d[EPT], a[EPT];
    __device__ __forceinline__ void set(int j, float dj) {
        d[j] = dj;
        a[j] = (dj >= ZS_EXP_FAST_MIN) ? zs_exp_fast(dj) : (dj < ZS_EXP_ZERO ? 0.0f : -1.0f);
    }
    __device__ __forceinline__ float exact(int j) const { return zs_expf(zs_pick(d, j)); }
    __device__ __forceinline__ void inc(int j, int eg, uint32_t* ie, uint32_t* io) const {
        float aj = zs_pick(a, j);
        uint32_t q;
        if (aj == 0.0f) { *ie = *io = 0u; return; }
        if (aj > 0.0f && zs_cert_inc(aj, eg, &q)) { *ie = *io = q; return; }
        seq_pair p = seq_pair_of(exact(j), eg);
        *ie = p.e;
        *io = p.o;
    }
    __device__ __forceinline__ float val(int j) const { return exact(j); }
};

// term = -(p * ((l - max) - ln_sum)) with p = expf(l - max) * inv, 0 unless p > 0
// (hallucination.rs:143: `entropy -= p * ((l - max) - ln_sum)`).
template <int EPT>
struct ent_terms {
    float d[EPT], a[EPT];
    float inv, lns;
    __device__ __forceinline__ void set(int j, float dj) {
        d[j] = dj;
        if (dj >= ZS_EXP_FAST_MIN) a[j] = -((zs_exp_fast(dj) * inv) * (dj - lns));
        else a[j] = (dj < ZS_EXP_ZERO) ? 0.0f : -1.0f;
    }
    __device__ __forceinline__ float exact(int j) const {
        float dj = zs_pick(d, j);
        float p = zs_expf(dj) * inv;
        if (!(p > 0.0f)) return 0.0f;
        float tt = dj - lns;
        return -(p * tt);
    }
    __device__ __forceinline__ void inc(int j, int eg, uint32_t* ie, uint32_t* io) const {
        float aj = zs_pick(a, j);
        uint32_t q;
        if (aj == 0.0f) { *ie = *io = 0u; return; }
        if (aj > 0.0f && zs_cert_inc(aj, eg, &q)) { *ie = *io = q; return; }
        seq_pair p = seq_pair_of(exact(j), eg);
        *ie = p.e;
        *io = p.o;
    }
    __device__ __forceinline__ float val(int j) const { return exact(j); }
};
