// zs_sampler.h -- state and helpers shared by the sampler kernels
// (zs_sample.hip: the GPU-wide big-row kernels and the output kernel;
// zs_row.hip: the one-workgroup-per-row step).
#pragma once
#include <hip/hip_runtime.h>
#include "zs_internal.h"
#include "zs_dev.h"
#include "zs_seq.h"
#include "zs_terms.h"
struct zs_sargs {
    zs_batch b;
    uint32_t* p_cnt;
    uint32_t* p_id;
    uint32_t* p_flags;
    float* p_y;
    zs_row_state* rst;
    uint32_t* pairs;
    uint32_t* pv;
    uint32_t nch;
    uint32_t max_vocab;
    uint32_t* p_sub;
    uint32_t max_subs;
    double* k_ap;
    zs_sub_sum* k_sum;
    zs_tp_bucket* tp_bk;
    uint32_t* tp_cl;
    uint32_t* tp_pre;
    uint32_t* kcnt;
    zs_sub_sum* s_rec;
    float* s_apx;
    float* gath;
    float* s_hterm;
    uint32_t pstride;   // entries per row of the merged patch list (p_id, p_flags, p_y): max_vocab
};

#define ZS_ST_FALLBACK 0x200u

// zs_row.hip: the one-workgroup-per-row front of the step (patches, row
// statistics, candidates, greedy / small rows, the exact S and entropy sums)
extern "C" int zs_row_launch(const zs_sargs& a, hipStream_t stream);
// zs_sums.hip: the row sums S_obs and the sampler's S, then the entropy,
// spread over the GPU (one kernel per call, `which` 0..4 in launch order)
extern "C" int zs_sums_launch(const zs_sargs& a, uint32_t which, hipStream_t stream);

__device__ __forceinline__ bool zs_penalty_active(const zs_row_params& P) {
    return P.repeat != 1.0f || P.presence != 0.0f || P.frequency != 0.0f;
}
__device__ __forceinline__ float zs_temper(float y, float T) {
    // sampler.rs:47-51: divide only when T != 1 (T > 0 here)
    return (T > 0.0f && T != 1.0f) ? y / T : y;
}
__device__ __forceinline__ bool zs_allowed_bit(const zs_batch& b, uint32_t r, uint32_t idx) {
    uint32_t w = b.d_allow_bits[(size_t)r * b.allow_words + (idx >> 5)];
    return (w >> (idx & 31)) & 1u;
}

// Small survivor sets (n <= ZS_SMALL_CAP, all other logits are -inf after
// top-k / mask) are sampled exactly by one wave of the row kernel: zero terms
// of the reference's full-vocabulary loops do not change a running sum.
#define ZS_SMALL_CAP 512

// Ascending bitonic sort of 64*E u64 keys by one wave, element i = lane*E + e
// in register e of lane i / E: strides below E inside the lane, the others by
// lane exchanges.
template <int E>
__device__ __forceinline__ void wave_sort_u64_e(unsigned long long (&v)[E]) {
    const uint32_t lane = (uint32_t)zs_lane();
#pragma unroll
    for (uint32_t k = 2; k <= 64u * E; k <<= 1) {
#pragma unroll
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            if (j < (uint32_t)E) {
#pragma unroll
                for (uint32_t e = 0; e < (uint32_t)E; e++) {
                    const uint32_t pe = e ^ j;
                    if (pe > e) {
                        const bool asc = ((lane * E + e) & k) == 0u;
                        const unsigned long long x = v[e], y = v[pe];
                        if ((x > y) == asc) { v[e] = y; v[pe] = x; }
                    }
                }
            } else {
#pragma unroll
                for (uint32_t e = 0; e < (uint32_t)E; e++) {
                    const unsigned long long o = __shfl_xor(v[e], (int)(j / E), 64);
                    const uint32_t i = lane * E + e;
                    const bool asc = (i & k) == 0u, lower = (i & j) == 0u;
                    v[e] = (lower == asc) ? (o < v[e] ? o : v[e]) : (o > v[e] ? o : v[e]);
                }
            }
        }
    }
}

// Exact sampler over a small survivor set (n <= 64 * E, every other element
// below the top-k threshold, masked or -inf), by one wave: the reference's
// sequential f32 sums are done literally, one addition at a time in the
// reference's order, with no workgroup synchronisation (sampler.rs:46-127).
// Called by the 64 lanes of one wave; returns the token on every lane.
template <int E>
__device__ uint32_t small_path_wave(uint64_t seed, uint64_t counter, uint32_t V, const zs_row_params& P, uint32_t n, float m,
                                    const float* sval, const uint32_t* sidx) {
    const uint32_t lane = (uint32_t)zs_lane();
    // survivors by index: element i (sorted) in register i % E of lane i / E
    unsigned long long key[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        const uint32_t i = lane * E + e;
        key[e] = i < n ? (((unsigned long long)sidx[i] << 32) | zs_f2u(sval[i])) : ~0ull;
    }
    wave_sort_u64_e<E>(key);
    uint32_t id[E];
    float p[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        const bool live = lane * E + e < n;
        id[e] = (uint32_t)(key[e] >> 32);
        p[e] = live ? zs_expf(zs_u2f((uint32_t)key[e]) - m) : 0.0f;
    }
    // s0 + v[0] + v[1] + ... in order (sampler.rs:68, 80, 107)
    auto seq_sum = [&](const float (&v)[E], float s0) {
        float s = s0;
        for (uint32_t L = 0; L * E < n; L++)
#pragma unroll
            for (int e = 0; e < E; e++)
                if (L * E + e < n) s = s + zs_readlane_f(v[e], L);
        return s;
    };
    // softmax (sampler.rs:67-69)
    const float S = seq_sum(p, -0.0f);
#pragma unroll
    for (int e = 0; e < E; e++) p[e] = p[e] / S;
    // min-p (sampler.rs:72-88)
    if (P.min_p > 0.0f) {
        float pm = 0.0f;
#pragma unroll
        for (int e = 0; e < E; e++) if (lane * E + e < n) pm = fmaxf(pm, p[e]);
        pm = wave_max_f(pm);
        const float cut = P.min_p * pm;
#pragma unroll
        for (int e = 0; e < E; e++) if (p[e] < cut) p[e] = 0.0f;
        const float kept = seq_sum(p, 0.0f);
        if (kept > 0.0f)
#pragma unroll
            for (int e = 0; e < E; e++) p[e] = p[e] / kept;
    }
    // top-p (sampler.rs:91-115): cumsum in (p desc, idx asc) order
    if (P.top_p < 1.0f) {
        uint32_t vstar = 0, istar = 0xffffffffu;
        const bool none = !(P.top_p > 0.0f);  // cumsum 0 >= top_p: nothing kept
        if (!none) {
            unsigned long long k2[E];
#pragma unroll
            for (int e = 0; e < E; e++)
                k2[e] = lane * E + e < n ? (((unsigned long long)(~zs_f2u(p[e])) << 32) | id[e]) : ~0ull;
            wave_sort_u64_e<E>(k2);
            float cum = 0.0f;
            bool found = false;
            for (uint32_t L = 0; L * E < n && !found; L++) {
#pragma unroll
                for (int e = 0; e < E; e++) {
                    if (found || L * E + e >= n) continue;
                    const unsigned long long ks = zs_readlane_u64(k2[e], L);
                    cum = cum + zs_u2f(~(uint32_t)(ks >> 32));
                    if (cum >= P.top_p) {
                        vstar = ~(uint32_t)(ks >> 32);
                        istar = (uint32_t)ks;
                        found = true;
                    }
                }
            }
        }
        float f[E];
#pragma unroll
        for (int e = 0; e < E; e++) {
            const uint32_t pb = zs_f2u(p[e]);
            const bool keep = !none && (pb > vstar || (pb == vstar && id[e] <= istar));
            f[e] = keep ? p[e] : 0.0f;
        }
        const float sum = seq_sum(f, -0.0f);
        if (sum > 0.0f)
#pragma unroll
            for (int e = 0; e < E; e++) p[e] = f[e] / sum;
    }
    // draw (sampler.rs:118-127); r == 0 stops at index 0 whatever its p
    const float rr = zs_philox_uniform(seed, counter, 0u);
    if (rr <= 0.0f) return 0;
    float cum = 0.0f;
    for (uint32_t L = 0; L * E < n; L++) {
#pragma unroll
        for (int e = 0; e < E; e++) {
            if (L * E + e >= n) continue;
            cum = cum + zs_readlane_f(p[e], L);
            if (cum >= rr) return zs_readlane_u(id[e], L);
        }
    }
    return V - 1;
}

