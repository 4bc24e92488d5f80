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
    zs_sub_sum* k_xsum;  // crossing records beside k_sum (same indexing)
    zs_tp_bucket* tp_bk;
    uint32_t* tp_cl;
    uint32_t* tp_pre;
    uint32_t* kcnt;
    uint32_t* tp_task;   // buckets zs_k_tp_sort presorts: count, then (row << 8 | candidate)
    zs_sub_sum* s_rec;
    zs_sub_sum* s_xrec;  // crossing records beside s_rec (same indexing)
    float* s_apx;
    float* gath;
    float* s_hterm;
    uint32_t pstride;   // entries per row of the merged patch list (p_id, p_flags, p_y): max_vocab
    uint32_t row_split; // zs_k_row: 2B workgroups, rows may split their stream in two halves
    unsigned long long* rw_part;
    uint32_t* rw_ctr;
};

#define ZS_ST_FALLBACK 0x200u

// zs_row.hip: the per-row front of the step (patches, row statistics,
// candidates, greedy and small rows)
extern "C" int zs_row_launch(const zs_sargs& a, hipStream_t stream);
// zs_sums.hip: the row sums (the big rows' sampler S; S_obs, then the
// entropy) spread over the GPU (one kernel per call, `which` 0..7)
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

#ifndef ZS_SP_T
#define ZS_SP_T(i) do { } while (0)
#endif

// The wave's values (element i = lane * E + e in register e of lane i / E;
// the first n) written to LDS scratch in element order, for a serial pass.
template <int E>
__device__ __forceinline__ void wave_stage_f(float* buf, const float (&v)[E], uint32_t n) {
    const uint32_t lane = (uint32_t)zs_lane();
#pragma unroll
    for (int e = 0; e < E; e++)
        if (lane * E + e < n) buf[lane * E + e] = v[e];
    __builtin_amdgcn_s_waitcnt(0);   // the wave's own LDS writes before its reads
    __builtin_amdgcn_wave_barrier();
}
// Index of the first element after which s0 + buf[0] + ... + buf[i] (f32,
// one addition at a time in order) reaches thresh (never for NaN); n if none.
// *s gets the sum up to and including that element (all n when none). Every
// lane runs it on the same LDS values (broadcast reads) and ends with the same
// result.
__device__ __forceinline__ uint32_t serial_scan_f(const float* buf, uint32_t n, float s0, float thresh, float* s) {
    float acc = s0;
    uint32_t i = 0;
    for (; i + 4 <= n; i += 4) {
        const float4 q = *reinterpret_cast<const float4*>(buf + i);
        acc = acc + q.x;
        if (acc >= thresh) { *s = acc; return i; }
        acc = acc + q.y;
        if (acc >= thresh) { *s = acc; return i + 1; }
        acc = acc + q.z;
        if (acc >= thresh) { *s = acc; return i + 2; }
        acc = acc + q.w;
        if (acc >= thresh) { *s = acc; return i + 3; }
    }
    for (; i < n; i++) {
        acc = acc + buf[i];
        if (acc >= thresh) { *s = acc; return i; }
    }
    *s = acc;
    return n;
}

// Exact sampler over a small survivor set (n <= 64 * E, every other element
// below the top-k threshold, masked or -inf), by one wave: the reference's
// sequential f32 sums are done literally, one addition at a time in the
// reference's order, with no workgroup synchronisation (sampler.rs:46-127).
// The additions run over LDS copies of the values (sval, sidx: the survivors
// on entry, then scratch; 16-byte aligned). Called by the 64 lanes of one
// wave; returns the token on every lane.
template <int E>
__device__ uint32_t small_path_wave(uint64_t seed, uint64_t counter, uint32_t V, const zs_row_params& P, uint32_t n, float m,
                                    float* sval, uint32_t* sidx) {
    const uint32_t lane = (uint32_t)zs_lane();
#ifdef ZS_WALK_DEBUG
    unsigned long long sp_t0 = wall_clock64();
#endif
    // survivors by index: element i (sorted) in register i % E of lane i / E
    unsigned long long key[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        const uint32_t i = lane * E + e;
        key[e] = i < n ? (((unsigned long long)sidx[i] << 32) | zs_f2u(sval[i])) : ~0ull;
    }
    wave_sort_u64_e<E>(key);
    ZS_SP_T(0);
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
        wave_stage_f<E>(sval, v, n);
        float s;
        serial_scan_f(sval, n, s0, NAN, &s);
        __builtin_amdgcn_wave_barrier();
        return s;
    };
    // softmax (sampler.rs:67-69)
    ZS_SP_T(1);
    const float S = seq_sum(p, -0.0f);
#pragma unroll
    for (int e = 0; e < E; e++) p[e] = p[e] / S;
    ZS_SP_T(2);
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
            ZS_SP_T(3);
            float ps[E];
#pragma unroll
            for (int e = 0; e < E; e++) {
                ps[e] = zs_u2f(~(uint32_t)(k2[e] >> 32));
                if (lane * E + e < n) sidx[lane * E + e] = (uint32_t)k2[e];
            }
            wave_stage_f<E>(sval, ps, n);
            float cum;
            const uint32_t i = serial_scan_f(sval, n, 0.0f, P.top_p, &cum);
            if (i < n) {
                vstar = zs_f2u(sval[i]);
                istar = sidx[i];
            }
            __builtin_amdgcn_wave_barrier();
            ZS_SP_T(4);
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
        ZS_SP_T(5);
    }
    // draw (sampler.rs:118-127); r == 0 stops at index 0 whatever its p
    const float rr = zs_philox_uniform(seed, counter, 0u);
    if (rr <= 0.0f) return 0;
#pragma unroll
    for (int e = 0; e < E; e++)
        if (lane * E + e < n) sidx[lane * E + e] = id[e];
    wave_stage_f<E>(sval, p, n);
    float cum;
    const uint32_t i = serial_scan_f(sval, n, 0.0f, rr, &cum);
    ZS_SP_T(6);
    return i < n ? sidx[i] : V - 1;
}

