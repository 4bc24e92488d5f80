// zs_spec.hip -- speculative-decode verification over k draft positions.
//
// temperature <= 0: greedy verification exactly as spec_decode.rs:241-279
// (accept drafts while argmax(target_i) == draft_i, first-max argmax with
// strict >, bonus = argmax of the first mismatching row or of row k).
//
// temperature > 0: rejection sampling (Leviathan et al. 2023; Chen et al.
// 2023), which the reference does not implement (rest.rs:2639). To make it
// reproducible bit-for-bit on any reduction order, probabilities are integer
// quantised: with z = x / T (f32, no division when T == 1), m = max z and
// e = expf(z - m) (glibc-identical), the weight of id v is
//   P_v = rint(e_v * 2^24)               (target),   Q_v likewise (draft).
// Draft i (token d) is accepted iff U_i * Q_d * sum(P) <= P_d * sum(Q) * 2^32,
// U_i the 32-bit Philox word of (seed, counter, tag 1+i). At the first
// rejection i the replacement token is drawn from R_v = max(0, P_v sum(Q) -
// Q_v sum(P)) (from P when sum(R) == 0) with tag 1+k+i; when all k drafts are
// accepted the bonus token is drawn from the target row k with tag 1+2k. A draw
// with weights W and word U returns the first id whose inclusive prefix of W
// exceeds floor(U * sum(W) / 2^32). Draft ids >= V are rejected. A row whose
// target or draft logits contain NaN / +inf or are all -inf is verified
// greedily.
#include <hip/hip_runtime.h>
#include "zs_internal.h"
#include "zs_dev.h"

#define SP_NT 256
#define SP_CH 8192
#define SP_BIG_NT 1024

typedef unsigned __int128 u128;


__device__ __forceinline__ const float* sp_row(const zs_spec_args& a, uint32_t r, uint32_t pos) {
    if (pos <= a.k) return a.target + ((size_t)r * (a.k + 1) + pos) * a.ld;
    return a.draft + ((size_t)r * a.k + (pos - a.k - 1)) * a.ld;
}
__device__ __forceinline__ float sp_z(float x, float T) { return (T > 0.0f && T != 1.0f) ? x / T : x; }
__device__ __forceinline__ uint64_t sp_weight(float z, float m) {
    float e = zs_expf(z - m);
    return (uint64_t)rint((double)e * 16777216.0);
}

// pass 1: per chunk max of z, flags, first-max argmax of x
__global__ __launch_bounds__(SP_NT) void zs_k_spec_stats(zs_spec_args a) {
    const uint32_t c = blockIdx.x, pos = blockIdx.y, r = blockIdx.z;
    const uint32_t npos = a.draft ? 2 * a.k + 1 : a.k + 1;
    if (pos >= npos) return;
    const uint32_t base = c * SP_CH;
    if (base >= a.V) return;
    __shared__ float fsh[SP_NT / 64];
    __shared__ uint32_t ush[SP_NT / 64];
    __shared__ unsigned long long gsh[SP_NT / 64];
    const float T = a.temperature[r];
    const float* row = sp_row(a, r, pos);
    float zmax = -INFINITY;
    uint32_t fl = 0;
    unsigned long long best = 0;  // (value key, ~idx): first strict max
    for (uint32_t i = base + threadIdx.x; i < min(a.V, base + SP_CH); i += SP_NT) {
        float x = row[i];
        float z = sp_z(x, T);
        if (z != z) fl |= 1u;
        else if (z == INFINITY) fl |= 2u;
        zmax = fmaxf(zmax, z);
        if (x > -INFINITY) {  // strict > over init -inf (NaN never wins)
            float xx = (x == 0.0f) ? 0.0f : x;
            unsigned long long k = ((unsigned long long)zs_total_key(xx) << 32) | (0xffffffffu - i);
            best = k > best ? k : best;
        }
    }
    zmax = block_max_f<SP_NT>(zmax, fsh);
    fl = block_or_u<SP_NT>(fl, ush);
    for (int d = 32; d > 0; d >>= 1) {
        unsigned long long o = __shfl_xor(best, d, 64);
        best = o > best ? o : best;
    }
    if (zs_lane() == 0) gsh[zs_wid()] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int i = 0; i < SP_NT / 64; i++) best = gsh[i] > best ? gsh[i] : best;
        zs_spec_chunk& o = a.cst[((size_t)r * a.npos_max + pos) * a.nch + c];
        o.zmax = zmax;
        o.flags = fl;
        o.amax_val = best ? zs_key_to_float((uint32_t)(best >> 32)) : -INFINITY;
        o.amax_idx = best ? 0xffffffffu - (uint32_t)(best & 0xffffffffull) : 0xffffffffu;
    }
}

// pass 2: chunk sums of the integer weights
__global__ __launch_bounds__(SP_NT) void zs_k_spec_sums(zs_spec_args a) {
    const uint32_t c = blockIdx.x, pos = blockIdx.y, r = blockIdx.z;
    const uint32_t npos = a.draft ? 2 * a.k + 1 : a.k + 1;
    if (pos >= npos) return;
    const uint32_t base = c * SP_CH;
    if (base >= a.V) return;
    const float T = a.temperature[r];
    if (!(T > 0.0f)) return;
    __shared__ unsigned long long sh[SP_NT / 64];
    const uint32_t nch = (a.V + SP_CH - 1) / SP_CH;
    const zs_spec_chunk* cs = a.cst + ((size_t)r * a.npos_max + pos) * a.nch;
    float m = -INFINITY;
    for (uint32_t i = 0; i < nch; i++) m = fmaxf(m, cs[i].zmax);
    const float* row = sp_row(a, r, pos);
    unsigned long long s = 0;
    if (m > -INFINITY && m < INFINITY)
        for (uint32_t i = base + threadIdx.x; i < min(a.V, base + SP_CH); i += SP_NT) s += sp_weight(sp_z(row[i], T), m);
    for (int d = 32; d > 0; d >>= 1) s += __shfl_xor(s, d, 64);
    if (zs_lane() == 0) sh[zs_wid()] = s;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (int i = 0; i < SP_NT / 64; i++) t += sh[i];
        a.cst[((size_t)r * a.npos_max + pos) * a.nch + c].wsum = t;
    }
}

// pass 3: one thread per row -- accept / reject decisions
__global__ void zs_k_spec_decide(zs_spec_args a) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.B) return;
    const uint32_t k = a.k, V = a.V;
    const uint32_t nch = (V + SP_CH - 1) / SP_CH;
    const uint32_t npos = a.draft ? 2 * k + 1 : k + 1;
    const float T = a.temperature[r];
    zs_spec_row out;
    out.m_t = out.m_d = 0.f;
    out.sum_t = out.sum_d = 0;
    // per position: max, flags, first-max argmax, weight sum
    bool degenerate = !(T > 0.0f) || !a.draft;
    float mpos[2 * ZS_SPEC_KMAX + 1];
    unsigned long long spos[2 * ZS_SPEC_KMAX + 1];
    uint32_t apos[ZS_SPEC_KMAX + 1];
    for (uint32_t p = 0; p < npos; p++) {
        const zs_spec_chunk* cs = a.cst + ((size_t)r * a.npos_max + p) * a.nch;
        float m = -INFINITY, bv = -INFINITY;
        uint32_t fl = 0, bi = 0xffffffffu;
        unsigned long long s = 0;
        for (uint32_t c = 0; c < nch; c++) {
            m = fmaxf(m, cs[c].zmax);
            fl |= cs[c].flags;
            if (cs[c].amax_idx != 0xffffffffu && (bi == 0xffffffffu || cs[c].amax_val > bv)) {
                bv = cs[c].amax_val;
                bi = cs[c].amax_idx;
            }
            s += cs[c].wsum;
        }
        if (p <= k) apos[p] = bi == 0xffffffffu ? 0u : bi;
        if (fl || m == -INFINITY) degenerate = true;
        mpos[p] = m;
        spos[p] = s;
    }
    const uint32_t* drafts = a.draft_ids + (size_t)r * k;
    if (degenerate) {
        uint32_t acc = 0, bonus = apos[k];
        for (uint32_t i = 0; i < k; i++) {
            if (apos[i] == drafts[i]) acc++;
            else { bonus = apos[i]; break; }
        }
        a.accepted[r] = acc;
        a.next[r] = bonus;
        out.mode = 0;
        a.rs[r] = out;
        return;
    }
    uint32_t i = 0;
    for (; i < k; i++) {
        uint32_t d = drafts[i];
        if (d >= V) break;
        uint64_t P = sp_weight(sp_z(sp_row(a, r, i)[d], T), mpos[i]);
        uint64_t Q = sp_weight(sp_z(sp_row(a, r, k + 1 + i)[d], T), mpos[k + 1 + i]);
        uint32_t U = zs_philox_u32(a.seed[r], a.counter[r], 1u + i);
        u128 lhs = (u128)U * Q * spos[i];
        u128 rhs = ((u128)P * spos[k + 1 + i]) << 32;
        if (!(lhs <= rhs)) break;
    }
    a.accepted[r] = i;
    out.mode = 1;
    out.pos = i;
    if (i == k) {
        out.residual = 0;
        out.m_t = mpos[k];
        out.sum_t = spos[k];
        out.word = zs_philox_u32(a.seed[r], a.counter[r], 1u + 2 * k);
    } else {
        out.residual = 1;
        out.m_t = mpos[i];
        out.m_d = mpos[k + 1 + i];
        out.sum_t = spos[i];
        out.sum_d = spos[k + 1 + i];
        out.word = zs_philox_u32(a.seed[r], a.counter[r], 1u + k + i);
    }
    a.rs[r] = out;
}

// u128 helpers for the workgroup scan
struct u128p { unsigned long long lo, hi; };
__device__ __forceinline__ u128 u128_of(u128p v) { return ((u128)v.hi << 64) | v.lo; }
__device__ __forceinline__ u128p u128p_of(u128 v) { return {(unsigned long long)v, (unsigned long long)(v >> 64)}; }
__device__ __forceinline__ u128 shfl_up_u128(u128 v, int d) {
    u128p p = u128p_of(v);
    p.lo = __shfl_up(p.lo, d, 64);
    p.hi = __shfl_up(p.hi, d, 64);
    return u128_of(p);
}
__device__ __forceinline__ u128 shfl_xor_u128(u128 v, int d) {
    u128p p = u128p_of(v);
    p.lo = __shfl_xor(p.lo, d, 64);
    p.hi = __shfl_xor(p.hi, d, 64);
    return u128_of(p);
}

struct spd_shared {
    unsigned long long lo[SP_BIG_NT / 64], hi[SP_BIG_NT / 64];
    int imin[SP_BIG_NT / 64];
    unsigned long long tlo, thi;
};

__device__ __forceinline__ u128 spd_weight(const zs_spec_args& a, const zs_spec_row& s, uint32_t r, float T,
                                           uint32_t v) {
    if (v >= a.V) return 0;
    uint64_t P = sp_weight(sp_z(sp_row(a, r, s.pos)[v], T), s.m_t);
    if (!s.residual) return P;
    uint64_t Q = sp_weight(sp_z(sp_row(a, r, a.k + 1 + s.pos)[v], T), s.m_d);
    u128 pp = (u128)P * s.sum_d, qq = (u128)Q * s.sum_t;
    return pp > qq ? pp - qq : 0;
}

// pass 4: one workgroup per row -- the replacement / bonus draw
__global__ __launch_bounds__(SP_BIG_NT) void zs_k_spec_draw(zs_spec_args a) {
    const uint32_t r = blockIdx.x;
    __shared__ spd_shared sh;
    zs_spec_row s = a.rs[r];
    if (s.mode != 1) return;
    const float T = a.temperature[r];
    const int t = threadIdx.x;
    const uint32_t V = a.V;
    // total weight (known for P; summed here for the residual)
    u128 total = s.sum_t;
    if (s.residual) {
        u128 acc = 0;
        for (uint32_t v = t; v < V; v += SP_BIG_NT) acc += spd_weight(a, s, r, T, v);
        for (int d = 32; d > 0; d >>= 1) acc += shfl_xor_u128(acc, d);
        if (zs_lane() == 0) { sh.lo[zs_wid()] = (unsigned long long)acc; sh.hi[zs_wid()] = (unsigned long long)(acc >> 64); }
        __syncthreads();
        total = 0;
        for (int i = 0; i < SP_BIG_NT / 64; i++) total += ((u128)sh.hi[i] << 64) | sh.lo[i];
        __syncthreads();
        if (total == 0) {  // p == q exactly: draw from the target instead
            s.residual = 0;
            total = s.sum_t;
        }
    }
    const u128 target = ((u128)s.word * total) >> 32;
    // first id whose inclusive prefix exceeds target, groups of 4*1024 ids
    u128 carry = 0;
    uint32_t found = 0xffffffffu;
    for (uint32_t g0 = 0; g0 < V && found == 0xffffffffu; g0 += 4 * SP_BIG_NT) {
        u128 w[4], loc = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) { w[q] = spd_weight(a, s, r, T, g0 + 4 * t + q); loc += w[q]; }
        // inclusive scan of loc over the workgroup
        u128 inc = loc;
        for (int d = 1; d < 64; d <<= 1) {
            u128 y = shfl_up_u128(inc, d);
            if (zs_lane() >= d) inc += y;
        }
        if (zs_lane() == 63) { sh.lo[zs_wid()] = (unsigned long long)inc; sh.hi[zs_wid()] = (unsigned long long)(inc >> 64); }
        __syncthreads();
        u128 pre = 0, tot = 0;
        for (int i = 0; i < SP_BIG_NT / 64; i++) {
            u128 wv = ((u128)sh.hi[i] << 64) | sh.lo[i];
            if (i < zs_wid()) pre += wv;
            tot += wv;
        }
        __syncthreads();
        u128 run = carry + pre + inc - loc;
        int my = ZS_BIGI;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            run += w[q];
            if (my == ZS_BIGI && w[q] > 0 && run > target) my = 4 * t + q;
        }
        int first = block_min_i<SP_BIG_NT>(my, sh.imin);
        if (first != ZS_BIGI) found = g0 + (uint32_t)first;
        carry += tot;
    }
    if (t == 0) a.next[r] = found == 0xffffffffu ? V - 1 : found;
}

extern "C" int zs_spec_launch(const zs_spec_args& a, hipStream_t stream) {
    const uint32_t npos = a.draft ? 2 * a.k + 1 : a.k + 1;
    const uint32_t nch = (a.V + SP_CH - 1) / SP_CH;
    dim3 grid(nch, npos, a.B);
    hipLaunchKernelGGL(zs_k_spec_stats, grid, dim3(SP_NT), 0, stream, a);
    hipLaunchKernelGGL(zs_k_spec_sums, grid, dim3(SP_NT), 0, stream, a);
    hipLaunchKernelGGL(zs_k_spec_decide, dim3((a.B + 63) / 64), dim3(64), 0, stream, a);
    hipLaunchKernelGGL(zs_k_spec_draw, dim3(a.B), dim3(SP_BIG_NT), 0, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
