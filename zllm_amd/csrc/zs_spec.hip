// zs_spec.hip -- speculative-decode verification over k draft positions.
//
// temperature <= 0: greedy verification exactly as spec_decode.rs:241-279
// (accept drafts while argmax(target_i) == draft_i, first-max argmax with
// strict >, bonus = argmax of the first mismatching row or of row k).
//
// temperature > 0: rejection sampling (Leviathan et al. 2023; Chen et al.
// 2023), which the reference does not implement (rest.rs:2639). To make it
// reproducible bit-for-bit on any reduction order, probabilities are integer
// quantised: with m = max x (NaN ignored) and c = log2(e) / T (one f32
// division per row), the weight of id v is
//   P_v = rint(2^24 * 2^t),  t = (x_v - m) * c   (target),   Q_v likewise (draft),
// from a fixed sequence of f32 operations (sp_weight), 0 below t = -25 (where
// the formula itself rounds to 0). No per-element division by T is needed.
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
#include <mutex>

#define SP_NT 256
#define SP_CH 8192
#define SP_EPT (SP_CH / SP_NT)   // 32 elements per thread, as 8 float4
#define SP_BIG_NT 1024
// weights are 0 below this log-ratio
#define SP_ZERO_T (-25.0f)

typedef unsigned __int128 u128;

__device__ __forceinline__ const float* sp_row(const zs_spec_args& a, uint32_t r, uint32_t pos) {
    if (pos <= a.k) return a.target + ((size_t)r * (a.k + 1) + pos) * a.ld;
    return a.draft + ((size_t)r * a.k + (pos - a.k - 1)) * a.ld;
}
// c = log2(e) / T, the factor of the exponent (T > 0)
__device__ __forceinline__ float sp_c(float T) { return __fdiv_rn(1.44269502f, T); }
// Integer weight rint(2^24 * 2^t), t = (x - m) * c, through a fixed sequence of
// correctly rounded f32 operations (t = n + f with n = floor(t), 2^f by a
// degree-7 Taylor polynomial in fmaf Horner form, exact scaling by 2^(24+n),
// rint), so the CPU restatement reproduces every weight bit for bit. t < -25
// gives 2^f * 2^(24+n) < 0.5, i.e. 0. For x <= m the weight is below 2^25, so
// 32 of them add up in 32 bits.
__device__ __forceinline__ uint32_t sp_weight(float x, float m, float c) {
    const float t = __fmul_rn(__fsub_rn(x, m), c);
    const float n = floorf(t);
    const float f = __fsub_rn(t, n);
    float p = 1.52527338e-05f;
    p = fmaf(p, f, 1.54035304e-04f);
    p = fmaf(p, f, 1.33335581e-03f);
    p = fmaf(p, f, 9.61812911e-03f);
    p = fmaf(p, f, 5.55041087e-02f);
    p = fmaf(p, f, 2.40226507e-01f);
    p = fmaf(p, f, 6.93147182e-01f);
    p = fmaf(p, f, 1.0f);
    const uint32_t w = (uint32_t)rintf(ldexpf(p, 24 + (int)n));
    return t >= SP_ZERO_T ? w : 0u;
}
// whether any x <= xc can have a positive weight
__device__ __forceinline__ bool sp_live(float xc, float m, float c) {
    return __fmul_rn(__fsub_rn(xc, m), c) >= SP_ZERO_T;
}
// the chunk's elements of thread t: float4 j covers ids base + (j*SP_NT + t)*4 .. +3
__device__ __forceinline__ void sp_load(const float* row, uint32_t base, uint32_t V, float (&x)[SP_EPT]) {
#pragma unroll
    for (int j = 0; j < SP_EPT / 4; j++) {
        const uint32_t id = base + (j * SP_NT + threadIdx.x) * 4;
        float4 v = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        if (id < V) v = *reinterpret_cast<const float4*>(row + id);
        x[4 * j] = v.x; x[4 * j + 1] = v.y; x[4 * j + 2] = v.z; x[4 * j + 3] = v.w;
    }
    if (base + SP_CH > V) {  // ids past V read as -inf (neutral in every pass)
#pragma unroll
        for (int e = 0; e < SP_EPT; e++)
            if (base + ((e >> 2) * SP_NT + threadIdx.x) * 4 + (e & 3) >= V) x[e] = -INFINITY;
    }
}
__device__ __forceinline__ uint32_t sp_id(uint32_t base, int e) {
    return base + ((e >> 2) * SP_NT + threadIdx.x) * 4 + (e & 3);
}

// One pass per chunk: the chunk maximum, flags, the first strict maximum of x
// (greedy verification) and, once the chunk maximum is known, the chunk sum of
// the weights w_v = W((x_v - m_c) c).
__global__ __launch_bounds__(SP_NT) void zs_k_spec_chunk(zs_spec_args a) {
    const uint32_t c = blockIdx.x, pos = blockIdx.y, r = blockIdx.z;
    const uint32_t npos = a.draft ? 2 * a.k + 1 : a.k + 1;
    if (pos >= npos) return;
    const uint32_t base = c * SP_CH;
    if (base >= a.V) return;
    __shared__ float fsh[SP_NT / 64];
    __shared__ uint32_t ush[SP_NT / 64];
    __shared__ unsigned long long gsh[SP_NT / 64], wsh[SP_NT / 64];
    float x[SP_EPT];
    sp_load(sp_row(a, r, pos), base, a.V, x);
    // first strict maximum (init -inf, NaN never wins) in index order: the
    // elements of a thread ascend with e; it is also the NaN-ignoring max
    float bv = -INFINITY;
    int be = -1;
    bool nan = false;
#pragma unroll
    for (int e = 0; e < SP_EPT; e++) {
        const float xv = x[e];
        nan |= xv != xv;
        if (xv > bv) { bv = xv; be = e; }
    }
    uint32_t fl = nan ? 1u : 0u;
    if (bv == INFINITY) fl |= 2u;
    // (value key, ~idx): larger value first, then the lower id; -0 == +0
    unsigned long long best = be < 0 ? 0ull
        : ((unsigned long long)zs_total_key(bv == 0.0f ? 0.0f : bv) << 32) | (0xffffffffu - sp_id(base, be));
    const float xmax = block_max_f<SP_NT>(bv, fsh);
    fl = block_or_u<SP_NT>(fl, ush);
    for (int d = 32; d > 0; d >>= 1) {
        unsigned long long o = __shfl_xor(best, d, 64);
        best = o > best ? o : best;
    }
    // chunk sum of the weights relative to the chunk maximum (at most 32
    // weights below 2^25 each per thread)
    const float T = a.temperature[r];
    unsigned long long wsum = 0;
    if (T > 0.0f && a.draft && xmax > -INFINITY && xmax < INFINITY) {
        const float cT = sp_c(T);
        uint32_t s32 = 0;
#pragma unroll
        for (int e = 0; e < SP_EPT; e++) s32 += sp_weight(x[e], xmax, cT);
        wsum = s32;
        for (int d = 32; d > 0; d >>= 1) wsum += __shfl_xor(wsum, d, 64);
    }
    if (zs_lane() == 0) { gsh[zs_wid()] = best; wsh[zs_wid()] = wsum; }
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long ws = 0;
        for (int i = 0; i < SP_NT / 64; i++) { best = gsh[i] > best ? gsh[i] : best; ws += wsh[i]; }
        zs_spec_chunk& o = a.cst[((size_t)r * a.npos_max + pos) * a.nch + c];
        o.xmax = xmax;
        o.flags = fl;
        o.amax_val = best ? zs_key_to_float((uint32_t)(best >> 32)) : -INFINITY;
        o.amax_idx = best ? 0xffffffffu - (uint32_t)(best & 0xffffffffull) : 0xffffffffu;
        o.wsum = ws;
    }
}

// The same per (row, position) by one workgroup walking the row's chunks once,
// two at a time. One workgroup per CU (its LDS request keeps a second one out):
// the verification then leaves most of each CU to the sampler's kernels when
// the two run side by side.
#define SR_NT 1024
#define SR_NW (SR_NT / 64)
#define SR_EPT (SP_CH / SR_NT)  // 8 elements per thread, as 2 float4
#define SR_PAIR 2               // chunks loaded together
#define SR_LDS_HOLD 90000       // bytes of LDS requested to keep occupancy at one workgroup per CU
__device__ __forceinline__ void sr_load(const float* row, uint32_t base, uint32_t V, float* x) {
#pragma unroll
    for (int j = 0; j < SR_EPT / 4; j++) {
        const uint32_t id = base + (j * SR_NT + threadIdx.x) * 4;
        float4 v = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        if (id < V) v = *reinterpret_cast<const float4*>(row + id);
        x[4 * j] = v.x; x[4 * j + 1] = v.y; x[4 * j + 2] = v.z; x[4 * j + 3] = v.w;
    }
    if (base + SP_CH > V) {  // ids past V read as -inf
#pragma unroll
        for (int e = 0; e < SR_EPT; e++)
            if (base + ((e >> 2) * SR_NT + threadIdx.x) * 4 + (e & 3) >= V) x[e] = -INFINITY;
    }
}
__device__ __forceinline__ uint32_t sr_id(uint32_t base, int e) {
    return base + ((e >> 2) * SR_NT + threadIdx.x) * 4 + (e & 3);
}

__global__ __launch_bounds__(SR_NT) void zs_k_spec_row(zs_spec_args a) {
    extern __shared__ uint32_t hold[];  // occupancy limiter only
    const uint32_t pos = blockIdx.x, r = blockIdx.y;
    const uint32_t V = a.V;
    const uint32_t nch = (V + SP_CH - 1) / SP_CH;
    __shared__ float wz[SR_PAIR][SR_NW];
    __shared__ uint32_t wf[ZS_MAX_CHUNKS][SR_NW];
    __shared__ unsigned long long wb[ZS_MAX_CHUNKS][SR_NW];
    __shared__ unsigned long long ws[ZS_MAX_CHUNKS][SR_NW];
    __shared__ float cz[ZS_MAX_CHUNKS];
    if (threadIdx.x == 0) hold[0] = 0;  // the request is used, so it is kept
    const float T = a.temperature[r];
    const bool weights = T > 0.0f && a.draft;
    const float cT = weights ? sp_c(T) : 1.0f;
    const float* row = sp_row(a, r, pos);
    const int lane = zs_lane(), wid = zs_wid();
    zs_spec_chunk* cs = a.cst + ((size_t)r * a.npos_max + pos) * a.nch;
    for (uint32_t c0 = 0; c0 < nch; c0 += SR_PAIR) {
        float x[SR_PAIR][SR_EPT];
#pragma unroll
        for (int h = 0; h < SR_PAIR; h++) sr_load(row, (c0 + h) * SP_CH, V, x[h]);
#pragma unroll
        for (int h = 0; h < SR_PAIR; h++) {
            const uint32_t c = c0 + h;
            if (c >= nch) break;
            const uint32_t base = c * SP_CH;
            float bv = -INFINITY;
            int be = -1;
            bool nan = false;
#pragma unroll
            for (int e = 0; e < SR_EPT; e++) {
                const float xv = x[h][e];
                nan |= xv != xv;
                if (xv > bv) { bv = xv; be = e; }
            }
            uint32_t fl = nan ? 1u : 0u;
            unsigned long long best = be < 0 ? 0ull
                : ((unsigned long long)zs_total_key(bv == 0.0f ? 0.0f : bv) << 32) | (0xffffffffu - sr_id(base, be));
            const float xmax = wave_max_f(bv);
            fl = wave_or_u(fl);
            for (int d = 32; d > 0; d >>= 1) {
                unsigned long long o = __shfl_xor(best, d, 64);
                best = o > best ? o : best;
            }
            if (lane == 0) { wz[h][wid] = xmax; wf[c][wid] = fl; wb[c][wid] = best; }
        }
        __syncthreads();
        // chunk maxima, then the chunk weight sums from the registers
#pragma unroll
        for (int h = 0; h < SR_PAIR; h++) {
            const uint32_t c = c0 + h;
            if (c >= nch) break;
            float m = -INFINITY;
            for (int w = 0; w < SR_NW; w++) m = fmaxf(m, wz[h][w]);
            if (threadIdx.x == 0) cz[c] = m;
            unsigned long long s = 0;
            if (weights && m > -INFINITY && m < INFINITY) {
                uint32_t s32 = 0;  // at most 8 weights below 2^25 each
#pragma unroll
                for (int e = 0; e < SR_EPT; e++) s32 += sp_weight(x[h][e], m, cT);
                s = s32;
                for (int d = 32; d > 0; d >>= 1) s += __shfl_xor(s, d, 64);
            }
            if (lane == 0) ws[c][wid] = s;
        }
        __syncthreads();
    }
    if (threadIdx.x < nch) {
        const uint32_t c = threadIdx.x;
        uint32_t fl = 0;
        unsigned long long best = 0, s = 0;
        for (int w = 0; w < SR_NW; w++) {
            fl |= wf[c][w];
            best = wb[c][w] > best ? wb[c][w] : best;
            s += ws[c][w];
        }
        if (cz[c] == INFINITY) fl |= 2u;
        zs_spec_chunk& o = cs[c];
        o.xmax = cz[c];
        o.flags = fl;
        o.amax_val = best ? zs_key_to_float((uint32_t)(best >> 32)) : -INFINITY;
        o.amax_idx = best ? 0xffffffffu - (uint32_t)(best & 0xffffffffull) : 0xffffffffu;
        o.wsum = s;
    }
}

// bit length of a u128
__device__ __forceinline__ int sp_bitlen(u128 v) {
    const unsigned long long hi = (unsigned long long)(v >> 64), lo = (unsigned long long)v;
    return hi ? 128 - __clzll((long long)hi) : (lo ? 64 - __clzll((long long)lo) : 0);
}
// sum of a row's weights, sum_c F_c * S_c, by one wave (lanes over chunks);
// every lane gets it
__device__ __forceinline__ u128 sp_row_sum(const zs_spec_chunk* cs, uint32_t nch, float M, float cT) {
    u128 s = 0;
    for (uint32_t c = (uint32_t)zs_lane(); c < nch; c += 64)
        s += (u128)((unsigned long long)sp_weight(cs[c].xmax, M, cT) * cs[c].wsum);
    for (int d = 32; d > 0; d >>= 1) {
        const unsigned long long lo = __shfl_xor((unsigned long long)s, d, 64);
        const unsigned long long hi = __shfl_xor((unsigned long long)(s >> 64), d, 64);
        s += ((u128)hi << 64) | lo;
    }
    return s;
}

// pass 2: one wave per row -- accept / reject decisions (lanes over chunks)
// and the sums of the final draw
__global__ __launch_bounds__(64) void zs_k_spec_decide(zs_spec_args a) {
    const uint32_t r = blockIdx.x;
    const int lane = zs_lane();
    const uint32_t k = a.k, V = a.V;
    const uint32_t nch = (V + SP_CH - 1) / SP_CH;
    const uint32_t npos = a.draft ? 2 * k + 1 : k + 1;
    const float T = a.temperature[r];
    zs_spec_row out;
    out.m_t = out.m_d = 0.f;
    out.ps = out.qs = 0;
    out.sum_lo = out.sum_hi = 0;
    bool degenerate = !(T > 0.0f) || !a.draft;
    float mpos[2 * ZS_SPEC_KMAX + 1];
    uint32_t apos[ZS_SPEC_KMAX + 1];
    auto cst = [&](uint32_t p) { return a.cst + ((size_t)r * a.npos_max + p) * a.nch; };
    for (uint32_t p = 0; p < npos; p++) {
        const zs_spec_chunk* cs = cst(p);
        float m = -INFINITY;
        uint32_t fl = 0;
        unsigned long long best = 0;  // (value key, ~id) of the first maximum
        for (uint32_t c = lane; c < nch; c += 64) {
            const zs_spec_chunk q = cs[c];
            m = fmaxf(m, q.xmax);
            fl |= q.flags;
            if (q.amax_idx != 0xffffffffu) {
                const unsigned long long key = ((unsigned long long)zs_total_key(q.amax_val) << 32) | (0xffffffffu - q.amax_idx);
                best = key > best ? key : best;
            }
        }
        m = wave_max_f(m);
        fl = wave_or_u(fl);
        for (int d = 32; d > 0; d >>= 1) {
            unsigned long long o = __shfl_xor(best, d, 64);
            best = o > best ? o : best;
        }
        if (fl || m == -INFINITY) degenerate = true;
        if (p <= k) apos[p] = best ? 0xffffffffu - (uint32_t)(best & 0xffffffffull) : 0u;
        mpos[p] = m;
    }
    const uint32_t* drafts = a.draft_ids + (size_t)r * k;
    if (degenerate) {
        if (lane != 0) return;
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
    const float cT = sp_c(T);
    // P_d = w_d * F_c of the chunk holding d
    auto weight_at = [&](uint32_t p, uint32_t d) -> unsigned long long {
        const float mc = cst(p)[d / SP_CH].xmax;
        return (unsigned long long)sp_weight(sp_row(a, r, p)[d], mc, cT) * sp_weight(mc, mpos[p], cT);
    };
    uint32_t i = 0;
    u128 sp = 0, sq = 0;
    int sh = 0;
    for (; i < k; i++) {
        sp = sp_row_sum(cst(i), nch, mpos[i], cT);
        sq = sp_row_sum(cst(k + 1 + i), nch, mpos[k + 1 + i], cT);
        sh = max(0, sp_bitlen(sp | sq) - 40);
        const uint32_t d = drafts[i];
        if (d >= V) break;
        const unsigned long long Ps = (unsigned long long)(sp >> sh), Qs = (unsigned long long)(sq >> sh);
        const unsigned long long P = weight_at(i, d), Q = weight_at(k + 1 + i, d);
        const uint32_t U = zs_philox_u32(a.seed[r], a.counter[r], 1u + i);
        const u128 lhs = ((u128)U * Q) * Ps;  // < 2^122
        const u128 rhs = ((u128)P * Qs) << 32;                      // < 2^122
        if (!(lhs <= rhs)) break;
    }
    out.mode = 1;
    out.pos = i;
    if (i == k) {
        const u128 st = sp_row_sum(cst(k), nch, mpos[k], cT);
        out.residual = 0;
        out.m_t = mpos[k];
        out.sum_lo = (unsigned long long)st;
        out.sum_hi = (unsigned long long)(st >> 64);
        out.word = zs_philox_u32(a.seed[r], a.counter[r], 1u + 2 * k);
    } else {
        out.residual = 1;
        out.m_t = mpos[i];
        out.m_d = mpos[k + 1 + i];
        out.ps = (unsigned long long)(sp >> sh);
        out.qs = (unsigned long long)(sq >> sh);
        out.sum_lo = (unsigned long long)sp;  // the target's sum: the draw when R is all 0
        out.sum_hi = (unsigned long long)(sp >> 64);
        out.word = zs_philox_u32(a.seed[r], a.counter[r], 1u + k + i);
    }
    if (lane != 0) return;
    a.accepted[r] = i;
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

// Draw weight of id v (given its target / draft logits and its chunk's maxima
// and scales): P, or the residual max(0, P Qs - Q Ps) (below 2^90).
struct sp_chunk_w {
    float mt, md;
    unsigned long long ft, fd;
};
// tpos: the target position the draw's P comes from (pos after a rejection,
// k after k acceptances)
__device__ __forceinline__ sp_chunk_w sp_chunk_scales(const zs_spec_args& a, uint32_t r, const zs_spec_row& s, uint32_t c,
                                                      float cT, uint32_t tpos) {
    sp_chunk_w w;
    w.mt = a.cst[((size_t)r * a.npos_max + tpos) * a.nch + c].xmax;
    w.ft = sp_weight(w.mt, s.m_t, cT);
    w.md = 0.0f;
    w.fd = 0;
    if (s.residual) {
        w.md = a.cst[((size_t)r * a.npos_max + a.k + 1 + s.pos) * a.nch + c].xmax;
        w.fd = sp_weight(w.md, s.m_d, cT);
    }
    return w;
}
__device__ __forceinline__ u128 spd_weight2(const zs_spec_row& s, const sp_chunk_w& cw, float cT, float xt, float xd) {
    const unsigned long long P = (unsigned long long)sp_weight(xt, cw.mt, cT) * cw.ft;
    if (!s.residual) return P;
    const unsigned long long Q = (unsigned long long)sp_weight(xd, cw.md, cT) * cw.fd;
    const u128 pp = (u128)P * s.qs, qq = (u128)Q * s.ps;
    return pp > qq ? pp - qq : 0;
}

// pass 3: chunk sums of the residual weights (rows that rejected a draft)
__global__ __launch_bounds__(SP_NT) void zs_k_spec_rsum(zs_spec_args a) {
    const uint32_t c = blockIdx.x, r = blockIdx.y;
    const uint32_t base = c * SP_CH;
    if (base >= a.V) return;
    const zs_spec_row s = a.rs[r];
    if (s.mode != 1 || !s.residual) return;
    __shared__ unsigned long long lo[SP_NT / 64], hi[SP_NT / 64];
    const float cT = sp_c(a.temperature[r]);
    const sp_chunk_w cw = sp_chunk_scales(a, r, s, c, cT, s.pos);
    float xt[SP_EPT], xd[SP_EPT];
    sp_load(sp_row(a, r, s.pos), base, a.V, xt);
    sp_load(sp_row(a, r, a.k + 1 + s.pos), base, a.V, xd);
    u128 acc = 0;
#pragma unroll
    for (int e = 0; e < SP_EPT; e++)
        acc += spd_weight2(s, cw, cT, xt[e], xd[e]);
    for (int d = 32; d > 0; d >>= 1) acc += shfl_xor_u128(acc, d);
    if (zs_lane() == 0) { lo[zs_wid()] = (unsigned long long)acc; hi[zs_wid()] = (unsigned long long)(acc >> 64); }
    __syncthreads();
    if (threadIdx.x == 0) {
        u128 t = 0;
        for (int i = 0; i < SP_NT / 64; i++) t += ((u128)hi[i] << 64) | lo[i];
        zs_spec_chunk& o = a.cst[((size_t)r * a.npos_max + 0) * a.nch + c];
        o.rlo = (unsigned long long)t;
        o.rhi = (unsigned long long)(t >> 64);
    }
}

// pass 4: one workgroup per row -- the replacement / bonus draw: the chunk
// holding the target from the chunk sums, then the first id of that chunk whose
// inclusive prefix exceeds the target
__global__ __launch_bounds__(SP_BIG_NT) void zs_k_spec_draw(zs_spec_args a) {
    const uint32_t r = blockIdx.x;
    __shared__ unsigned long long lo[SP_BIG_NT / 64], hi[SP_BIG_NT / 64];
    __shared__ int imin[SP_BIG_NT / 64];
    __shared__ uint32_t csel;
    __shared__ unsigned long long clo, chi, rzero;
    zs_spec_row s = a.rs[r];
    if (s.mode != 1) return;
    const float cT = sp_c(a.temperature[r]);
    const int t = threadIdx.x;
    const uint32_t V = a.V;
    const uint32_t nch = (V + SP_CH - 1) / SP_CH;
    const zs_spec_chunk* c0 = a.cst + ((size_t)r * a.npos_max + 0) * a.nch;                   // residual sums
    const zs_spec_chunk* cp = a.cst + ((size_t)r * a.npos_max + (s.residual ? s.pos : a.k)) * a.nch;  // P sums
    if (t < 64) {
        // residual total; p == q exactly leaves no residual: draw from the target
        u128 rt = 0;
        if (s.residual)
            for (uint32_t c = t; c < nch; c += 64) rt += ((u128)c0[c].rhi << 64) | c0[c].rlo;
        for (int d = 32; d > 0; d >>= 1) rt += shfl_xor_u128(rt, d);
        const bool resid = s.residual && rt != 0;
        const u128 total = resid ? rt : (((u128)s.sum_hi << 64) | s.sum_lo);
        // floor(word * total / 2^32) without overflow: total < 2^108
        const u128 target = (((u128)s.word * (unsigned long long)(total >> 64)) << 32) +
                            (((u128)s.word * (unsigned long long)total) >> 32);
        // chunk prefix over the lanes (nch <= 64 for the vocab limit)
        u128 w = 0;
        if ((uint32_t)t < nch)
            w = resid ? (((u128)c0[t].rhi << 64) | c0[t].rlo)
                      : (u128)((unsigned long long)sp_weight(cp[t].xmax, s.m_t, cT) * cp[t].wsum);
        u128 inc = w;
        for (int d = 1; d < 64; d <<= 1) {
            u128 y = shfl_up_u128(inc, d);
            if (t >= d) inc += y;
        }
        const bool hit = w > 0 && inc > target;
        const unsigned long long bal = __ballot(hit);
        const int first = bal ? __ffsll((long long)bal) - 1 : -1;
        const u128 before = __shfl(first >= 0 ? (unsigned long long)(inc - w) : 0ull, first >= 0 ? first : 0, 64);
        const u128 beforeh = __shfl(first >= 0 ? (unsigned long long)((inc - w) >> 64) : 0ull, first >= 0 ? first : 0, 64);
        if (t == 0) {
            csel = first >= 0 ? (uint32_t)first : 0xffffffffu;
            const u128 rem = target - ((beforeh << 64) | (unsigned long long)before);
            clo = (unsigned long long)rem;
            chi = (unsigned long long)(rem >> 64);
            rzero = resid ? 1ull : 0ull;
        }
    }
    __syncthreads();
    const uint32_t c = csel;
    if (c == 0xffffffffu) {
        if (t == 0) a.next[r] = V - 1;
        return;
    }
    const uint32_t tpos = s.residual ? s.pos : a.k;
    if (!rzero) s.residual = 0;
    const u128 rem = ((u128)chi << 64) | clo;  // target minus the weight of the chunks before
    const uint32_t base = c * SP_CH;
    const sp_chunk_w cw = sp_chunk_scales(a, r, s, c, cT, tpos);
    // 8192 ids, 8 per thread in two float4 of each row
    const float* rt = sp_row(a, r, s.pos);
    const float* rd = s.residual ? sp_row(a, r, a.k + 1 + s.pos) : rt;
    u128 w[8], loc = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint32_t id = base + (h * SP_BIG_NT + t) * 4;
        float4 vt = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY), vd = vt;
        if (id < V) {
            vt = *reinterpret_cast<const float4*>(rt + id);
            vd = *reinterpret_cast<const float4*>(rd + id);
        }
        const float xt[4] = {vt.x, vt.y, vt.z, vt.w}, xd[4] = {vd.x, vd.y, vd.z, vd.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            w[4 * h + q] = id + q < V ? spd_weight2(s, cw, cT, xt[q], xd[q]) : 0;
        }
    }
    // inclusive prefix in id order: ids of thread t are base + 4t..4t+3 (h=0)
    // and base + 4096 + 4t..+3 (h=1); scan the two halves one after the other
    int found = ZS_BIGI;
    u128 carry = 0;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        u128 l = w[4 * h] + w[4 * h + 1] + w[4 * h + 2] + w[4 * h + 3];
        u128 inc = l;
        for (int d = 1; d < 64; d <<= 1) {
            u128 y = shfl_up_u128(inc, d);
            if (zs_lane() >= d) inc += y;
        }
        if (zs_lane() == 63) { lo[zs_wid()] = (unsigned long long)inc; hi[zs_wid()] = (unsigned long long)(inc >> 64); }
        __syncthreads();
        u128 pre = 0, tot = 0;
        for (int i = 0; i < SP_BIG_NT / 64; i++) {
            u128 wv = ((u128)hi[i] << 64) | lo[i];
            if (i < zs_wid()) pre += wv;
            tot += wv;
        }
        __syncthreads();
        u128 run = carry + pre + inc - l;
        int my = ZS_BIGI;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            run += w[4 * h + q];
            if (my == ZS_BIGI && w[4 * h + q] > 0 && run > rem) my = h * 4 * SP_BIG_NT + 4 * t + q;
        }
        const int f = block_min_i<SP_BIG_NT>(my, imin);
        if (found == ZS_BIGI) found = f;
        carry += tot;
    }
    if (t == 0) a.next[r] = found == ZS_BIGI ? V - 1 : base + (uint32_t)found;
}

extern "C" int zs_spec_launch(const zs_spec_args& a, const zs_prof& prof, hipStream_t stream) {
    const uint32_t npos = a.draft ? 2 * a.k + 1 : a.k + 1;
    const uint32_t nch = (a.V + SP_CH - 1) / SP_CH;
    int ev = 0;
    auto mark = [&](const char* name) {
        if (!prof.on) return;
        prof.names[ev] = name;
        (void)hipEventRecord((hipEvent_t)prof.events[ev], stream);
        ev++;
    };
    dim3 grid(nch, npos, a.B);
    mark(nullptr);
    if (a.background) {
        hipLaunchKernelGGL(zs_k_spec_row, dim3(npos, a.B), dim3(SR_NT), SR_LDS_HOLD, stream, a);
        mark("zs_k_spec_row");
    } else {
    hipLaunchKernelGGL(zs_k_spec_chunk, grid, dim3(SP_NT), 0, stream, a);
    mark("zs_k_spec_chunk");
    }
    hipLaunchKernelGGL(zs_k_spec_decide, dim3(a.B), dim3(64), 0, stream, a);
    hipLaunchKernelGGL(zs_k_spec_rsum, dim3(nch, a.B), dim3(SP_NT), 0, stream, a);
    hipLaunchKernelGGL(zs_k_spec_draw, dim3(a.B), dim3(SP_BIG_NT), 0, stream, a);
    mark("zs_k_spec_draw");
    if (prof.on) *prof.n = ev - 1;
    return hipGetLastError() == hipSuccess ? 0 : -1;
}

// ---------------------------------------------------------------------------
// zs_spec_verify_static: the same verification without a context, for callers
// that cannot allocate (HIP graph capture, serving loops that forbid
// hipMalloc). The chunk records and per-row state live in `scratch`, one copy
// per GPU for the life of the process. The host never passes the array's own
// name to a kernel (in host code it is only a stand-in for the symbol): the
// device address of each GPU's copy is looked up once with
// hipGetSymbolAddress, with that GPU current, and kept per device.
// Every kernel writes the records it later reads, so nothing needs clearing.
// Calls that overlap on one GPU share the array and race.
// ---------------------------------------------------------------------------
struct zs_spec_static_area {
    zs_spec_chunk cst[ZS_SPEC_STATIC_MAX_RECORDS];
    zs_spec_row rs[ZS_SPEC_STATIC_MAX_ROWS];
};
static __device__ __align__(256) zs_spec_static_area scratch;

#define ZS_STATIC_MAX_DEVICES 64
static zs_spec_static_area* g_static_area[ZS_STATIC_MAX_DEVICES];
static std::mutex g_static_mu;

// Device address of the current GPU's copy of `scratch` (looked up once per
// device), or null when the lookup fails.
static zs_spec_static_area* zs_spec_static_area_of(int dev) {
    if (dev < 0 || dev >= ZS_STATIC_MAX_DEVICES) return nullptr;
    std::lock_guard<std::mutex> lk(g_static_mu);
    if (!g_static_area[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return nullptr;
        g_static_area[dev] = static_cast<zs_spec_static_area*>(p);
    }
    return g_static_area[dev];
}

extern "C" int zs_spec_verify_static(const zs_spec_batch* b, void* stream) {
    if (!b) return ZS_EINVAL;
    if (b->B == 0) return ZS_OK;
    if (b->V == 0 || b->k > ZS_SPEC_KMAX || b->B > ZS_SPEC_STATIC_MAX_ROWS) return ZS_ELIMIT;
    if (!b->d_target || (b->k && !b->d_draft_ids) || !b->d_temperature || !b->d_seed || !b->d_counter ||
        !b->d_accepted || !b->d_next)
        return ZS_EINVAL;
    if (b->ld < b->V || (b->ld & 3u) || ((uintptr_t)b->d_target & 15u) || ((uintptr_t)b->d_draft & 15u))
        return ZS_EINVAL;
    if (b->flags & ~(uint32_t)ZS_SPEC_BACKGROUND) return ZS_EINVAL;
    const uint32_t k = b->k;
    const bool draft = k && b->d_draft;
    const uint64_t npos = draft ? 2ull * k + 1 : (uint64_t)k + 1;
    const uint64_t nch = (b->V + SP_CH - 1) / SP_CH;
    if ((uint64_t)b->B * npos * nch > ZS_SPEC_STATIC_MAX_RECORDS) return ZS_ELIMIT;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return ZS_EHIP;
    zs_spec_static_area* area = zs_spec_static_area_of(dev);
    if (!area) return ZS_EHIP;
    zs_spec_args a{};
    a.B = b->B; a.V = b->V; a.k = k; a.ld = b->ld;
    a.target = b->d_target; a.draft = k ? b->d_draft : nullptr; a.draft_ids = b->d_draft_ids;
    a.temperature = b->d_temperature; a.seed = b->d_seed; a.counter = b->d_counter;
    a.accepted = b->d_accepted; a.next = b->d_next;
    a.cst = area->cst;        // device address of this GPU's copy
    a.rs = area->rs;
    a.nch = (uint32_t)nch;
    a.npos_max = (uint32_t)npos;
    a.background = (b->flags & ZS_SPEC_BACKGROUND) ? 1u : 0u;
    zs_prof prof{0, nullptr, nullptr, nullptr};
    return zs_spec_launch(a, prof, (hipStream_t)stream) ? ZS_EHIP : ZS_OK;
}
