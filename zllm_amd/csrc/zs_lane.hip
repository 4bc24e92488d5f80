// zs_lane.hip -- the batched GPU lane of the reference (continuous batching,
// gpu/batch.rs:176-192): batched argmax, Gumbel-max temperature sampling,
// top-K extraction and the top-K nucleus draw, with the reference semantics of
// shaders.rs:758-937 and gpu/sampling.rs:9-56, on-device (no readback).
//
// The WGSL kernels reduce with a 256-thread workgroup: thread t scans ids
// t, t+256, ... keeping the first strict maximum, then a stride-128..1 tree
// keeps the lower slot unless the upper one is strictly greater. The winner
// among equal maxima is therefore the slot with the smallest bit-reversed
// 8-bit slot number, then the smallest id within that slot; candidates must be
// strictly greater than the initial -1e30 (NaN never wins). These kernels
// reduce a composite key that encodes exactly that order, which lets any
// workgroup shape reproduce the WGSL result.
#include <hip/hip_runtime.h>
#include "zs_internal.h"
#include "zs_dev.h"

#define LN_NT 1024

__device__ __forceinline__ uint32_t zs_bitrev8(uint32_t x) { return __brev(x) >> 24; }

// composite for the WGSL argmax order: larger value, then preferred slot, then lower id
__device__ __forceinline__ unsigned long long wg_key(float v, uint32_t idx) {
    if (!(v > -1e30f)) return 0ull;  // not a candidate (also NaN)
    float vv = (v == 0.0f) ? 0.0f : v;
    uint32_t slot = idx & 255u, hi = idx >> 8;
    return ((unsigned long long)zs_total_key(vv) << 32) | ((unsigned long long)(255u - zs_bitrev8(slot)) << 24) |
           (unsigned long long)(0xffffffu - (hi & 0xffffffu));
}
__device__ __forceinline__ uint32_t wg_key_idx(unsigned long long k) {
    uint32_t slot = zs_bitrev8(255u - (uint32_t)((k >> 24) & 255u));
    uint32_t hi = 0xffffffu - (uint32_t)(k & 0xffffffu);
    return (hi << 8) | slot;
}

__device__ __forceinline__ unsigned long long block_max_u64(unsigned long long v, unsigned long long* sh) {
    for (int d = 32; d > 0; d >>= 1) {
        unsigned long long o = __shfl_xor(v, d, 64);
        v = o > v ? o : v;
    }
    if (zs_lane() == 0) sh[zs_wid()] = v;
    __syncthreads();
    unsigned long long r = 0;
    for (int i = 0; i < LN_NT / 64; i++) r = sh[i] > r ? sh[i] : r;
    __syncthreads();
    return r;
}

// shaders.rs:805-815
__device__ __forceinline__ uint32_t zs_hash_u32(uint32_t x) {
    uint32_t h = x;
    h ^= h >> 16; h *= 0x7feb352du;
    h ^= h >> 15; h *= 0x846ca68bu;
    h ^= h >> 16;
    return h;
}
// rand01 from the id's half of the hash, hi = zs_hash_u32(i)
__device__ __forceinline__ float zs_rand01_h(uint32_t s, uint32_t hi) {
    uint32_t r = zs_hash_u32(s ^ hi);
    return ((float)(r >> 8) + 0.5f) / 16777216.0f;
}
__device__ __forceinline__ float zs_rand01(uint32_t s, uint32_t i) { return zs_rand01_h(s, zs_hash_u32(i)); }

// ih[i] = zs_hash_u32(i): the id half of every row's uniforms, computed once
// per context (BSAMPLE reads it instead of hashing each id again)
__global__ void zs_k_lane_hash_fill(uint32_t* ih, uint32_t n) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) ih[i] = zs_hash_u32(i);
}
extern "C" int zs_lane_hash_fill(uint32_t* ih, uint32_t n, hipStream_t stream) {
    hipLaunchKernelGGL(zs_k_lane_hash_fill, dim3((n + 255) / 256), dim3(256), 0, stream, ih, n);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
// WGSL `log` has no precision contract; this build fixes it as the f32
// rounding of the double log. Fast path: ln x in double from the atanh series
// of m in [sqrt(1/2), sqrt(2)) (x = m 2^e), relative error below 2^-44.7
// over every positive normal float up to 18 (the arguments here: u in (0, 1)
// and -ln u <= 17.33); its f32 rounding is certain unless the value lies
// within 2^-40 (relative) of a midpoint between floats (about 2e-5 of the
// inputs), where the double log is evaluated as the reference does; so are
// arguments outside that range.
__device__ __forceinline__ double zs_log_series(float x) {
    const uint32_t ix = __float_as_uint(x);
    int e = (int)(ix >> 23) - 127;
    float m = __uint_as_float((ix & 0x7fffffu) | 0x3f800000u);
    if (m > 1.41421356f) { m *= 0.5f; e += 1; }
    const double md = (double)m, num = md - 1.0, den = md + 1.0;
    double r = __builtin_amdgcn_rcp(den);
    r = fma(fma(-den, r, 1.0), r, r);
    r = fma(fma(-den, r, 1.0), r, r);
    const double f = num * r, f2 = f * f;
    double p = 1.0 / 15;
    p = fma(p, f2, 1.0 / 13);
    p = fma(p, f2, 1.0 / 11);
    p = fma(p, f2, 1.0 / 9);
    p = fma(p, f2, 1.0 / 7);
    p = fma(p, f2, 1.0 / 5);
    p = fma(p, f2, 1.0 / 3);
    p = fma(p, f2, 1.0);
    return fma((double)e, 0.6931471805599453, 2.0 * f * p);
}
__device__ __forceinline__ float zs_log_cr(float x) {
    // zeros (u = 1 gives -ln u = -0, whose log is -inf), infinities, NaN and
    // subnormals take the double log
    if (!(x >= 0x1p-126f && x <= 18.0f)) return (float)log((double)x);   // rare
    const double a = zs_log_series(x);
    const float r = (float)a;
    const double rd = (double)r, err = fabs(a) * 0x1p-40;
    const double up = (double)__uint_as_float(__float_as_uint(r) + (r >= 0.0f ? 1u : 0xffffffffu));
    const double dn = (double)__uint_as_float(__float_as_uint(r) + (r >= 0.0f ? 0xffffffffu : 1u));
    if (fabs(a - 0.5 * (rd + up)) <= err || fabs(a - 0.5 * (rd + dn)) <= err) return (float)log((double)x);  // rare
    return r;
}

// Gumbel term -ln(-ln u) with v_log_f32: within ZS_GUMBEL_EPS of the exact
// term for every u the hash can give (2^24 values, checked by
// tests/c/calib_gumbel.hip: the largest difference is 2^-19).
#define ZS_GUMBEL_EPS 0x1p-16f
__device__ __forceinline__ float zs_gumbel_fast(float u) {
    const float w = -(__builtin_amdgcn_logf(u) * 0.693147180559945309f);
    return -(__builtin_amdgcn_logf(w) * 0.693147180559945309f);
}
// Largest distance between an approximate Gumbel value a = RN(x/T) + g~ and
// its exact b (both rounded sums): the term's error plus an ulp each way.
__device__ __forceinline__ float zs_gumbel_band(float a) { return ZS_GUMBEL_EPS + fabsf(a) * 0x1p-22f; }
__device__ __forceinline__ float zs_gumbel_exact(float x, float inv_t, uint32_t sd, uint32_t i) {
    const float u = zs_rand01(sd, i);
    const float g = -zs_log_cr(-zs_log_cr(u));
    float v = x * inv_t;
    return v + g;
}

// BARGMAX (shaders.rs:761-789): one workgroup per row.
__global__ __launch_bounds__(LN_NT) void zs_k_bargmax(const float* logits, uint32_t V, uint64_t ld, uint32_t* out) {
    __shared__ unsigned long long sh[LN_NT / 64];
    const uint32_t r = blockIdx.x;
    const float* row = logits + (size_t)r * ld;
    unsigned long long best = 0;
    for (uint32_t i0 = threadIdx.x * 4; i0 < V; i0 += LN_NT * 4) {
        float4 v4 = *reinterpret_cast<const float4*>(row + i0);
        float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t i = i0 + q;
            if (i >= V) continue;
            const unsigned long long k = wg_key(vv[q], i);
            best = k > best ? k : best;
        }
    }
    best = block_max_u64(best, sh);
    if (threadIdx.x == 0) out[r] = best ? wg_key_idx(best) : 0u;
}

// BSAMPLE (shaders.rs:796-850; rows with temperature <= 0 take the argmax)
// over segments of BS_SEG ids, one workgroup each (rows x segments fill the
// GPU). Two steps: every id's value with the fast Gumbel term, then the exact
// values (correctly rounded logs) only for the ids whose fast value lies
// within two bands of the segment's fast maximum -- the row's exact winner is
// among them, any other id being strictly below it. The segment's best exact
// key is merged into keys[row] with a 64-bit atomic max; zs_k_bsample_fin
// turns the keys into ids and clears them for the next call.
#define BS_NT 256
#define BS_SEG (BS_NT * 32)
__global__ __launch_bounds__(BS_NT) void zs_k_bsample(const float* logits, uint32_t V, uint64_t ld, const float* temp,
                                                      const uint32_t* seed, const uint32_t* ih,
                                                      unsigned long long* keys) {
    __shared__ unsigned long long shk[BS_NT / 64];
    __shared__ float shf[BS_NT / 64];
    const uint32_t r = blockIdx.y;
    const uint32_t s0 = blockIdx.x * BS_SEG, s1 = min(s0 + BS_SEG, V);
    const float* row = logits + (size_t)r * ld;
    const float ts = temp[r];
    const bool greedy = ts <= 0.0f;
    const float inv_t = greedy ? 1.0f : 1.0f / ts;
    const uint32_t sd = seed[r];
    const uint32_t last4 = (V - 1) & ~3u;
    unsigned long long best = 0;
    // exact keys of the thread's ids of the segment (greedy rows; threads
    // whose fast values cannot decide)
    auto exact_all = [&]() {
        for (uint32_t i0 = s0 + threadIdx.x * 4; i0 < s1; i0 += BS_NT * 4) {
            const float4 v4 = *reinterpret_cast<const float4*>(row + min(i0, last4));
            const float vv[4] = {v4.x, v4.y, v4.z, v4.w};
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const uint32_t i = i0 + q;
                if (i >= s1) continue;
                const float v = greedy ? vv[q] : zs_gumbel_exact(vv[q], inv_t, sd, i);
                const unsigned long long k = wg_key(v, i);
                best = k > best ? k : best;
            }
        }
    };
    if (greedy) {
        exact_all();
    } else {
        float ba = -INFINITY, bb = -INFINITY, bx = 0.0f;
        uint32_t bi = 0;
        bool exact = false;
        for (uint32_t i0 = s0 + threadIdx.x * 4; i0 < s1; i0 += BS_NT * 16) {
            float4 v4[4];
            uint4 h4[4];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const uint32_t j = min(i0 + (uint32_t)u * BS_NT * 4, last4);
                v4[u] = *reinterpret_cast<const float4*>(row + j);
                h4[u] = *reinterpret_cast<const uint4*>(ih + j);
            }
            float va[16], xs[16];
#pragma unroll
            for (int u = 0; u < 4; u++) {
                const float vv[4] = {v4[u].x, v4[u].y, v4[u].z, v4[u].w};
                const uint32_t hh[4] = {h4[u].x, h4[u].y, h4[u].z, h4[u].w};
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t i = i0 + (uint32_t)u * BS_NT * 4 + q;
                    xs[4 * u + q] = i < s1 ? vv[q] : -INFINITY;
                    const float v = xs[4 * u + q] * inv_t;
                    va[4 * u + q] = v + zs_gumbel_fast(zs_rand01_h(sd, hh[q]));
                }
            }
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const float a = va[e];
                const bool fin = fabsf(a) < 1e29f;
                exact = exact | ((!fin) & (a == a) & (a != -INFINITY));   // -inf and NaN never win
                const float vf = fin ? a : -INFINITY;
                const bool gt = vf > ba;
                bb = fmaxf(bb, fminf(vf, ba));
                bx = gt ? xs[e] : bx;
                bi = gt ? i0 + (uint32_t)(e >> 2) * BS_NT * 4 + (uint32_t)(e & 3) : bi;
                ba = fmaxf(ba, vf);
            }
        }
        const bool near = bb > -INFINITY && ba - bb <= 2.0f * zs_gumbel_band(fmaxf(fabsf(ba), fabsf(bb)));
        float m = ba;
        for (int d = 32; d > 0; d >>= 1) m = fmaxf(m, __shfl_xor(m, d, 64));
        if (zs_lane() == 0) shf[zs_wid()] = m;
        __syncthreads();
        m = -INFINITY;
#pragma unroll
        for (int w = 0; w < BS_NT / 64; w++) m = fmaxf(m, shf[w]);
        const bool cand = exact || (ba > -INFINITY && ba >= m - 2.0f * zs_gumbel_band(fmaxf(fabsf(m), fabsf(ba))));
        if (cand) {
            if (exact || near) exact_all();   // rare
            else best = wg_key(zs_gumbel_exact(bx, inv_t, sd, bi), bi);
        }
    }
    for (int d = 32; d > 0; d >>= 1) {
        const unsigned long long o = __shfl_xor(best, d, 64);
        best = o > best ? o : best;
    }
    if (zs_lane() == 0) shk[zs_wid()] = best;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long b = 0;
#pragma unroll
        for (int w = 0; w < BS_NT / 64; w++) b = shk[w] > b ? shk[w] : b;
        if (b) atomicMax(&keys[r], b);
    }
}
__global__ void zs_k_bsample_fin(unsigned long long* keys, uint32_t B, uint32_t* out) {
    const uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= B) return;
    const unsigned long long k = keys[r];
    out[r] = k ? wg_key_idx(k) : 0u;
    keys[r] = 0ull;
}

// BTOPK (shaders.rs:859-905): the K largest (value desc, id asc) among values in
// [-3e38, 3e38) (NaN and values outside never qualify: they are never "below"
// the previous winner or "better" than the -3e38 seed); sentinel (-3e38,
// 0xffffffff) pads rows with fewer candidates. Keys merge -0.0 and +0.0 (they
// compare equal in WGSL); the output keeps each element's own value.
#define TK_MAX 1024
__device__ __forceinline__ bool tk_cand(float v) { return v >= -3.0e38f && v < 3.0e38f; }
__device__ __forceinline__ uint32_t tk_key(float v) { return zs_total_key(v == 0.0f ? 0.0f : v); }

__global__ __launch_bounds__(LN_NT) void zs_k_btopk(const float* logits, uint32_t V, uint64_t ld, uint32_t K,
                                                     float* vals, uint32_t* idxs) {
    __shared__ uint32_t hist[256];
    __shared__ uint32_t u[4];
    __shared__ unsigned long long buf[TK_MAX];
    __shared__ uint32_t scan_sh[LN_NT / 64];
    const uint32_t r = blockIdx.x;
    const int t = threadIdx.x;
    const float* row = logits + (size_t)r * ld;
    // radix select of the K-th largest candidate key
    uint32_t ncand = 0;
    for (uint32_t i = t; i < V; i += LN_NT) ncand += tk_cand(row[i]) ? 1u : 0u;
    ncand = block_sum_u<LN_NT>(ncand, scan_sh);
    const uint32_t KK = ncand < K ? ncand : K;
    uint32_t prefix = 0, mask = 0, need = KK;
    if (KK > 0) {
        for (int shift = 24; shift >= 0; shift -= 8) {
            if (t < 256) hist[t] = 0;
            __syncthreads();
            for (uint32_t i = t; i < V; i += LN_NT) {
                float v = row[i];
                if (!tk_cand(v)) continue;
                uint32_t k = tk_key(v);
                if ((k & mask) == prefix) atomicAdd(&hist[(k >> shift) & 255u], 1u);
            }
            __syncthreads();
            if (t < 64) {
                uint32_t c[4], loc = 0;
                for (int q = 0; q < 4; q++) { c[q] = hist[255 - 4 * t - q]; loc += c[q]; }
                uint32_t inc = wave_incl_scan_u(loc);
                uint32_t before = inc - loc;
                for (int q = 0; q < 4; q++) {
                    if (before < need && need <= before + c[q]) { u[0] = 255 - 4 * t - q; u[1] = need - before; }
                    before += c[q];
                }
            }
            __syncthreads();
            prefix |= u[0] << shift;
            mask |= 0xffu << shift;
            need = u[1];
            __syncthreads();
        }
    }
    // gather: keys above the K-th, then the lowest-id `need` equal ones (ids in order)
    if (t == 0) u[2] = 0;
    __syncthreads();
    uint32_t carry = 0;
    for (uint32_t base = 0; base < V && KK > 0; base += LN_NT) {
        uint32_t i = base + t;
        float v = i < V ? row[i] : NAN;
        bool c = i < V && tk_cand(v);
        uint32_t k = c ? tk_key(v) : 0;
        bool gt = c && k > prefix, eq = c && k == prefix;
        uint32_t tot;
        uint32_t ex = block_excl_scan_u<LN_NT>(eq ? 1u : 0u, scan_sh, &tot);
        if (gt || (eq && carry + ex < need)) {
            uint32_t pos = atomicAdd(&u[2], 1u);
            if (pos < TK_MAX) buf[pos] = ((unsigned long long)(~k) << 32) | i;
        }
        carry += tot;
    }
    __syncthreads();
    uint32_t n = KK;
    uint32_t np2 = 1;
    while (np2 < n) np2 <<= 1;
    for (uint32_t i = n + t; i < np2; i += LN_NT) buf[i] = ~0ull;
    __syncthreads();
    if (np2 > 1) block_sort_u64<LN_NT>(buf, np2);
    for (uint32_t j = t; j < K; j += LN_NT) {
        if (j < n) {
            uint32_t id = (uint32_t)(buf[j] & 0xffffffffull);
            vals[(size_t)r * K + j] = row[id];
            idxs[(size_t)r * K + j] = id;
        } else {
            vals[(size_t)r * K + j] = -3.0e38f;
            idxs[(size_t)r * K + j] = 0xffffffffu;
        }
    }
}

// Two-phase BTOPK for K <= 64: every 16384-id chunk keeps its own top-K by
// (key desc, id asc) -- a superset of the row's top-K restricted to the chunk
// -- and one workgroup per row sorts the chunk lists. Same result as
// zs_k_btopk; one read of the row over the whole chip instead of six passes
// by one workgroup.
#define TC_NT 256
#define TC_CH 16384
#define TC_EPT (TC_CH / TC_NT)
#define TC_SORT 256
#define TC_K 64
#define TC_MAXCH 32
__global__ __launch_bounds__(TC_NT) void zs_k_btopk_chunks(const float* logits, uint32_t V, uint64_t ld, uint32_t K,
                                                            unsigned long long* ck, uint32_t* cn, uint32_t nch) {
    __shared__ uint32_t tmax[TC_NT];
    __shared__ unsigned long long s64[TC_SORT];
    __shared__ uint32_t hist[256];
    __shared__ uint32_t u[4];
    __shared__ uint32_t scan_sh[TC_NT / 64];
    const uint32_t c = blockIdx.x, r = blockIdx.y;
    const int t = threadIdx.x, lane = zs_lane(), wid = zs_wid();
    const uint32_t base = c * TC_CH;
    const float* row = logits + (size_t)r * ld;
    unsigned long long* out = ck + ((size_t)r * nch + c) * TC_K;
    // keys of the thread's elements: float4 j covers ids base + (j*NT + t)*4 .. +3;
    // 0 for ids past V and for non-candidates (below every candidate key)
    uint32_t key[TC_EPT];
#pragma unroll
    for (int j = 0; j < TC_EPT / 4; j++) {
        const uint32_t id = base + (j * TC_NT + t) * 4;
        float4 v = make_float4(NAN, NAN, NAN, NAN);
        if (id + 3 < V) v = *reinterpret_cast<const float4*>(row + id);
        else {
            if (id < V) v.x = row[id];
            if (id + 1 < V) v.y = row[id + 1];
            if (id + 2 < V) v.z = row[id + 2];
        }
        const float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; q++) key[4 * j + q] = tk_cand(vv[q]) ? tk_key(vv[q]) : 0u;
    }
    auto idx_of = [&](int e) { return base + ((e >> 2) * TC_NT + t) * 4 + (e & 3); };
    uint32_t tm = 0;
#pragma unroll
    for (int e = 0; e < TC_EPT; e++) tm = max(tm, key[e]);
    // theta: the K-th largest of the 256 thread maxima (maxima of distinct
    // elements, so at least K keys are >= theta when K threads hold one)
    const uint32_t srt = wave_sort_u32(tm);
    tmax[wid * 64 + lane] = srt;
    __syncthreads();
    if (t < 64) {
        uint32_t m = srt;
#pragma unroll
        for (int w = 1; w < TC_NT / 64; w++) {
            m = max(m, tmax[w * 64 + 63 - lane]);
#pragma unroll
            for (int j = 32; j > 0; j >>= 1) {
                const uint32_t o = __shfl_xor(m, j, 64);
                m = (lane & j) ? max(m, o) : min(m, o);
            }
        }
        if (lane == 64 - (int)K) u[0] = m;
    }
    __syncthreads();
    const uint32_t theta = max(u[0], 1u);
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < TC_EPT; e++) cnt += key[e] >= theta ? 1u : 0u;
    uint32_t nsup;
    uint32_t pos = block_excl_scan_u<TC_NT>(cnt, scan_sh, &nsup);
    if (nsup <= TC_SORT) {
#pragma unroll
        for (int e = 0; e < TC_EPT; e++)
            if (key[e] >= theta) s64[pos++] = ((unsigned long long)(~key[e]) << 32) | idx_of(e);
        __syncthreads();
        const uint32_t n = min(K, nsup);
        if (nsup <= 64) {
            if (t < 64) {
                unsigned long long v = (uint32_t)t < nsup ? s64[t] : ~0ull;
                v = wave_sort_u64(v);
                if ((uint32_t)t < n) out[t] = v;
            }
        } else {
            for (uint32_t i = nsup + t; i < TC_SORT; i += TC_NT) s64[i] = ~0ull;
            __syncthreads();
            block_sort_u64<TC_NT>(s64, TC_SORT);
            if ((uint32_t)t < n) out[t] = s64[t];
        }
        if (t == 0) cn[(size_t)r * nch + c] = n;
        return;
    }
    // many keys tie near theta: exact K-th key by an 8-bit radix select, then
    // the keys above it and the lowest ids among the keys equal to it
    uint32_t ncand = 0;
#pragma unroll
    for (int e = 0; e < TC_EPT; e++) ncand += key[e] ? 1u : 0u;
    ncand = block_sum_u<TC_NT>(ncand, scan_sh);
    const uint32_t KK = min(K, ncand);
    uint32_t prefix = 0, mask = 0, need = KK;
    for (int shift = 24; shift >= 0; shift -= 8) {
        hist[t] = 0;
        __syncthreads();
#pragma unroll
        for (int e = 0; e < TC_EPT; e++)
            if (key[e] && (key[e] & mask) == prefix) atomicAdd(&hist[(key[e] >> shift) & 255u], 1u);
        __syncthreads();
        if (t < 64) {
            uint32_t cc[4], loc = 0;
            for (int q = 0; q < 4; q++) { cc[q] = hist[255 - 4 * t - q]; loc += cc[q]; }
            uint32_t inc = wave_incl_scan_u(loc);
            uint32_t before = inc - loc;
            for (int q = 0; q < 4; q++) {
                if (before < need && need <= before + cc[q]) { u[1] = 255 - 4 * t - q; u[2] = need - before; }
                before += cc[q];
            }
        }
        __syncthreads();
        prefix |= u[1] << shift;
        mask |= 0xffu << shift;
        need = u[2];
        __syncthreads();
    }
    if (t == 0) u[3] = 0;
    __syncthreads();
    uint32_t carry = 0;  // the KK chosen keys are gathered in s64, then sorted
#pragma unroll
    for (int j = 0; j < TC_EPT / 4; j++) {  // ids ascend with j, then t, then q
        uint32_t ce = 0;
#pragma unroll
        for (int q = 0; q < 4; q++) ce += key[4 * j + q] == prefix ? 1u : 0u;
        uint32_t tot;
        uint32_t rank = carry + block_excl_scan_u<TC_NT>(ce, scan_sh, &tot);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const uint32_t k = key[4 * j + q];
            bool take = k && k > prefix;
            if (k && k == prefix) { take = rank < need; rank++; }
            if (take) {
                const uint32_t p = atomicAdd(&u[3], 1u);
                if (p < TC_K) s64[p] = ((unsigned long long)(~k) << 32) | idx_of(4 * j + q);
            }
        }
        carry += tot;
    }
    __syncthreads();
    if (t < 64) {
        unsigned long long v = (uint32_t)t < KK ? s64[t] : ~0ull;
        v = wave_sort_u64(v);
        if ((uint32_t)t < KK) out[t] = v;
    }
    if (t == 0) cn[(size_t)r * nch + c] = KK;
}

// One wave per row: the chunk lists are sorted (best first), so the row's
// best K is a running merge -- the elementwise min of the kept list and the
// reversed next list holds the 64 best of both as a bitonic sequence, which
// six exchange steps sort.
#define TM_ROWS 4
struct tm_draw {   // the nucleus draw after the merge (zs_lane_step's top-K path)
    const float* temp;
    const uint32_t *top_k;
    const float* top_p;
    const uint32_t* seed;
    uint32_t* out;
};
__device__ __forceinline__ uint32_t lane_draw64(float v, uint32_t id, uint32_t K, float T, uint32_t top_k, float tp,
                                                uint32_t seed);
template <bool DRAW>
__global__ __launch_bounds__(64 * TM_ROWS) void zs_k_btopk_merge(const float* logits, uint32_t B, uint64_t ld,
                                                                  uint32_t K, const unsigned long long* ck,
                                                                  const uint32_t* cn, uint32_t nch, float* vals,
                                                                  uint32_t* idxs, tm_draw d) {
    const uint32_t r = blockIdx.x * TM_ROWS + zs_wid();
    if (r >= B) return;
    const int lane = zs_lane();
    unsigned long long cur = ~0ull;
    for (uint32_t c = 0; c < nch; c++) {
        const uint32_t n = cn[(size_t)r * nch + c];
        unsigned long long b = (uint32_t)lane < n ? ck[((size_t)r * nch + c) * TC_K + lane] : ~0ull;
        b = __shfl(b, 63 - lane, 64);
        unsigned long long m = b < cur ? b : cur;
#pragma unroll
        for (int j = 32; j > 0; j >>= 1) {
            const unsigned long long o = __shfl_xor(m, j, 64);
            m = (lane & j) ? (o > m ? o : m) : (o < m ? o : m);
        }
        cur = m;
    }
    float v = -3.0e38f;
    uint32_t id = 0xffffffffu;
    if ((uint32_t)lane < K) {
        if (cur != ~0ull) {
            id = (uint32_t)(cur & 0xffffffffull);
            v = logits[(size_t)r * ld + id];
        }
        vals[(size_t)r * K + lane] = v;
        idxs[(size_t)r * K + lane] = id;
    }
    if (DRAW) {
        // the pool as zs_k_sample_topk64 reads it back
        const uint32_t res = lane_draw64((uint32_t)lane < K ? v : -INFINITY, (uint32_t)lane < K ? id : 0u, K,
                                         d.temp[r], d.top_k[r], d.top_p[r], d.seed[r]);
        if (lane == 0) d.out[r] = res;
    }
}

// gpu/sampling.rs:24-31
__device__ __forceinline__ float zs_rng01(uint32_t seed) {
    uint64_t z = (uint64_t)seed * 0x9E3779B97F4A7C15ull + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return ((float)(z >> 40) + 0.5f) / 16777216.0f;
}

// gpu/sampling.rs:35-56, one thread per row over its descending pool.
__global__ void zs_k_sample_topk(const float* vals, const uint32_t* idxs, uint32_t B, uint32_t K,
                                 const float* temp, const uint32_t* top_k, const float* top_p,
                                 const uint32_t* seed, uint32_t* out) {
    uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= B) return;
    const float* v = vals + (size_t)r * K;
    const uint32_t* id = idxs + (size_t)r * K;
    uint32_t n = 0;
    while (n < K && v[n] > -3.0e37f) n++;
    if (n == 0 || temp[r] <= 0.0f) { out[r] = id[0]; return; }
    const float T = temp[r];
    uint32_t kk = top_k[r] == 0 ? n : (top_k[r] < n ? top_k[r] : n);
    const float maxv = v[0];
    float z = -0.0f;
    for (uint32_t i = 0; i < kk; i++) z = z + zs_expf((v[i] - maxv) / T);
    uint32_t cut = kk;
    const float tp = top_p[r];
    if (tp > 0.0f && tp < 1.0f) {
        float cum = 0.0f;
        for (uint32_t i = 0; i < kk; i++) {
            cum = cum + zs_expf((v[i] - maxv) / T) / z;
            if (cum >= tp) { cut = i + 1; break; }
        }
    }
    float zc = -0.0f;
    for (uint32_t i = 0; i < cut; i++) zc = zc + zs_expf((v[i] - maxv) / T) / z;
    const float target = zs_rng01(seed[r]) * zc;
    float acc = 0.0f;
    uint32_t res = id[cut - 1];
    for (uint32_t i = 0; i < cut; i++) {
        acc = acc + zs_expf((v[i] - maxv) / T) / z;
        if (acc >= target) { res = id[i]; break; }
    }
    out[r] = res;
}

// The same draw by one wave for a pool of at most 64 (lane i holds entry i:
// value v, id; lanes >= K hold -inf): the exponentials in parallel, the
// sequential sums (sampler order, f32) as chains of lane reads (the index is
// uniform: v_readlane, no LDS permute). Returns the id (uniform).
__device__ __forceinline__ uint32_t lane_draw64(float v, uint32_t id, uint32_t K, float T, uint32_t top_k, float tp,
                                                uint32_t seed) {
    const int lane = zs_lane();
    const uint32_t id0 = __shfl(id, 0, 64);
    // n: length of the leading run of values above the sentinel
    const unsigned long long fail = __ballot(!((uint32_t)lane < K && v > -3.0e37f));
    const uint32_t n = fail ? (uint32_t)__ffsll((long long)fail) - 1u : 64u;
    if (n == 0 || T <= 0.0f) return id0;
    const uint32_t kk = top_k == 0 ? n : (top_k < n ? top_k : n);
    const float maxv = __shfl(v, 0, 64);
    const float e = (uint32_t)lane < kk ? zs_expf((v - maxv) / T) : 0.0f;
    float z = -0.0f;
    for (uint32_t i = 0; i < kk; i++) z = z + zs_readlane_f(e, i);
    const float p = e / z;
    uint32_t cut = kk;
    if (tp > 0.0f && tp < 1.0f) {
        float cum = 0.0f;
        for (uint32_t i = 0; i < kk; i++) {
            cum = cum + zs_readlane_f(p, i);
            if (cum >= tp) { cut = i + 1; break; }
        }
    }
    float zc = -0.0f;
    for (uint32_t i = 0; i < cut; i++) zc = zc + zs_readlane_f(p, i);
    const float target = zs_rng01(seed) * zc;
    float acc = 0.0f;
    uint32_t pick = cut - 1;
    for (uint32_t i = 0; i < cut; i++) {
        acc = acc + zs_readlane_f(p, i);
        if (acc >= target) { pick = i; break; }
    }
    return __shfl(id, (int)pick, 64);
}

__global__ __launch_bounds__(64 * TM_ROWS) void zs_k_sample_topk64(const float* vals, const uint32_t* idxs,
                                                                    uint32_t B, uint32_t K, const float* temp,
                                                                    const uint32_t* top_k, const float* top_p,
                                                                    const uint32_t* seed, uint32_t* out) {
    const uint32_t r = blockIdx.x * TM_ROWS + zs_wid();
    if (r >= B) return;
    const int lane = zs_lane();
    const float v = (uint32_t)lane < K ? vals[(size_t)r * K + lane] : -INFINITY;
    const uint32_t id = (uint32_t)lane < K ? idxs[(size_t)r * K + lane] : 0u;
    const uint32_t res = lane_draw64(v, id, K, temp[r], top_k[r], top_p[r], seed[r]);
    if (lane == 0) out[r] = res;
}

// ih: zs_lane_hash_fill of at least round_up(V, 4) ids; keys: B zeroed u64
// (left zeroed) -- both used when temp is set
extern "C" int zs_lane_argmax_launch(const float* logits, uint32_t B, uint32_t V, uint64_t ld, const float* temp,
                                     const uint32_t* seed, const uint32_t* ih, unsigned long long* keys,
                                     uint32_t* out, hipStream_t stream) {
    if (temp) {
        hipLaunchKernelGGL(zs_k_bsample, dim3((V + BS_SEG - 1) / BS_SEG, B), dim3(BS_NT), 0, stream, logits, V, ld,
                           temp, seed, ih, keys);
        hipLaunchKernelGGL(zs_k_bsample_fin, dim3((B + 255) / 256), dim3(256), 0, stream, keys, B, out);
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    hipLaunchKernelGGL(zs_k_bargmax, dim3(B), dim3(LN_NT), 0, stream, logits, V, ld, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
// ck / cn: scratch of at least B * ceil(V / TC_CH) * 64 keys and B * ceil(V / TC_CH)
// counts (two-phase path, K <= 64, V <= 32 * TC_CH); nullptr forces one pass
extern "C" int zs_lane_topk_launch(const float* logits, uint32_t B, uint32_t V, uint64_t ld, uint32_t K,
                                   float* vals, uint32_t* idxs, unsigned long long* ck, uint32_t* cn,
                                   hipStream_t stream) {
    const uint32_t nch = (V + TC_CH - 1) / TC_CH;
    if (ck && cn && K <= TC_K && nch <= TC_MAXCH) {
        hipLaunchKernelGGL(zs_k_btopk_chunks, dim3(nch, B), dim3(TC_NT), 0, stream, logits, V, ld, K, ck, cn, nch);
        hipLaunchKernelGGL(zs_k_btopk_merge<false>, dim3((B + TM_ROWS - 1) / TM_ROWS), dim3(64 * TM_ROWS), 0, stream,
                           logits, B, ld, K, ck, cn, nch, vals, idxs, tm_draw{});
    } else {
        hipLaunchKernelGGL(zs_k_btopk, dim3(B), dim3(LN_NT), 0, stream, logits, V, ld, K, vals, idxs);
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
// The top-K pool and its nucleus draw: on the two-phase path the merge kernel
// draws too (one launch and no read-back of the pool), else the two launches.
extern "C" int zs_lane_sample_topk_launch(const float* vals, const uint32_t* idxs, uint32_t B, uint32_t K,
                                          const float* temp, const uint32_t* top_k, const float* top_p,
                                          const uint32_t* seed, uint32_t* out, hipStream_t stream);
extern "C" int zs_lane_topk_draw_launch(const float* logits, uint32_t B, uint32_t V, uint64_t ld, uint32_t K,
                                        float* vals, uint32_t* idxs, unsigned long long* ck, uint32_t* cn,
                                        const float* temp, const uint32_t* top_k, const float* top_p,
                                        const uint32_t* seed, uint32_t* out, hipStream_t stream) {
    const uint32_t nch = (V + TC_CH - 1) / TC_CH;
    if (ck && cn && K <= TC_K && nch <= TC_MAXCH) {
        hipLaunchKernelGGL(zs_k_btopk_chunks, dim3(nch, B), dim3(TC_NT), 0, stream, logits, V, ld, K, ck, cn, nch);
        hipLaunchKernelGGL(zs_k_btopk_merge<true>, dim3((B + TM_ROWS - 1) / TM_ROWS), dim3(64 * TM_ROWS), 0, stream,
                           logits, B, ld, K, ck, cn, nch, vals, idxs, tm_draw{temp, top_k, top_p, seed, out});
        return hipGetLastError() == hipSuccess ? 0 : -1;
    }
    if (zs_lane_topk_launch(logits, B, V, ld, K, vals, idxs, ck, cn, stream)) return -1;
    return zs_lane_sample_topk_launch(vals, idxs, B, K, temp, top_k, top_p, seed, out, stream);
}
extern "C" int zs_lane_sample_topk_launch(const float* vals, const uint32_t* idxs, uint32_t B, uint32_t K,
                                          const float* temp, const uint32_t* top_k, const float* top_p,
                                          const uint32_t* seed, uint32_t* out, hipStream_t stream) {
    if (K <= 64)
        hipLaunchKernelGGL(zs_k_sample_topk64, dim3((B + TM_ROWS - 1) / TM_ROWS), dim3(64 * TM_ROWS), 0, stream, vals,
                           idxs, B, K, temp, top_k, top_p, seed, out);
    else
        hipLaunchKernelGGL(zs_k_sample_topk, dim3((B + 63) / 64), dim3(64), 0, stream, vals, idxs, B, K, temp, top_k,
                           top_p, seed, out);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
