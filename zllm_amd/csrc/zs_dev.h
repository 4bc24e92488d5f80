// zs_dev.h -- wave64 / workgroup primitives for gfx950 (CDNA4).
#pragma once
#include <hip/hip_runtime.h>
#include "zs_math.h"

#define ZS_WAVE 64
#define ZS_BIGI 0x7fffffff

__device__ __forceinline__ int zs_lane() { return (int)(threadIdx.x & 63); }
__device__ __forceinline__ int zs_wid() { return (int)(threadIdx.x >> 6); }

__device__ __forceinline__ float wave_max_f(float v) {
    for (int d = 32; d > 0; d >>= 1) v = fmaxf(v, __shfl_xor(v, d, 64));
    return v;
}
__device__ __forceinline__ double wave_sum_d(double v) {
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}
__device__ __forceinline__ uint32_t wave_sum_u(uint32_t v) {
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}
__device__ __forceinline__ int wave_min_i(int v) {
    for (int d = 32; d > 0; d >>= 1) v = min(v, __shfl_xor(v, d, 64));
    return v;
}
__device__ __forceinline__ int wave_max_i(int v) {
    for (int d = 32; d > 0; d >>= 1) v = max(v, __shfl_xor(v, d, 64));
    return v;
}
__device__ __forceinline__ uint32_t wave_or_u(uint32_t v) {
    for (int d = 32; d > 0; d >>= 1) v |= __shfl_xor(v, d, 64);
    return v;
}
// Inclusive scan (plain add) over the wave.
__device__ __forceinline__ uint32_t wave_incl_scan_u(uint32_t x) {
    int lane = zs_lane();
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
    }
    return x;
}
// Inclusive scan with saturation at ZS_INC_CAP.
__device__ __forceinline__ uint32_t wave_incl_scan_sat(uint32_t x) {
    int lane = zs_lane();
    for (int d = 1; d < 64; d <<= 1) {
        uint32_t y = __shfl_up(x, d, 64);
        if (lane >= d) x = zs_sat_add(x, y);
    }
    return x;
}

// Workgroup-wide reductions. `sh` needs NT/64 slots of the given type.
template <int NT>
__device__ __forceinline__ float block_max_f(float v, float* sh) {
    v = wave_max_f(v);
    if (zs_lane() == 0) sh[zs_wid()] = v;
    __syncthreads();
    float r = sh[0];
    for (int i = 1; i < NT / 64; i++) r = fmaxf(r, sh[i]);
    __syncthreads();
    return r;
}
template <int NT>
__device__ __forceinline__ double block_sum_d(double v, double* sh) {
    v = wave_sum_d(v);
    if (zs_lane() == 0) sh[zs_wid()] = v;
    __syncthreads();
    double r = 0.0;
    for (int i = 0; i < NT / 64; i++) r += sh[i];
    __syncthreads();
    return r;
}
template <int NT>
__device__ __forceinline__ uint32_t block_sum_u(uint32_t v, uint32_t* sh) {
    v = wave_sum_u(v);
    if (zs_lane() == 0) sh[zs_wid()] = v;
    __syncthreads();
    uint32_t r = 0;
    for (int i = 0; i < NT / 64; i++) r += sh[i];
    __syncthreads();
    return r;
}
template <int NT>
__device__ __forceinline__ int block_min_i(int v, int* sh) {
    v = wave_min_i(v);
    if (zs_lane() == 0) sh[zs_wid()] = v;
    __syncthreads();
    int r = sh[0];
    for (int i = 1; i < NT / 64; i++) r = min(r, sh[i]);
    __syncthreads();
    return r;
}
template <int NT>
__device__ __forceinline__ int block_max_i(int v, int* sh) {
    v = wave_max_i(v);
    if (zs_lane() == 0) sh[zs_wid()] = v;
    __syncthreads();
    int r = sh[0];
    for (int i = 1; i < NT / 64; i++) r = max(r, sh[i]);
    __syncthreads();
    return r;
}
template <int NT>
__device__ __forceinline__ uint32_t block_or_u(uint32_t v, uint32_t* sh) {
    v = wave_or_u(v);
    if (zs_lane() == 0) sh[zs_wid()] = v;
    __syncthreads();
    uint32_t r = 0;
    for (int i = 0; i < NT / 64; i++) r |= sh[i];
    __syncthreads();
    return r;
}
// Exclusive scan in thread order; returns the exclusive prefix, sets *total.
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan_u(uint32_t v, uint32_t* sh, uint32_t* total) {
    uint32_t inc = wave_incl_scan_u(v);
    if (zs_lane() == 63) sh[zs_wid()] = inc;
    __syncthreads();
    uint32_t pre = 0, tot = 0;
    for (int i = 0; i < NT / 64; i++) {
        uint32_t w = sh[i];
        if (i < zs_wid()) pre += w;
        tot += w;
    }
    __syncthreads();
    *total = tot;
    return pre + inc - v;
}
// Exclusive scan of doubles in thread order; sets *total.
template <int NT>
__device__ __forceinline__ double block_excl_scan_d(double v, double* sh, double* total) {
    const int lane = zs_lane();
    double inc = v;
    for (int d = 1; d < 64; d <<= 1) {
        double y = __shfl_up(inc, d, 64);
        if (lane >= d) inc += y;
    }
    if (lane == 63) sh[zs_wid()] = inc;
    __syncthreads();
    double pre = 0.0, tot = 0.0;
    for (int i = 0; i < NT / 64; i++) {
        double w = sh[i];
        if (i < zs_wid()) pre += w;
        tot += w;
    }
    __syncthreads();
    *total = tot;
    return pre + (inc - v);
}
// Same with saturating add (exclusive value computed without subtraction).
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan_sat(uint32_t v, uint32_t* sh, uint32_t* total) {
    uint32_t inc = wave_incl_scan_sat(v);
    uint32_t ex = __shfl_up(inc, 1, 64);
    if (zs_lane() == 0) ex = 0;
    if (zs_lane() == 63) sh[zs_wid()] = inc;
    __syncthreads();
    uint32_t pre = 0, tot = 0;
    for (int i = 0; i < NT / 64; i++) {
        uint32_t w = sh[i];
        if (i < zs_wid()) pre = zs_sat_add(pre, w);
        tot = zs_sat_add(tot, w);
    }
    __syncthreads();
    *total = tot;
    return zs_sat_add(pre, ex);
}

// In-LDS bitonic sort, ascending, of n (power of two) 64-bit keys.
// Ascending bitonic sort across the wave, one value per lane (lane i ends
// with the i-th smallest).
__device__ __forceinline__ uint32_t wave_sort_u32(uint32_t v) {
    const int lane = zs_lane();
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            uint32_t o = __shfl_xor(v, j, 64);
            bool keep_min = ((lane & j) == 0) == ((lane & k) == 0 || k == 64);
            v = keep_min ? min(v, o) : max(v, o);
        }
    }
    return v;
}
__device__ __forceinline__ unsigned long long wave_sort_u64(unsigned long long v) {
    const int lane = zs_lane();
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1) {
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            unsigned long long o = __shfl_xor(v, j, 64);
            bool keep_min = ((lane & j) == 0) == ((lane & k) == 0 || k == 64);
            v = keep_min ? (o < v ? o : v) : (o > v ? o : v);
        }
    }
    return v;
}

// Value of lane l (uniform over the wave) read into a scalar register:
// unlike __shfl with a uniform source (an LDS permute), no LDS round trip.
__device__ __forceinline__ float zs_readlane_f(float v, uint32_t l) {
    return __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), (int)l));
}
__device__ __forceinline__ uint32_t zs_readlane_u(uint32_t v, uint32_t l) {
    return (uint32_t)__builtin_amdgcn_readlane((int)v, (int)l);
}
__device__ __forceinline__ unsigned long long zs_readlane_u64(unsigned long long v, uint32_t l) {
    return ((unsigned long long)zs_readlane_u((uint32_t)(v >> 32), l) << 32) | zs_readlane_u((uint32_t)v, l);
}

// Ascending bitonic sort of n (power of two, n <= NT * E) u64 keys in LDS,
// held in registers while sorted: element i = thread * E + e. Strides below E
// stay inside a thread, strides below 64 * E are lane exchanges, larger ones
// go through `a`. Every thread of the block must call it.
template <int NT, int E>
__device__ void block_sort_reg_u64(unsigned long long* a, uint32_t n) {
    const uint32_t t = threadIdx.x, lane = (uint32_t)zs_lane();
    unsigned long long v[E];
#pragma unroll
    for (int e = 0; e < E; e++) {
        const uint32_t i = t * E + e;
        v[e] = i < n ? a[i] : ~0ull;
    }
    for (uint32_t k = 2; k <= n; k <<= 1) {
        for (uint32_t j = k >> 1; j > 0; j >>= 1) {
            if (j < (uint32_t)E) {
                // compile-time strides keep the register indices static
#pragma unroll
                for (uint32_t jj = E / 2; jj > 0; jj >>= 1) {
                    if (jj != j) continue;
#pragma unroll
                    for (uint32_t e = 0; e < (uint32_t)E; e++) {
                        const uint32_t pe = e ^ jj;
                        if (pe > e) {
                            const bool asc = ((t * E + e) & k) == 0u;
                            const unsigned long long x = v[e], y = v[pe];
                            if ((x > y) == asc) { v[e] = y; v[pe] = x; }
                        }
                    }
                }
            } else {
                unsigned long long o[E];
                if (j < 64u * E) {
#pragma unroll
                    for (int e = 0; e < E; e++) o[e] = __shfl_xor(v[e], (int)(j / E), 64);
                } else {
#pragma unroll
                    for (int e = 0; e < E; e++) if (t * E + e < n) a[t * E + e] = v[e];
                    __syncthreads();
#pragma unroll
                    for (int e = 0; e < E; e++) o[e] = t * E + e < n ? a[(t * E + e) ^ j] : ~0ull;
                    __syncthreads();
                }
#pragma unroll
                for (uint32_t e = 0; e < (uint32_t)E; e++) {
                    const uint32_t i = t * E + e;
                    const bool asc = (i & k) == 0u, lower = (i & j) == 0u;
                    v[e] = (lower == asc) ? (o[e] < v[e] ? o[e] : v[e]) : (o[e] > v[e] ? o[e] : v[e]);
                }
            }
        }
    }
    (void)lane;
#pragma unroll
    for (int e = 0; e < E; e++) if (t * E + e < n) a[t * E + e] = v[e];
    __syncthreads();
}
// block_sort_reg_u64 with E chosen from n (n <= 16 * NT)
template <int NT>
__device__ void block_sort_u64(unsigned long long* a, uint32_t n) {
    if (n <= NT) block_sort_reg_u64<NT, 1>(a, n);
    else if (n <= 2 * NT) block_sort_reg_u64<NT, 2>(a, n);
    else if (n <= 4 * NT) block_sort_reg_u64<NT, 4>(a, n);
    else if (n <= 8 * NT) block_sort_reg_u64<NT, 8>(a, n);
    else block_sort_reg_u64<NT, 16>(a, n);
}

template <int NT>
__device__ void block_bitonic_u64(unsigned long long* a, int n) {
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += NT) {
                int ixj = i ^ j;
                if (ixj > i) {
                    unsigned long long x = a[i], y = a[ixj];
                    bool up = (i & k) == 0;
                    if ((x > y) == up) { a[i] = y; a[ixj] = x; }
                }
            }
            __syncthreads();
        }
    }
}
