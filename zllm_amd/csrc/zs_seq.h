// zs_seq.h -- workgroup-parallel exact reproduction of a sequential f32 sum of
// non-negative terms (the `sum()` / `cumsum +=` loops of sampler.rs:68, 80,
// 103, 107, 121).
//
// A group is NT*EPT terms held EPT per thread; element e = EPT*tid + j is the
// e-th term in summation order. Inside one binade of the running sum every term
// adds an integer number of grid units (zs_seq_inc), so a saturating prefix
// scan gives the exact running sum up to the first "event" (a term whose
// rounding is a tie, or that carries the sum out of its binade). Events are
// applied with a real f32 add and the scan restarts after them.
#pragma once
#include "zs_dev.h"

template <int NT>
struct seq_sh {
    uint32_t scan[NT / 64];
    int imin[NT / 64];
    float s;
    int stop;
};

struct seq_find_res {
    int ev, st;    // first event / first element reaching thresh (ZS_BIGI if none)
    int eg;        // grid exponent of the running sum at group start
    uint32_t k0;   // running sum / grid at group start
    uint32_t total;
};

// excl[j] receives the exact running sum (in grid units, minus k0) before
// element EPT*tid + j; it is exact for every element up to the first event.
template <int NT, int EPT>
__device__ __forceinline__ seq_find_res seq_find(const float (&tv)[EPT], int start, float s, float thresh,
                                                 uint32_t (&excl)[EPT], seq_sh<NT>& sh) {
    const int t = threadIdx.x;
    seq_find_res R;
    R.eg = zs_grid_exp(s);
    R.k0 = zs_grid_k(s);
    const uint32_t kthr = zs_grid_thresh(thresh, R.eg);
    uint32_t inc[EPT], tie[EPT], loc = 0;
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        int e = EPT * t + j;
        if (e >= start) inc[j] = zs_seq_inc(tv[j], R.eg, &tie[j]);
        else { inc[j] = 0; tie[j] = 0; }
        loc = zs_sat_add(loc, inc[j]);
    }
    uint32_t tot;
    uint32_t run = block_excl_scan_sat<NT>(loc, sh.scan, &tot);
    int my_ev = ZS_BIGI, my_st = ZS_BIGI;
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        int e = EPT * t + j;
        excl[j] = run;
        if (e < start) continue;
        run = zs_sat_add(run, inc[j]);
        if (my_ev == ZS_BIGI && (tie[j] || R.k0 + run >= ZS_BINADE)) my_ev = e;
        if (my_st == ZS_BIGI && kthr != 0xffffffffu && R.k0 + run >= kthr) my_st = e;
    }
    R.ev = block_min_i<NT>(my_ev, sh.imin);
    R.st = block_min_i<NT>(my_st, sh.imin);
    R.total = tot;
    return R;
}

// Value of the running sum just before group element `pos` (pos < first event),
// broadcast to the workgroup.
template <int NT, int EPT>
__device__ __forceinline__ float seq_value_at(const seq_find_res& R, const uint32_t (&excl)[EPT], int pos,
                                              seq_sh<NT>& sh) {
    if (threadIdx.x == pos / EPT) {
        uint32_t ex = excl[0];
#pragma unroll
        for (int j = 0; j < EPT; j++) if (j == pos % EPT) ex = excl[j];
        sh.s = zs_grid_value(R.k0 + ex, R.eg);
    }
    __syncthreads();
    float v = sh.s;
    __syncthreads();
    return v;
}

// Advance the exact running sum s over the group's elements >= start.
// Returns the first element after which the sum is >= thresh (s is then
// undefined), or -1 with s = the sum after the whole group.
template <int NT, int EPT>
__device__ int seq_group(const float (&tv)[EPT], int start, float& s, float thresh, seq_sh<NT>& sh) {
    const int t = threadIdx.x;
    while (start < NT * EPT) {
        uint32_t excl[EPT];
        seq_find_res R = seq_find<NT, EPT>(tv, start, s, thresh, excl, sh);
        if (R.st < R.ev) return R.st;
        if (R.ev == ZS_BIGI) {
            s = zs_grid_value(R.k0 + R.total, R.eg);
            return -1;
        }
        if (t == R.ev / EPT) {
            const int jj = R.ev % EPT;
            uint32_t ex = excl[0];
            float term = tv[0];
#pragma unroll
            for (int j = 0; j < EPT; j++) if (j == jj) { ex = excl[j]; term = tv[j]; }
            float sb = zs_grid_value(R.k0 + ex, R.eg);
            float ns = sb + term;
            sh.s = ns;
            sh.stop = (ns >= thresh) ? 1 : 0;
        }
        __syncthreads();
        s = sh.s;
        int stop = sh.stop;
        __syncthreads();
        if (stop) return R.ev;
        start = R.ev + 1;
    }
    return -1;
}
