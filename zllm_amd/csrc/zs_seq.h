// zs_seq.h -- workgroup-parallel exact reproduction of a sequential f32 sum of
// non-negative terms (the `sum()` / `cumsum +=` loops of sampler.rs:68, 80,
// 103, 107, 121, logprobs.rs:36, hallucination.rs:135, 143).
//
// While the running sum s = k*g stays inside one binade (grid g = ulp(s),
// k < 2^24), adding a term t gives k' = k + round_half_even(k + t/g) - k: an
// integer increment that does not depend on k, except when t/g has fraction
// exactly 1/2, where the result goes to the even neighbour. Each term is
// therefore a map parity(k) -> increment, written as the pair (inc if k even,
// inc if k odd); pairs compose associatively:
//   (A then B)[p] = A[p] + B[(p + A[p]) & 1].
// A workgroup prefix-scans the pairs of a group of NT*EPT terms, takes the path
// of the actual start parity, and finds the first term that carries the sum out
// of its binade (an "event", resolved with a real f32 add) and the first term
// after which the sum reaches a threshold. Element e = EPT*tid + j is the e-th
// term in summation order. Terms are supplied by a functor:
//   f.inc(j, eg, &ie, &io)  increments of the thread's j-th term on grid 2^(eg-150)
//   f.val(j)                the term's exact f32 value (only called at events)
#pragma once
#include "zs_dev.h"

template <int NT>
struct seq_sh {
    uint32_t a[NT / 64], b[NT / 64];     // wave totals, then wave prefixes
    uint32_t te, to;                     // group total (even / odd start)
    int ev, st, tie;                     // first event / stop / tie of the group
    float s;
    int stop;
};

struct seq_pair { uint32_t e, o; };


// Element j of a register array, as a masked OR of the bit patterns: a plain
// compare-and-select chain is recognised by the compiler as a dynamically
// indexed array and moved to scratch memory.
template <int EPT>
__device__ __forceinline__ uint32_t seq_pick_u(const uint32_t (&v)[EPT], int j) {
    uint32_t r = 0u;
#pragma unroll
    for (int q = 0; q < EPT; q++) r |= v[q] & (0u - (uint32_t)(q == j));
    return r;
}

template <int EPT>
__device__ __forceinline__ float seq_pick_f(const float (&v)[EPT], int j) {
    uint32_t r = 0u;
#pragma unroll
    for (int q = 0; q < EPT; q++) r |= __float_as_uint(v[q]) & (0u - (uint32_t)(q == j));
    return __uint_as_float(r);
}

__device__ __forceinline__ seq_pair seq_compose(seq_pair A, seq_pair B) {
    seq_pair C;
    C.e = zs_sat_add(A.e, (A.e & 1u) ? B.o : B.e);
    C.o = zs_sat_add(A.o, (A.o & 1u) ? B.e : B.o);
    return C;
}

// Increment pair of a term whose exact value is t.
__device__ __forceinline__ seq_pair seq_pair_of(float t, int eg) {
    uint32_t tie;
    uint32_t q = zs_seq_inc(t, eg, &tie);
    seq_pair p;
    if (tie) {  // q = floor(t/g): k + q goes up by one when it is odd
        p.e = q + (q & 1u);
        p.o = q + ((q + 1u) & 1u);
    } else {
        p.e = p.o = q;
    }
    return p;
}

// Functor over an array of exact float terms.
template <int EPT>
struct seq_terms {
    const float (&v)[EPT];
    __device__ seq_terms(const float (&x)[EPT]) : v(x) {}
    __device__ __forceinline__ void inc(int j, int eg, uint32_t* ie, uint32_t* io) const {
        seq_pair p = seq_pair_of(seq_pick_f(v, j), eg);
        *ie = p.e;
        *io = p.o;
    }
    __device__ __forceinline__ float val(int j) const {
        return seq_pick_f(v, j);
    }
};

struct seq_find_res {
    int ev, st;    // first event / first element reaching thresh (ZS_BIGI if none)
    int tie;       // first element whose increment depends on the sum's parity
    int eg;        // grid exponent of the running sum at group start
    uint32_t k0;   // running sum / grid at group start
    uint32_t total;  // increments of the whole group (actual path)
};

// excl[j]: running sum (grid units, minus k0) before the thread's j-th element,
// exact up to the first event.
template <int NT, int EPT, class F>
__device__ __forceinline__ seq_find_res seq_find(const F& f, int start, float s, float thresh,
                                                 uint32_t (&excl)[EPT], seq_sh<NT>& sh) {
    const int t = threadIdx.x;
    seq_find_res R;
    R.eg = zs_grid_exp(s);
    R.k0 = zs_grid_k(s);
    const uint32_t kthr = zs_grid_thresh(thresh, R.eg);
    const uint32_t p0 = R.k0 & 1u;
    // even / odd increments kept in separate arrays so that the parity select
    // below stays a register select (a struct member select through a dynamic
    // index would be lowered to scratch memory)
    uint32_t ie[EPT], io[EPT];
    seq_pair loc = {0u, 0u};
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        int e = EPT * t + j;
        uint32_t a0 = 0u, a1 = 0u;
        if (e >= start) f.inc(j, R.eg, &a0, &a1);
        ie[j] = a0;
        io[j] = a1;
        loc = seq_compose(loc, seq_pair{a0, a1});
    }
    // inclusive scan of the thread maps over the wave
    seq_pair inc = loc;
    const int lane = zs_lane();
    for (int d = 1; d < 64; d <<= 1) {
        seq_pair y;
        y.e = __shfl_up(inc.e, d, 64);
        y.o = __shfl_up(inc.o, d, 64);
        seq_pair c = seq_compose(y, inc);
        if (lane >= d) inc = c;
    }
    seq_pair ex;
    ex.e = __shfl_up(inc.e, 1, 64);
    ex.o = __shfl_up(inc.o, 1, 64);
    if (lane == 0) ex.e = ex.o = 0u;
    constexpr int NW = NT / 64;
    if (lane == 63) { sh.a[zs_wid()] = inc.e; sh.b[zs_wid()] = inc.o; }
    __syncthreads();
    // wave 0 scans the wave totals (lane w = wave w) and publishes each wave's
    // exclusive prefix and the group total
    if (zs_wid() == 0) {
        seq_pair w = {0u, 0u};
        if (lane < NW) { w.e = sh.a[lane]; w.o = sh.b[lane]; }
        seq_pair wi = w;
#pragma unroll
        for (int d = 1; d < NW; d <<= 1) {
            seq_pair y;
            y.e = __shfl_up(wi.e, d, 64);
            y.o = __shfl_up(wi.o, d, 64);
            seq_pair c = seq_compose(y, wi);
            if (lane >= d) wi = c;
        }
        seq_pair we;
        we.e = __shfl_up(wi.e, 1, 64);
        we.o = __shfl_up(wi.o, 1, 64);
        if (lane == 0) we.e = we.o = 0u;
        if (lane < NW) { sh.a[lane] = we.e; sh.b[lane] = we.o; }
        if (lane == NW - 1) { sh.te = wi.e; sh.to = wi.o; }
        if (lane == 0) { sh.ev = ZS_BIGI; sh.st = ZS_BIGI; sh.tie = ZS_BIGI; }
    }
    __syncthreads();
    const seq_pair pre = seq_compose(seq_pair{sh.a[zs_wid()], sh.b[zs_wid()]}, ex);
    uint32_t run = p0 ? pre.o : pre.e;
    int my_ev = ZS_BIGI, my_st = ZS_BIGI, my_tie = ZS_BIGI;
#pragma unroll
    for (int j = 0; j < EPT; j++) {
        int e = EPT * t + j;
        excl[j] = run;
        if (e < start) continue;
        if (my_tie == ZS_BIGI && ie[j] != io[j]) my_tie = e;
        uint32_t par = (R.k0 + run) & 1u;
        const uint32_t o = io[j], ev = ie[j];
        run = zs_sat_add(run, par ? o : ev);
        if (my_ev == ZS_BIGI && R.k0 + run >= ZS_BINADE) my_ev = e;
        if (my_st == ZS_BIGI && kthr != 0xffffffffu && R.k0 + run >= kthr) my_st = e;
    }
    R.total = p0 ? sh.to : sh.te;
    // first event / stop / tie over the group
    my_ev = wave_min_i(my_ev);
    my_st = wave_min_i(my_st);
    my_tie = wave_min_i(my_tie);
    if (lane == 0) {
        if (my_ev != ZS_BIGI) atomicMin(&sh.ev, my_ev);
        if (my_st != ZS_BIGI) atomicMin(&sh.st, my_st);
        if (my_tie != ZS_BIGI) atomicMin(&sh.tie, my_tie);
    }
    __syncthreads();
    const int ev = sh.ev, st = sh.st, tie = sh.tie;
    __syncthreads();
    R.ev = ev;
    R.st = st;
    R.tie = tie;
    return R;
}

// Value of the running sum just before group element `pos` (pos <= first event),
// broadcast to the workgroup.
template <int NT, int EPT>
__device__ __forceinline__ float seq_value_at(const seq_find_res& R, const uint32_t (&excl)[EPT], int pos,
                                              seq_sh<NT>& sh) {
    if (threadIdx.x == pos / EPT) {
        uint32_t ex = seq_pick_u(excl, pos % EPT);
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
template <int NT, int EPT, class F>
__device__ __forceinline__ int seq_group_f(const F& f, int start, float& s, float thresh, seq_sh<NT>& sh) {
    const int t = threadIdx.x;
    while (start < NT * EPT) {
        uint32_t excl[EPT];
        seq_find_res R = seq_find<NT, EPT>(f, start, s, thresh, excl, sh);
        if (R.st < R.ev) return R.st;
        if (R.ev == ZS_BIGI) {
            s = zs_grid_value(R.k0 + R.total, R.eg);
            return -1;
        }
        if (t == R.ev / EPT) {
            const int jj = R.ev % EPT;
            uint32_t ex = seq_pick_u(excl, jj);
            float sb = zs_grid_value(R.k0 + ex, R.eg);
            float ns = sb + f.val(jj);
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

template <int NT, int EPT>
__device__ __forceinline__ int seq_group(const float (&tv)[EPT], int start, float& s, float thresh,
                                         seq_sh<NT>& sh) {
    seq_terms<EPT> f(tv);
    return seq_group_f<NT, EPT>(f, start, s, thresh, sh);
}

// Adds the same term t to the running sum s up to c times, one thread, in
// closed form per binade: on a fixed grid the increment is constant once the
// parity rule is settled (a tie term moves k to an even value on its first
// addition and keeps it even). Returns the 0-based count of the addition
// after which s >= thresh (s is then that sum), or -1 with s = the sum after
// all c additions.
__device__ __forceinline__ long long seq_repeat(float& s, float t, uint32_t c, float thresh) {
    uint32_t done = 0;
    while (done < c) {
        const int eg = zs_grid_exp(s);
        const uint32_t k = zs_grid_k(s);
        seq_pair p = seq_pair_of(t, eg);
        const uint32_t inc = (k & 1u) ? p.o : p.e;
        const bool steady = (p.e == p.o) || !(inc & 1u);
        if (inc == 0u) {
            // the sum no longer moves: no further stop possible
            return -1;
        }
        if (!steady || k + inc >= ZS_BINADE) {
            s = s + t;
            done++;
            if (s >= thresh) return (long long)done - 1;
            continue;
        }
        // additions that stay inside the binade: k + n*inc < 2^24
        uint32_t n = (ZS_BINADE - 1u - k) / inc;
        if (n > c - done) n = c - done;
        const uint32_t kthr = zs_grid_thresh(thresh, eg);
        if (kthr != 0xffffffffu && k + (unsigned long long)n * inc >= kthr) {
            const uint32_t need = kthr <= k ? 1u : (kthr - k + inc - 1u) / inc;
            s = zs_grid_value(k + need * inc, eg);
            return (long long)done + need - 1;
        }
        s = zs_grid_value(k + n * inc, eg);
        done += n;
    }
    return -1;
}
