// zs_sample.hip -- the per-step sampler over a batch of fp32 logit rows.
//
// Reference semantics (per row, in the order of rest.rs:2594-2624):
//   x~ = apply_mask(x)                    logit_fsm.rs:247-270 (bans, allow bits)
//   y  = adjust_logits(x~)                decode_ctrl.rs:107-126
//   token = sample_with_rng(y, cfg, r)    sampler.rs:31-128
//   logprobs / token_uncertainty on x~    logprobs.rs:34-54, hallucination.rs:129-154
//
// Kernels (one launch each, in stream order):
//   zs_k_row      (zs_row.hip) one workgroup per row: patch list, candidate
//                 lists, the sampler's decisions (greedy, non-finite, top-k and
//                 small survivor sets sampled on chip); the other rows are
//                 "big".
//   zs_k_sapx, zs_k_sround, zs_k_sstitch   (zs_sums.hip) the exact row sums:
//                 the observers' S and a big row's sampler S, then the entropy
//                 (on the context's side stream, joined before zs_k_final).
//   zs_k_pv .. zs_k_tp_sort   big rows: probabilities and the top-p bucket plan.
//   zs_k_big      one 1024-thread workgroup per big row: top-k select, min-p,
//                 the top-p walk.
//   zs_k_kcount, zs_k_kwrite, zs_k_roundK, zs_k_stitchK   the kept list: its
//                 sum and the draw.
//   zs_k_final    chosen-token outputs.
//
// Exactness: every value that decides the sampled id is computed with the same
// IEEE f32 operations as the reference (glibc-identical expf, IEEE division,
// sequential sums reproduced exactly, see zs_math.h), so sampled ids are
// bit-identical to sampler.rs for the same uniform r.
#include <hip/hip_runtime.h>
#include "zs_internal.h"
#include "zs_dev.h"
#include "zs_seq.h"
#include "zs_terms.h"
#include "zs_sampler.h"
#include "zs_walk.h"

// ===========================================================================
// zs_k_big: exact emulation of the reference's sequential sums over a full row.
// ===========================================================================
#define BK_NB 2048   // buckets per level of the top-p walk
#define BK_NC 4      // copies of each bucket counter (by lane)
#define BK_SERIAL 128   // exact buckets up to this size are walked by one thread
#ifndef BK_WEPT
#define BK_WEPT 4  // values per thread of one quick-walk group
#endif
#define BK_WG (ZS_BIG_NT * BK_WEPT)
static_assert(BK_NB * BK_NC <= ZS_SORT_CAP, "per-copy bucket counters live in the sort buffer");

struct big_shared {
    seq_sh<ZS_BIG_NT> q;
    uint32_t u[8];
    float s;
    uint32_t hist[BK_NB + 1];    // level 0: bucket starts by rank (rank 0 = largest values)
    uint32_t hist1[BK_NB + 1];   // level 1 (refinement of one oversize bucket)
    uint32_t hist2[256];         // level 2: counts of single values
    alignas(16) uint32_t sortbuf[ZS_SORT_CAP];
};

struct big_row {
    const float* row;
    const uint32_t* allow;
    bool masked;
    const uint32_t* pid;
    const uint32_t* pfl;
    const float* py;
    const uint32_t* psub;
    uint32_t nsub;
    uint32_t V;
    float T;
};

// Raw loads of group g for thread t: 4 logits and the allow word.
struct big_raw {
    float4 v;
    uint32_t w;
};
// (tix: the thread's slot of the group's ZS_BIG_NT; a smaller workgroup takes
// several slots)
__device__ __forceinline__ big_raw big_fetch(const big_row& R, uint32_t g, uint32_t tix = threadIdx.x) {
    const uint32_t idx0 = g * ZS_BIG_G + 4 * tix;
    big_raw o;
    o.v = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    o.w = 0xffffffffu;
    if (idx0 < R.V) {
        o.v = *reinterpret_cast<const float4*>(R.row + idx0);
        if (R.masked) o.w = R.allow[idx0 >> 5] >> (idx0 & 31);
    }
    return o;
}
// x~ (observers: mask and bans) and z (sampler: patched y, divided by T) of the
// 4 elements idx0..idx0+3 of group g; the group's patches are those of its
// ZS_BIG_G / ZS_SUB sub-chunks (per-sub-chunk patch offsets written by zs_k_row).
__device__ __forceinline__ void big_finish(const big_row& R, uint32_t g, const big_raw& raw, float (&x)[4],
                                           float (&z)[4], uint32_t tix = threadIdx.x) {
    const uint32_t idx0 = g * ZS_BIG_G + 4 * tix;
    x[0] = raw.v.x; x[1] = raw.v.y; x[2] = raw.v.z; x[3] = raw.v.w;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if (idx0 + q >= R.V) x[q] = -INFINITY;
        else if (R.masked && !((raw.w >> q) & 1u)) x[q] = -INFINITY;
        z[q] = x[q];
    }
    const uint32_t s0 = g * (ZS_BIG_G / ZS_SUB);
    const uint32_t p0 = R.psub[s0], p1 = R.psub[min(s0 + ZS_BIG_G / ZS_SUB, R.nsub)];
    for (uint32_t p = p0; p < p1; p++) {
        uint32_t off = R.pid[p] - idx0;
        if (off < 4) {
            uint32_t fl = R.pfl[p];
            float py = R.py[p];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                if ((uint32_t)q != off) continue;
                if (fl & ZS_PF_BAN) { x[q] = -INFINITY; z[q] = -INFINITY; }
                if (fl & ZS_PF_Y) z[q] = py;
            }
        }
    }
    // (-inf stays -inf: with T = inf, -inf / T is NaN, but a row with a real
    // -inf element is non-finite and never reaches these kernels; the -inf
    // here are ids past the row)
#pragma unroll
    for (int q = 0; q < 4; q++) z[q] = z[q] == -INFINITY ? -INFINITY : zs_temper(z[q], R.T);
}
__device__ __forceinline__ void big_load2(const big_row& R, uint32_t g, float (&x)[4], float (&z)[4],
                                          big_shared& sh) {
    big_finish(R, g, big_fetch(R, g), x, z);
}
// Calls f(g, z) for every group in order, with the loads of BK_U groups in
// flight at once (a single 16-byte load per thread leaves a one-workgroup
// stream latency-bound). f returns true to stop; it must be uniform.
#define BK_U 8
template <class F>
__device__ __forceinline__ void big_stream_z(const big_row& R, uint32_t ng, const F& f) {
    for (uint32_t g0 = 0; g0 < ng; g0 += BK_U) {
        big_raw raw[BK_U];
#pragma unroll
        for (int u = 0; u < BK_U; u++) raw[u] = g0 + u < ng ? big_fetch(R, g0 + u) : big_raw{};
#pragma unroll
        for (int u = 0; u < BK_U; u++) {
            if (g0 + u >= ng) break;
            float x[4], z[4];
            big_finish(R, g0 + u, raw[u], x, z);
            if (f(g0 + u, z)) return;
        }
    }
}
__device__ __forceinline__ void big_load_z(const big_row& R, uint32_t g, float (&z)[4], big_shared& sh) {
    float x[4];
    big_load2(R, g, x, z, sh);
}

__device__ __forceinline__ float big_term_e(float z, bool has_thr, float thr, float m) {
    if (has_thr && z < thr) return 0.0f;
    return zs_expf(z - m);
}

// ---------------------------------------------------------------------------
// Exact top-p walk (sampler.rs:91-104): the running f32 sum over the
// probabilities in (p desc, index asc) order, up to the first element after
// which it reaches top_p. The sum depends on the order only through parity
// ties and binade crossings (events): inside a binade, every non-tie term adds
// a fixed integer number of grid units whatever its position. Values are
// therefore bucketed by their high bits and visited bucket by bucket in
// descending order, in any order inside a bucket; a bucket holding an event,
// a tie or the stop is redone in exact descending order -- sorted in LDS, or,
// when larger than the LDS, refined by the next 11 bits, and at the last level
// (all values share their 24 high bits) walked as repeated values by count.
// Equal values are adjacent in that order, and the stop is reported as
// (value, rank among the equal values passed): the index order among equal
// probabilities is resolved afterwards on the row.
// ---------------------------------------------------------------------------
struct walk_out {
    bool stopped;
    uint32_t v;      // stop value (f32 bits)
    uint32_t rank;   // 0-based rank of the stop among the elements equal to v
};

// descending bitonic sort of n (power of two) u32 values in LDS
__device__ __forceinline__ void bk_sort_desc(uint32_t* a, int n) {
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += ZS_BIG_NT) {
                int ixj = i ^ j;
                if (ixj > i) {
                    uint32_t x = a[i], y = a[ixj];
                    bool desc = (i & k) == 0;
                    if ((x < y) == desc) { a[i] = y; a[ixj] = x; }
                }
            }
            __syncthreads();
        }
    }
}

// The same for np2 <= ZS_BIG_NT, one value per thread: exchanges inside a
// wave by shuffles, only the strides of 64 and more through LDS.
__device__ __forceinline__ void bk_sort_desc_small(uint32_t* a, int np2) {
    const int t = threadIdx.x;
    uint32_t x = t < np2 ? a[t] : 0u;
    for (int k = 2; k <= np2; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            uint32_t y;
            if (j >= 64) {
                if (t < np2) a[t] = x;
                __syncthreads();
                y = t < np2 ? a[t ^ j] : 0u;
                __syncthreads();
            } else {
                y = __shfl_xor(x, j, 64);
            }
            const bool desc = (t & k) == 0, lower = (t & j) == 0;
            x = (lower == desc) ? max(x, y) : min(x, y);
        }
    }
    if (t < np2) a[t] = x;
    __syncthreads();
}

// Walk n <= ZS_SORT_CAP values in exact descending order (sorted in LDS).
__device__ __forceinline__ walk_out bk_walk_sorted(const uint32_t* vals, uint32_t n, float& s, float thresh, big_shared& sh) {
    walk_out o = {false, 0u, 0u};
    uint32_t np2 = 1;
    while (np2 < n) np2 <<= 1;
    for (uint32_t i = threadIdx.x; i < np2; i += ZS_BIG_NT) sh.sortbuf[i] = i < n ? vals[i] : 0u;
    __syncthreads();
    if (np2 > ZS_BIG_NT) bk_sort_desc(sh.sortbuf, (int)np2);
    else if (np2 > 1) bk_sort_desc_small(sh.sortbuf, (int)np2);
    if (n <= BK_SERIAL) {
        // a bucket of this size is walked faster by one thread than by the
        // workgroup scan (whose cost is its latency chain, not its width)
        if (threadIdx.x == 0) {
            float ss = s;
            uint32_t stp = 0xffffffffu;
            for (uint32_t i0 = 0; i0 < n && stp == 0xffffffffu; i0 += 8) {
                float v8[8];
#pragma unroll
                for (int q = 0; q < 8; q++) v8[q] = i0 + q < n ? zs_u2f(sh.sortbuf[i0 + q]) : 0.0f;
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    if (stp != 0xffffffffu || i0 + q >= n) continue;
                    ss = ss + v8[q];
                    if (ss >= thresh) stp = i0 + q;
                }
            }
            sh.s = ss;
            sh.u[4] = stp;
        }
        __syncthreads();
        s = sh.s;
        const uint32_t stp = sh.u[4];
        __syncthreads();
        if (stp != 0xffffffffu) {
            const uint32_t v = sh.sortbuf[stp];
            uint32_t lo = 0, hi = stp;
            while (lo < hi) {
                uint32_t mid = (lo + hi) >> 1;
                if (sh.sortbuf[mid] > v) lo = mid + 1; else hi = mid;
            }
            o.stopped = true;
            o.v = v;
            o.rank = stp - lo;
        }
        __syncthreads();
        return o;
    }
    for (uint32_t q0 = 0; q0 < n; q0 += ZS_BIG_G) {
        float tv[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint32_t i = q0 + 4 * threadIdx.x + q;
            tv[q] = i < n ? zs_u2f(sh.sortbuf[i]) : 0.0f;
        }
        int stp = seq_group<ZS_BIG_NT, 4>(tv, 0, s, thresh, sh.q);
        if (stp >= 0) {
            const uint32_t pos = q0 + (uint32_t)stp;
            const uint32_t v = sh.sortbuf[pos];
            // first position holding v (the sorted values are descending)
            uint32_t lo = 0, hi = pos;
            while (lo < hi) {
                uint32_t mid = (lo + hi) >> 1;
                if (sh.sortbuf[mid] > v) lo = mid + 1; else hi = mid;
            }
            o.stopped = true;
            o.v = v;
            o.rank = pos - lo;
            break;
        }
    }
    __syncthreads();
    return o;
}

// Last level: all n values share bits 31..8 (`prefix`); count each of the 256
// possible values and add them as repeated terms, largest first.
__device__ __forceinline__ walk_out bk_walk_counts(const uint32_t* vals, uint32_t n, uint32_t prefix, float& s, float thresh,
                                   big_shared& sh) {
    uint32_t* cc = sh.sortbuf;  // per (value, copy) counts
    for (int i = threadIdx.x; i < 256 * BK_NC; i += ZS_BIG_NT) cc[i] = 0;
    __syncthreads();
    const uint32_t cp = threadIdx.x & (BK_NC - 1);
    for (uint32_t i = threadIdx.x; i < n; i += ZS_BIG_NT) atomicAdd(&cc[(vals[i] & 255u) * BK_NC + cp], 1u);
    __syncthreads();
    for (int i = threadIdx.x; i < 256; i += ZS_BIG_NT) {
        uint32_t c = 0;
#pragma unroll
        for (int k = 0; k < BK_NC; k++) c += cc[i * BK_NC + k];
        sh.hist2[i] = c;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        float ss = s;
        uint32_t stopped = 0, v = 0, rank = 0;
        for (int lo = 255; lo >= 0 && !stopped; lo--) {
            const uint32_t c = sh.hist2[lo];
            if (!c) continue;
            const uint32_t bits = prefix | (uint32_t)lo;
            long long k = seq_repeat(ss, zs_u2f(bits), c, thresh);
            if (k >= 0) { stopped = 1; v = bits; rank = (uint32_t)k; }
        }
        sh.s = ss;
        sh.u[4] = stopped;
        sh.u[5] = v;
        sh.u[6] = rank;
    }
    __syncthreads();
    walk_out o;
    s = sh.s;
    o.stopped = sh.u[4] != 0;
    o.v = sh.u[5];
    o.rank = sh.u[6];
    __syncthreads();
    return o;
}

// Bucket index of value v at level L (0: bits 31..19, 1: bits 18..8), as a rank
// (0 = the bucket of the largest values).
template <int L>
__device__ __forceinline__ uint32_t bk_rank(uint32_t v) {
    return L == 0 ? (BK_NB - 1u) - min(v >> 19, (uint32_t)(BK_NB - 1)) : (BK_NB - 1u) - ((v >> 8) & (BK_NB - 1u));
}

template <int L>
__device__ __forceinline__ walk_out bk_exact(const uint32_t* vals, uint32_t n, float& s, float thresh, uint32_t* tmp, big_shared& sh);

// Walk vals[from, to), laid out bucket by bucket (level L, starts in `start`),
// from running sum s. The values of a bucket are in any order.
template <int L>
__device__ __forceinline__ walk_out bk_walk(const uint32_t* vals, uint32_t from, uint32_t to, const uint32_t* start, float& s,
                            float thresh, uint32_t* tmp, big_shared& sh) {
    walk_out o = {false, 0u, 0u};
    uint32_t pos = from;
    float s_bstart = s;  // running sum at the start of the bucket open at pos
    while (pos < to) {
        float tv[BK_WEPT];
#pragma unroll
        for (int q = 0; q < BK_WEPT; q++) {
            uint32_t ps = pos + BK_WEPT * threadIdx.x + q;
            tv[q] = ps < to ? zs_u2f(vals[ps]) : 0.0f;
        }
        uint32_t excl[BK_WEPT];
        seq_find_res F = seq_find<ZS_BIG_NT, BK_WEPT>(seq_terms<BK_WEPT>(tv), 0, s, thresh, excl, sh.q);
        const int first = min(min(F.ev, F.st), F.tie);
        if (first == ZS_BIGI) {
            const uint32_t last = min(pos + BK_WG, to) - 1;
            const uint32_t bst = start[bk_rank<L>(vals[last])];
            if (bst >= pos) s_bstart = seq_value_at<ZS_BIG_NT, BK_WEPT>(F, excl, (int)(bst - pos), sh.q);
            s = zs_grid_value(F.k0 + F.total, F.eg);
            pos += BK_WG;
            continue;
        }
        // the bucket holding the first event / tie / stop is redone in exact order
        const uint32_t rk = bk_rank<L>(vals[pos + (uint32_t)first]);
        const uint32_t bst = start[rk], bend = start[rk + 1];
        if (bst >= pos) s = seq_value_at<ZS_BIG_NT, BK_WEPT>(F, excl, (int)(bst - pos), sh.q);
        else s = s_bstart;
        o = bk_exact<L + 1>(vals + bst, bend - bst, s, thresh, tmp, sh);
        if (o.stopped) return o;
        s_bstart = s;
        pos = bend;
    }
    return o;
}

// Exact descending walk of one bucket of level L-1 (its values share the
// bucket's high bits).
template <int L>
__device__ __forceinline__ walk_out bk_exact(const uint32_t* vals, uint32_t n, float& s, float thresh, uint32_t* tmp, big_shared& sh) {
    if (n <= ZS_SORT_CAP) return bk_walk_sorted(vals, n, s, thresh, sh);
    if constexpr (L >= 2) {
        return bk_walk_counts(vals, n, vals[0] & ~255u, s, thresh, sh);
    } else {
        // refine by bits 18..8 into tmp, bucket by bucket
        uint32_t* cur = sh.sortbuf;  // counts, then cursors, per (rank, copy)
        const uint32_t cp = threadIdx.x & (BK_NC - 1);
        for (int i = threadIdx.x; i < BK_NB * BK_NC; i += ZS_BIG_NT) cur[i] = 0;
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < n; i += ZS_BIG_NT) atomicAdd(&cur[bk_rank<1>(vals[i]) * BK_NC + cp], 1u);
        __syncthreads();
        {
            uint32_t c2[2];
#pragma unroll
            for (int k2 = 0; k2 < 2; k2++) {
                const int rk = 2 * threadIdx.x + k2;
                uint32_t c = 0;
#pragma unroll
                for (int k = 0; k < BK_NC; k++) c += cur[rk * BK_NC + k];
                c2[k2] = c;
            }
            uint32_t ctot;
            const uint32_t cex = block_excl_scan_u<ZS_BIG_NT>(c2[0] + c2[1], sh.hist2, &ctot);
            sh.hist1[2 * threadIdx.x] = cex;
            sh.hist1[2 * threadIdx.x + 1] = cex + c2[0];
            if (threadIdx.x == 0) sh.hist1[BK_NB] = ctot;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < BK_NB; i += ZS_BIG_NT) {
            uint32_t acc = sh.hist1[i];
#pragma unroll
            for (int k = 0; k < BK_NC; k++) { uint32_t c = cur[i * BK_NC + k]; cur[i * BK_NC + k] = acc; acc += c; }
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < n; i += ZS_BIG_NT) {
            const uint32_t v = vals[i];
            tmp[atomicAdd(&cur[bk_rank<1>(v) * BK_NC + cp], 1u)] = v;
        }
        __threadfence_block();
        __syncthreads();
        return bk_walk<1>(tmp, 0, n, sh.hist1, s, thresh, nullptr, sh);
    }
}

// The sampler's softmax denominator of a big row is known before zs_k_big when
// the rounds summed it (every big row but those whose top-k threshold
// zs_k_big selects).
__device__ __forceinline__ bool big_s_from_rounds(const zs_row_state& st) {
    return ((st.rounds >> ZS_SUM_SAMP_S) & 1u) != 0u;
}
__device__ __forceinline__ float big_s_value(const zs_row_state& st) { return st.samp_S; }

// Rows whose top-p walk runs on bucket totals (zs_k_tp_*): p comes from
// zs_k_pv, no min-p (the walked values are the p themselves), the top-k
// threshold is known, and the largest p alone stays below top_p (else the walk
// stops at its first element).
__device__ __forceinline__ bool tp_fast_row(const zs_row_state& st, const zs_row_params& P) {
    if (st.mode != ZS_MODE_BIG || !big_s_from_rounds(st) || st.has_thr == 2) return false;
    if (P.min_p > 0.0f || !(P.top_p < 1.0f && P.top_p > 0.0f)) return false;
    return !(1.0f / big_s_value(st) >= P.top_p);
}

// Probabilities p = exp(z - max) / S (sampler.rs:68-69) of the big rows whose
// S is known, one workgroup per (group of ZS_BIG_G elements, row): the exact
// exponentials are the bulk of a big row's arithmetic, spread here over the
// whole GPU instead of one workgroup per row. Rows of the bucket-total walk
// also add their positive p to the per-bucket counts and masses.
// 256-thread workgroups, each thread 4 of the group's ZS_BIG_NT slots: most
// rows of a batch are not big, and launching their workgroups' waves (which
// only read the row state) costs in proportion to the waves
#define PV_NT 256
__global__ __launch_bounds__(PV_NT) void zs_k_pv(zs_sargs a) {
    const uint32_t g = blockIdx.x, r = blockIdx.y;
    // (the presort task list of this step starts empty: zs_k_tp_plan and
    // zs_k_tp_inc, launched after this kernel, append to it)
    if (g == 0 && r == 0 && threadIdx.x == 0) a.tp_task[0] = 0u;
    const zs_row_state& st = a.rst[r];
    if (st.mode != ZS_MODE_BIG || !big_s_from_rounds(st)) return;
    const zs_batch& b = a.b;
    const uint32_t V = b.V;
    const zs_row_params P = b.d_params[r];
    const bool hist = tp_fast_row(st, P);
    __shared__ uint32_t hc[ZS_TP_NB];
    __shared__ float hm[ZS_TP_NB];
    if (hist) {
        for (uint32_t i = threadIdx.x; i < ZS_TP_NB; i += PV_NT) { hc[i] = 0u; hm[i] = 0.0f; }
        __syncthreads();
    }
    big_row R;
    R.row = b.d_logits + (size_t)r * b.ld;
    R.masked = (P.flags & ZS_ROW_MASKED) && b.d_allow_bits;
    R.allow = R.masked ? b.d_allow_bits + (size_t)r * b.allow_words : nullptr;
    R.pid = a.p_id + (size_t)r * a.pstride;
    R.pfl = a.p_flags + (size_t)r * a.pstride;
    R.py = a.p_y + (size_t)r * a.pstride;
    R.psub = a.p_sub + (size_t)r * (a.max_subs + 1);
    R.nsub = (V + ZS_SUB - 1) / ZS_SUB;
    R.V = V;
    R.T = P.temperature;
    const bool use_thr = st.has_thr != 0;
    const float thr = zs_key_to_float(st.thr_key), m = st.z_max, S = big_s_value(st);
    constexpr int NS = ZS_BIG_NT / PV_NT;
    big_raw raw[NS];
#pragma unroll
    for (int u = 0; u < NS; u++) raw[u] = big_fetch(R, g, threadIdx.x + u * PV_NT);
#pragma unroll
    for (int u = 0; u < NS; u++) {
        const uint32_t tix = threadIdx.x + u * PV_NT, idx0 = g * ZS_BIG_G + 4 * tix;
        if (idx0 >= V) break;
        float x[4], z[4];
        big_finish(R, g, raw[u], x, z, tix);
        uint4 o;
        uint32_t* ob = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
        for (int q = 0; q < 4; q++) ob[q] = zs_f2u(idx0 + q < V ? big_term_e(z[q], use_thr, thr, m) / S : 0.0f);
        *reinterpret_cast<uint4*>(a.pv + (size_t)r * a.max_vocab + idx0) = o;
        if (hist) {
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float p = zs_u2f(ob[q]);
                if (p > 0.0f) {
                    const uint32_t rk = bk_rank<0>(ob[q]);
                    atomicAdd(&hc[rk], 1u);
                    atomicAdd(&hm[rk], p);
                }
            }
        }
    }
    if (hist) {
        __syncthreads();
        zs_tp_bucket* bk = a.tp_bk + (size_t)r * ZS_TP_NB;
        for (uint32_t i = threadIdx.x; i < ZS_TP_NB; i += PV_NT) {
            if (hc[i]) {
                atomicAdd(&bk[i].cnt, hc[i]);
                atomicAdd(&bk[i].mass, hm[i]);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Top-p walk on bucket totals (sampler.rs:91-104), for the rows of
// tp_fast_row. The running f32 sum over the p in descending order is fixed by
// integer increments inside each binade of the sum (zs_math.h), so a bucket
// the sum crosses without an event adds the total of its elements' increments
// on the grid of that binade, whatever their order. The kernels below
//   zs_k_tp_plan  (one workgroup per row): bucket starts, the predicted grid of
//                 every bucket from the approximate prefix masses, and the
//                 candidate buckets that may hold an event (the prefix range,
//                 widened by a bound on the f32 rounding error, crosses a
//                 power of two or top_p; the first bucket);
//   zs_k_tp_inc   (all CUs): per-bucket increment totals on the predicted grid
//                 and the exact-half (tie) flags; every positive p is gathered
//                 into the bucket layout; buckets with ties become candidates;
//   zs_k_tp_sort  (one workgroup per candidate): sorts the bucket in
//                 descending order and stores the prefix of its increment
//                 maps on the predicted grid (a parity pair, so ties are
//                 exact) and the prefix of its increments on the next grid;
// leave the walk itself to one wave in zs_k_big (tp_walk), which adds bucket
// totals with wave scans and resolves a bucket with an event by binary
// searches on the stored prefixes (or by adding its sorted values one by one).
// A walk that meets anything it cannot resolve exactly (an event in a bucket
// that was not presorted, a grid other than the two prepared) reports failure
// and the row takes the workgroup walk below.
// ---------------------------------------------------------------------------
#define TP_M_EG 0xffu
#define TP_M_CAND 0x100u
#define TP_M_TIE0 0x200u
#define TP_M_TIE1 0x400u
#define TP_M_SORTED 0x800u
#define TP_ROW_FAST 1u
#define TP_SORT_MAX 4096
#define TP_SORT_NT 1024
#define TP_SERIAL_N 512

__global__ __launch_bounds__(ZS_BIG_NT) void zs_k_tp_plan(zs_sargs a) {
    const uint32_t r = blockIdx.x;
    const int t = threadIdx.x;
    uint32_t* cl = a.tp_cl + (size_t)r * ZS_TP_CL;
    const zs_row_state& st = a.rst[r];
    const zs_row_params P = a.b.d_params[r];
    if (!tp_fast_row(st, P)) {
        if (t == 0) cl[0] = 0u;
        return;
    }
    __shared__ uint32_t su[ZS_BIG_NT / 64];
    __shared__ double sd[ZS_BIG_NT / 64];
    zs_tp_bucket* bk = a.tp_bk + (size_t)r * ZS_TP_NB;
    static_assert(ZS_TP_NB == 2 * ZS_BIG_NT, "two buckets per thread");
    uint32_t c[2];
    double m[2];
#pragma unroll
    for (int k2 = 0; k2 < 2; k2++) {
        c[k2] = bk[2 * t + k2].cnt;
        m[k2] = (double)bk[2 * t + k2].mass;
    }
    uint32_t ctot;
    double mtot;
    const uint32_t cex = block_excl_scan_u<ZS_BIG_NT>(c[0] + c[1], su, &ctot);
    const double mex = block_excl_scan_d<ZS_BIG_NT>(m[0] + m[1], sd, &mtot);
    const double top_p = (double)P.top_p;
    uint32_t cand[2], meta[2];
#pragma unroll
    for (int k2 = 0; k2 < 2; k2++) {
        const uint32_t start = cex + (k2 ? c[0] : 0u);
        const double P0 = k2 ? mex + m[0] : mex, P1 = P0 + m[k2];
        // margin for |f32 running sum - prefix mass| (rounding of the additions
        // and of the float mass accumulation); a wrong prediction is caught by
        // the walk, so this is a typical bound, not a worst case
        const double delta = ldexp(P1 * (16.0 * sqrt((double)(start + c[k2])) + 64.0), -24) + 1e-30;
        const double lo = P0 - delta > 0.0 ? P0 - delta : 0.0, hi = P1 + delta;
        // the sum stops at top_p: buckets past it are never walked, and a
        // binade above top_p is never entered
        const int e0 = zs_grid_exp((float)lo), e1 = zs_grid_exp((float)fmin(hi, top_p));
        const bool cd = c[k2] != 0u && lo < top_p && (P0 == 0.0 || e0 != e1 || hi >= top_p);
        cand[k2] = cd ? 1u : 0u;
        meta[k2] = (uint32_t)(cd ? e0 : e1) | (cd ? TP_M_CAND : 0u);
        zs_tp_bucket& B = bk[2 * t + k2];
        B.start = start;
        B.cur = start;
        B.meta = meta[k2];
        B.tot = 0ull;
    }
    uint32_t ntot;
    const uint32_t pos = block_excl_scan_u<ZS_BIG_NT>(cand[0] + cand[1], su, &ntot);
    if (ntot > ZS_TP_CAND) {
        if (t == 0) cl[0] = 0u;
        return;
    }
    uint32_t q = pos;
#pragma unroll
    for (int k2 = 0; k2 < 2; k2++)
        if (cand[k2]) cl[2 + q++] = 2 * t + k2;
    if (t == 0) {
        cl[0] = TP_ROW_FAST;
        cl[1] = ntot;
        const uint32_t base = ntot ? atomicAdd(&a.tp_task[0], ntot) : 0u;
        for (uint32_t j = 0; j < ntot; j++) a.tp_task[1 + base + j] = (r << 8) | j;
    }
}

__global__ __launch_bounds__(ZS_BIG_NT) void zs_k_tp_inc(zs_sargs a) {
    const uint32_t g = blockIdx.x, r = blockIdx.y;
    uint32_t* cl = a.tp_cl + (size_t)r * ZS_TP_CL;
    if (!(cl[0] & TP_ROW_FAST)) return;
    const uint32_t V = a.b.V;
    const int t = threadIdx.x;
    __shared__ uint32_t lc[ZS_TP_NB];
    __shared__ unsigned long long lt[ZS_TP_NB];
    __shared__ uint32_t lf[ZS_TP_NB];
    for (uint32_t i = t; i < ZS_TP_NB; i += ZS_BIG_NT) { lc[i] = 0u; lt[i] = 0ull; lf[i] = 0u; }
    __syncthreads();
    zs_tp_bucket* bk = a.tp_bk + (size_t)r * ZS_TP_NB;
    const uint32_t idx0 = g * ZS_BIG_G + 4 * t;
    uint4 v = idx0 < V ? *reinterpret_cast<const uint4*>(a.pv + (size_t)r * a.max_vocab + idx0) : make_uint4(0u, 0u, 0u, 0u);
    const uint32_t pb[4] = {v.x, v.y, v.z, v.w};
    uint32_t off[4], rk[4];
#pragma unroll
    for (int q = 0; q < 4; q++) {
        rk[q] = bk_rank<0>(pb[q]);
        off[q] = 0u;
        if (zs_u2f(pb[q]) > 0.0f) {
            const int eg = (int)(bk[rk[q]].meta & TP_M_EG);
            const seq_pair pr = seq_pair_of(zs_u2f(pb[q]), eg);
            off[q] = atomicAdd(&lc[rk[q]], 1u);
            atomicAdd(&lt[rk[q]], (unsigned long long)pr.e);
            if (pr.e != pr.o) lf[rk[q]] = 1u;
        }
    }
    __syncthreads();
    for (uint32_t i = t; i < ZS_TP_NB; i += ZS_BIG_NT) {
        if (!lc[i]) continue;
        lc[i] = atomicAdd(&bk[i].cur, lc[i]);  // this group's base in the bucket
        atomicAdd(&bk[i].tot, lt[i]);
        if (lf[i]) {
            const uint32_t old = atomicOr(&bk[i].meta, TP_M_TIE0);
            if (!(old & (TP_M_TIE0 | TP_M_CAND))) {
                const uint32_t j = atomicAdd(&cl[1], 1u);
                if (j < ZS_TP_CAND) {
                    cl[2 + j] = i;
                    a.tp_task[1 + atomicAdd(&a.tp_task[0], 1u)] = (r << 8) | j;
                }
            }
        }
    }
    __syncthreads();
    uint32_t* gv = a.pairs + (size_t)r * a.max_vocab * 2;
#pragma unroll
    for (int q = 0; q < 4; q++)
        if (zs_u2f(pb[q]) > 0.0f) gv[lc[rk[q]] + off[q]] = pb[q];
}

// Composition of increment maps over a workgroup, in thread order: exclusive
// prefix of the thread maps (and of plain saturating sums alongside).
template <int NT>
__device__ __forceinline__ seq_pair tp_block_excl_pairs(seq_pair v, uint32_t& sv, uint32_t* sh, uint32_t* tot_s) {
    const int lane = zs_lane(), w = zs_wid();
    seq_pair inc = v;
    uint32_t sinc = sv;
    for (int d = 1; d < 64; d <<= 1) {
        seq_pair y;
        y.e = __shfl_up(inc.e, d, 64);
        y.o = __shfl_up(inc.o, d, 64);
        const uint32_t ys = __shfl_up(sinc, d, 64);
        if (lane >= d) { inc = seq_compose(y, inc); sinc = zs_sat_add(ys, sinc); }
    }
    seq_pair ex;
    ex.e = __shfl_up(inc.e, 1, 64);
    ex.o = __shfl_up(inc.o, 1, 64);
    uint32_t sex = __shfl_up(sinc, 1, 64);
    if (lane == 0) { ex.e = ex.o = 0u; sex = 0u; }
    if (lane == 63) { sh[3 * w] = inc.e; sh[3 * w + 1] = inc.o; sh[3 * w + 2] = sinc; }
    __syncthreads();
    seq_pair pre = {0u, 0u};
    uint32_t spre = 0u, stot = 0u;
    for (int i = 0; i < NT / 64; i++) {
        const seq_pair wi = {sh[3 * i], sh[3 * i + 1]};
        if (i < w) { pre = seq_compose(pre, wi); spre = zs_sat_add(spre, sh[3 * i + 2]); }
        stot = zs_sat_add(stot, sh[3 * i + 2]);
    }
    __syncthreads();
    *tot_s = stot;
    sv = zs_sat_add(spre, sex);
    return seq_compose(pre, ex);
}

// Bitonic compare-exchange step (k, j) over 4 values per thread, element i =
// 4 * thread + e, descending: strides 1 and 2 inside the thread, 4..255 by
// lane exchanges, larger ones through LDS.
__device__ __forceinline__ void tp_bitonic_step(uint32_t (&v)[4], uint32_t k, uint32_t j, uint32_t* sb) {
    const uint32_t t = threadIdx.x;
    if (j < 4u) {
#pragma unroll
        for (uint32_t e = 0; e < 4u; e++) {
            const uint32_t pe = e ^ j;
            if (pe > e) {
                const uint32_t i = 4u * t + e;
                const bool desc = (i & k) == 0u;
                const uint32_t x = v[e], y = v[pe];
                if ((x < y) == desc) { v[e] = y; v[pe] = x; }
            }
        }
        return;
    }
    uint32_t w[4];
    if (j < 256u) {
#pragma unroll
        for (uint32_t e = 0; e < 4u; e++) w[e] = __shfl_xor(v[e], (int)(j >> 2), 64);
    } else {
#pragma unroll
        for (uint32_t e = 0; e < 4u; e++) sb[4u * t + e] = v[e];
        __syncthreads();
#pragma unroll
        for (uint32_t e = 0; e < 4u; e++) w[e] = sb[(4u * t + e) ^ j];
        __syncthreads();
    }
#pragma unroll
    for (uint32_t e = 0; e < 4u; e++) {
        const uint32_t i = 4u * t + e;
        const bool desc = (i & k) == 0u, lower = (i & j) == 0u;
        v[e] = (lower == desc) ? max(v[e], w[e]) : min(v[e], w[e]);
    }
}

#ifdef ZS_WALK_DEBUG
// debug builds: sorted buckets by size class (<= 256, 1024, 4096), launches
__device__ unsigned long long ts_dbg[8];
extern "C" int zs_dbg_sort_stats(unsigned long long* out) {
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(ts_dbg), 8 * sizeof(unsigned long long)) != hipSuccess) return -1;
    static unsigned long long zero[8];
    return hipMemcpyToSymbol(HIP_SYMBOL(ts_dbg), zero, sizeof(zero)) == hipSuccess ? 0 : -1;
}
#endif
__device__ __forceinline__ void tp_sort_one(const zs_sargs& a, uint32_t c, uint32_t r) {
    const uint32_t t = threadIdx.x;
    const uint32_t* cl = a.tp_cl + (size_t)r * ZS_TP_CL;
    if (!(cl[0] & TP_ROW_FAST) || c >= min(cl[1], (uint32_t)ZS_TP_CAND)) return;
    const uint32_t bi = cl[2 + c];
    zs_tp_bucket* B = a.tp_bk + (size_t)r * ZS_TP_NB + bi;
    const uint32_t n = B->cnt, st0 = B->start;
    if (n == 0u || n > TP_SORT_MAX) return;
    __shared__ uint32_t sb[TP_SORT_MAX];
    __shared__ uint32_t sh[3 * TP_SORT_NT / 64];
    uint32_t* gv = a.pairs + (size_t)r * a.max_vocab * 2 + st0;
    uint32_t* q1 = gv + a.max_vocab;
    uint32_t* pe = a.tp_pre + (size_t)r * a.max_vocab * 2 + st0;
    uint32_t* po = pe + a.max_vocab;
    uint32_t np2 = 256;
    while (np2 < n) np2 <<= 1;
#ifdef ZS_WALK_DEBUG
    if (t == 0) atomicAdd(&ts_dbg[np2 <= 256 ? 0 : np2 <= 1024 ? 1 : 2], 1ull);
#endif
    uint32_t v[4];
#pragma unroll
    for (uint32_t e = 0; e < 4u; e++) {
        const uint32_t i = 4u * t + e;
        v[e] = i < n ? gv[i] : 0u;   // 0 (p = 0) sorts last
    }
    for (uint32_t k = 2; k <= np2; k <<= 1)
        for (uint32_t j = k >> 1; j > 0; j >>= 1) tp_bitonic_step(v, k, j, sb);
    // prefixes over the sorted order: thread t owns elements 4t..4t+3
    const int eg0 = (int)(B->meta & TP_M_EG), eg1 = eg0 + 1;
    seq_pair loc = {0u, 0u};
    uint32_t s1 = 0u, tie1 = 0u;
    seq_pair pr[4];
    uint32_t i1[4];
#pragma unroll
    for (uint32_t e = 0; e < 4u; e++) {
        const uint32_t i = 4u * t + e;
        const float x = i < n ? zs_u2f(v[e]) : 0.0f;
        pr[e] = seq_pair_of(x, eg0);
        uint32_t tie;
        i1[e] = zs_seq_inc(x, eg1, &tie);
        tie1 |= tie;
        loc = seq_compose(loc, pr[e]);
        s1 = zs_sat_add(s1, i1[e]);
    }
    uint32_t stot;
    seq_pair run = tp_block_excl_pairs<TP_SORT_NT>(loc, s1, sh, &stot);
    uint32_t srun = s1;
#pragma unroll
    for (uint32_t e = 0; e < 4u; e++) {
        const uint32_t i = 4u * t + e;
        run = seq_compose(run, pr[e]);
        srun = zs_sat_add(srun, i1[e]);
        if (i < n) {
            gv[i] = v[e];
            pe[i] = run.e;
            po[i] = run.o;
            q1[i] = srun;
        }
    }
    tie1 = __syncthreads_or(tie1);
    if (t == 0) atomicOr(&B->meta, TP_M_SORTED | (tie1 ? TP_M_TIE1 : 0u));
}
// One workgroup per listed (row, candidate bucket), from the task list of
// zs_k_tp_plan / zs_k_tp_inc: a small grid whatever the batch, so that rows
// without candidates cost no workgroups.
__global__ __launch_bounds__(TP_SORT_NT) void zs_k_tp_sort(zs_sargs a) {
    const uint32_t nt = a.tp_task[0];
    for (uint32_t i = blockIdx.x; i < nt; i += gridDim.x) {
        const uint32_t tk = a.tp_task[1 + i];
        tp_sort_one(a, tk & 0xffu, tk >> 8);
        __syncthreads();
    }
}

// First j in [lo, hi) with pred(j) (pred monotone: false then true), or hi;
// one wave, every lane calls it with the same arguments.
template <class F>
__device__ __forceinline__ uint32_t tp_first(uint32_t lo, uint32_t hi, const F& pred) {
    const uint32_t lane = (uint32_t)zs_lane();
    const uint32_t hi0 = hi;
    while (hi - lo > 64u) {
        const uint32_t seg = (hi - lo + 63u) / 64u;
        const uint32_t s0 = lo + lane * seg;
        const uint32_t j = min(s0 + seg, hi) - 1u;
        const unsigned long long m = __ballot(s0 < hi && pred(j));
        if (!m) return hi0;
        const uint32_t f = (uint32_t)__ffsll((long long)m) - 1u;
        const uint32_t nhi = min(lo + (f + 1u) * seg, hi);
        lo = lo + f * seg;
        hi = nhi;
    }
    const unsigned long long m = __ballot(lo + lane < hi && pred(lo + lane));
    return m ? lo + (uint32_t)__ffsll((long long)m) - 1u : hi0;
}

// The walk itself, by one wave (tp_fast_row rows): returns 1 with the stop
// (value, rank among equal values) in *wo, 2 when the sum never reaches top_p,
// 0 when the row must take the workgroup walk.
// Debug builds: wall-clock time of zs_k_big's phases, summed over rows
// (zs_dbg_big_stats): 0 top-k select, 1 S, 2 p / min-p, 3 top-p walk on bucket
// totals, 4 workgroup walk, 5 rest; 6 rows, 7 rows of the workgroup walk.
#ifdef ZS_WALK_DEBUG
__device__ unsigned long long bk_dbg[16];
#define BK_T(i)                                                  \
    do {                                                         \
        if (threadIdx.x == 0) {                                  \
            const unsigned long long c_ = wall_clock64();        \
            atomicAdd(&bk_dbg[i], c_ - bk_t0);                   \
            atomicMax(&bk_dbg[10 + (i)], c_ - bk_t0);            \
            bk_t0 = c_;                                          \
        }                                                        \
    } while (0)
extern "C" int zs_dbg_big_stats(unsigned long long* out) {
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(bk_dbg), 16 * sizeof(unsigned long long)) != hipSuccess) return -1;
    static unsigned long long zero[16];
    return hipMemcpyToSymbol(HIP_SYMBOL(bk_dbg), zero, sizeof(zero)) == hipSuccess ? 0 : -1;
}
#else
#define BK_T(i) do { } while (0)
#endif

#define TP_CH 1024   // values per LDS chunk of tp_walk's one-by-one additions
__device__ __forceinline__ int tp_walk(const zs_sargs& a, uint32_t r, float top_p, walk_out* wo, float* lbuf) {
    const uint32_t lane = (uint32_t)zs_lane();
    const zs_tp_bucket* bk = a.tp_bk + (size_t)r * ZS_TP_NB;
    const uint32_t* gv = a.pairs + (size_t)r * a.max_vocab * 2;
    const uint32_t* q1 = gv + a.max_vocab;
    const uint32_t* pe = a.tp_pre + (size_t)r * a.max_vocab * 2;
    const uint32_t* po = pe + a.max_vocab;
    float s = 0.0f;
    int eg = zs_grid_exp(s);
    unsigned long long k = 0ull;
    uint32_t kthr = zs_grid_thresh(top_p, eg);
    auto set_sum = [&](float ns) {
        s = ns;
        eg = zs_grid_exp(s);
        k = zs_grid_k(s);
        kthr = zs_grid_thresh(top_p, eg);
    };
    // the bucket records of the next two groups of 64 are loaded ahead; after
    // a bucket with an event the walk goes on in the same group (lanes from
    // l0 on), with no reload
    struct grp_ld { uint32_t cnt, meta, start; unsigned long long tot; };
    auto load = [&](uint32_t b) {
        grp_ld g = {0u, 0u, 0u, 0ull};
        if (b + lane < ZS_TP_NB) {
            g.cnt = bk[b + lane].cnt; g.meta = bk[b + lane].meta; g.start = bk[b + lane].start; g.tot = bk[b + lane].tot;
        }
        return g;
    };
    uint32_t b0 = 0, l0 = 0;
#ifdef ZS_WALK_DEBUG
    uint32_t d_ev = 0, d_ser = 0, d_bs = 0;
    unsigned long long d_t = 0;
    auto d_out = [&]() { if (lane == 0) { atomicMax(&bk_dbg[9], (unsigned long long)d_ev); atomicMax(&bk_dbg[15], (unsigned long long)d_ser); atomicMax(&bk_dbg[5], (unsigned long long)d_bs); atomicMax(&bk_dbg[0], d_t); } };
#endif
    grp_ld cur = load(0), nxt = load(64);
    while (b0 < ZS_TP_NB) {
        const uint32_t cnt = lane >= l0 ? cur.cnt : 0u, meta = cur.meta;
        const bool special = cnt && ((int)(meta & TP_M_EG) != eg || (meta & TP_M_TIE0));
        // totals on the grid, saturated: a group is only added whole while the
        // sum stays below the binade end
        const uint32_t inc = (cnt && !special) ? (uint32_t)min(cur.tot, (unsigned long long)ZS_INC_CAP) : 0u;
        const uint32_t incl = sm_wave_scan_sat(inc);
        const unsigned long long lim = min((unsigned long long)ZS_BINADE, (unsigned long long)kthr);
        const unsigned long long hm = __ballot(cnt && (special || k + incl >= lim));
        if (!hm) {
            k += (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
            b0 += 64;
            l0 = 0;
            cur = nxt;
            nxt = load(b0 + 64);
            continue;
        }
        const uint32_t f = (uint32_t)__ffsll((long long)hm) - 1u;
        k += f ? (uint32_t)__builtin_amdgcn_readlane((int)incl, (int)f - 1) : 0u;
        const uint32_t n = __shfl(cnt, (int)f, 64), bm = __shfl(meta, (int)f, 64);
        const uint32_t st0 = __shfl(cur.start, (int)f, 64);
        l0 = f + 1;
        if (l0 == 64) {
            b0 += 64;
            l0 = 0;
            cur = nxt;
            nxt = load(b0 + 64);
        }
        if (!(bm & TP_M_SORTED)) {
            return 0;
        }
#ifdef ZS_WALK_DEBUG
        d_ev++;
        const unsigned long long d_t0 = wall_clock64();
        if (n > TP_SERIAL_N) d_bs++;
#endif
        // the bucket in exact descending order, from the exact sum k * grid
        uint32_t pos = 0;
        bool done = false, stop = false;
        uint32_t at = 0;
        const int G0 = (int)(bm & TP_M_EG);
        if (n > TP_SERIAL_N && eg == G0) {
            const uint32_t* P = ((k & 1ull) ? po : pe) + st0;
            const unsigned long long lm = min((unsigned long long)ZS_BINADE, (unsigned long long)kthr);
            const uint32_t i = tp_first(0u, n, [&](uint32_t j) { return k + P[j] >= lm; });
            if (i == n) {
                k += P[n - 1];
                done = true;
            } else if (k + P[i] < ZS_BINADE) {
                stop = true;
                at = i;
            } else {
                const unsigned long long prev = k + (i ? P[i - 1] : 0u);
                const float ns = zs_grid_value((uint32_t)prev, eg) + zs_u2f(gv[st0 + i]);
                if (ns >= top_p) { stop = true; at = i; }
                else { set_sum(ns); pos = i + 1; }
            }
        }
        if (!done && !stop && n > TP_SERIAL_N && pos < n && eg == G0 + 1 && !(bm & TP_M_TIE1) &&
            q1[st0 + n - 1] < ZS_INC_CAP) {
            const uint32_t base = pos ? q1[st0 + pos - 1] : 0u;
            const unsigned long long lm = min((unsigned long long)ZS_BINADE, (unsigned long long)kthr);
            const uint32_t j = tp_first(pos, n, [&](uint32_t jj) { return k + (q1[st0 + jj] - base) >= lm; });
            if (j == n) {
                k += q1[st0 + n - 1] - base;
                done = true;
            } else if (k + (q1[st0 + j] - base) < ZS_BINADE) {
                stop = true;
                at = j;
            } else {
                const unsigned long long prev = k + (j > pos ? q1[st0 + j - 1] - base : 0u);
                const float ns = zs_grid_value((uint32_t)prev, eg) + zs_u2f(gv[st0 + j]);
                if (ns >= top_p) { stop = true; at = j; }
                else { set_sum(ns); pos = j + 1; }
            }
        }
        if (!done && !stop) {
            // one addition at a time (sampler.rs:103) over LDS copies of the
            // bucket's values, TP_CH at a time: the wave loads a chunk with all
            // its loads in flight, then every lane adds the same values in
            // order (broadcast reads). The values are positive: the running
            // sum never decreases, so one test per 4 values finds whether it
            // reached top_p among them.
            float ss = zs_grid_value((uint32_t)k, eg);
            const uint32_t* src = gv + st0;
#ifdef ZS_WALK_DEBUG
            d_ser += n - pos;
#endif
            for (uint32_t c0 = pos; c0 < n && !stop; c0 += TP_CH) {
                const uint32_t m = min((uint32_t)TP_CH, n - c0);
                uint32_t w[TP_CH / 64];
#pragma unroll
                for (int q = 0; q < TP_CH / 64; q++) {
                    const uint32_t i = lane + 64u * (uint32_t)q;
                    w[q] = i < m ? src[c0 + i] : 0u;
                }
#pragma unroll
                for (int q = 0; q < TP_CH / 64; q++) lbuf[lane + 64u * (uint32_t)q] = zs_u2f(w[q]);
                __builtin_amdgcn_s_waitcnt(0);
                __builtin_amdgcn_wave_barrier();
                // 32 values per batch of LDS reads (their latency off the
                // chain of additions; the zeros past m add nothing to the
                // positive sum); the batch that reaches top_p is added again
                // 4 values at a time to find the value
                static_assert(TP_CH % 32 == 0, "whole batches inside a chunk");
                for (uint32_t i0 = 0; i0 < m && !stop; i0 += 32) {
                    float4 q8[8];
#pragma unroll
                    for (int u = 0; u < 8; u++) q8[u] = *reinterpret_cast<const float4*>(lbuf + i0 + 4 * u);
                    float c = ss;
#pragma unroll
                    for (int u = 0; u < 8; u++) c = (((c + q8[u].x) + q8[u].y) + q8[u].z) + q8[u].w;
                    if (c < top_p) {
                        ss = c;
                        continue;
                    }
                    for (uint32_t i = i0; i < i0 + 32; i += 4) {
                        const float4 q4 = *reinterpret_cast<const float4*>(lbuf + i);
                        const float c1 = ss + q4.x, c2 = c1 + q4.y, c3 = c2 + q4.z, c4 = c3 + q4.w;
                        if (c4 >= top_p) {
                            const uint32_t e0 = c1 >= top_p ? 0u : c2 >= top_p ? 1u : c3 >= top_p ? 2u : 3u;
                            stop = true;
                            at = c0 + i + e0;
                            ss = e0 == 0 ? c1 : e0 == 1 ? c2 : e0 == 2 ? c3 : c4;
                            break;
                        }
                        ss = c4;
                    }
                }
                __builtin_amdgcn_wave_barrier();
            }
            if (!stop) set_sum(ss);
        }
#ifdef ZS_WALK_DEBUG
        d_t += wall_clock64() - d_t0;
        if (stop) d_out();
#endif
        if (stop) {
            const uint32_t vs = gv[st0 + at];
            const uint32_t first = tp_first(0u, at + 1, [&](uint32_t j) { return gv[st0 + j] <= vs; });
            wo->stopped = true;
            wo->v = vs;
            wo->rank = at - first;
            return 1;
        }
    }
    return 2;
}


__global__ __launch_bounds__(ZS_BIG_NT) void zs_k_big(zs_sargs a) {
    const uint32_t r = blockIdx.x;
    zs_row_state stt = a.rst[r];
    const bool run_samp = stt.mode == ZS_MODE_BIG;
    if (!run_samp) return;
#ifdef ZS_WALK_DEBUG
    unsigned long long bk_t0 = wall_clock64();
    const unsigned long long bk_start = bk_t0;
    if (threadIdx.x == 0) atomicAdd(&bk_dbg[6], 1ull);
#endif
    __shared__ big_shared sh;
    const int t = threadIdx.x;
    const zs_batch& b = a.b;
    const zs_row_params P = b.d_params[r];
    big_row R;
    R.row = b.d_logits + (size_t)r * b.ld;
    R.masked = (P.flags & ZS_ROW_MASKED) && b.d_allow_bits;
    R.allow = R.masked ? b.d_allow_bits + (size_t)r * b.allow_words : nullptr;
    R.pid = a.p_id + (size_t)r * a.pstride;
    R.pfl = a.p_flags + (size_t)r * a.pstride;
    R.py = a.p_y + (size_t)r * a.pstride;
    R.psub = a.p_sub + (size_t)r * (a.max_subs + 1);
    R.nsub = (b.V + ZS_SUB - 1) / ZS_SUB;
    R.V = b.V;
    R.T = P.temperature;
    const uint32_t V = b.V;
    const uint32_t ng = (V + ZS_BIG_G - 1) / ZS_BIG_G;
    const float m = stt.z_max;
    uint32_t* pv = a.pv + (size_t)r * a.max_vocab;

    // ---- top-k threshold by radix select when the candidates could not give it
    uint32_t has_thr = stt.has_thr;
    uint32_t thr_key = stt.thr_key;
    if (has_thr == 2) {
        uint32_t prefix = 0, mask = 0, need = P.top_k;
        for (int shift = 24; shift >= 0; shift -= 8) {
            for (int i = t; i < 256; i += ZS_BIG_NT) sh.hist[i] = 0;
            __syncthreads();
            for (uint32_t g = 0; g < ng; g++) {
                float z[4];
                big_load_z(R, g, z, sh);
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    if (g * ZS_BIG_G + 4 * t + q >= V) continue;
                    uint32_t k = zs_total_key(z[q]);
                    if ((k & mask) == prefix) atomicAdd(&sh.hist[(k >> shift) & 255u], 1u);
                }
            }
            __syncthreads();
            if (t < 64) {
                uint32_t c[4], loc = 0;
                for (int q = 0; q < 4; q++) { c[q] = sh.hist[255 - 4 * t - q]; loc += c[q]; }
                uint32_t inc = wave_incl_scan_u(loc);
                uint32_t before = inc - loc;
                for (int q = 0; q < 4; q++) {
                    if (before < need && need <= before + c[q]) { sh.u[0] = 255 - 4 * t - q; sh.u[1] = need - before; }
                    before += c[q];
                }
            }
            __syncthreads();
            prefix |= sh.u[0] << shift;
            mask |= 0xffu << shift;
            need = sh.u[1];
            __syncthreads();
        }
        thr_key = prefix;
        has_thr = 1;
    }
    BK_T(0);
    const bool use_thr = has_thr != 0;
    const float thr = zs_key_to_float(thr_key);

    // ---- softmax denominator: from the parallel rounds, else summed here
    float S = stt.samp_S;
    if (!((stt.rounds >> ZS_SUM_SAMP_S) & 1u)) {
        S = -0.0f;
        for (uint32_t g = 0; g < ng; g++) {
            float x[4], z[4];
            big_load2(R, g, x, z, sh);
            exp_terms<4> f;
#pragma unroll
            for (int q = 0; q < 4; q++) f.set(q, (use_thr && z[q] < thr) ? -INFINITY : z[q] - m);
            seq_group_f<ZS_BIG_NT, 4>(f, 0, S, NAN, sh.q);
        }
    }

    BK_T(1);
    // ---- probabilities p = exp(z - max) / S (sampler.rs:69), kept in pv for
    // the later passes; min-p kept mass (sampler.rs:72-88) in the same pass
    const bool minp = P.min_p > 0.0f;
    const float cut = minp ? P.min_p * (1.0f / S) : 0.0f;  // p_max: the max element has exp(0) = 1
    float kept = 0.0f;
    if (big_s_from_rounds(stt)) {
        // pv was filled by zs_k_pv; min-p needs the kept mass
        if (minp) {
            for (uint32_t g = 0; g < ng; g++) {
                const uint32_t idx0 = g * ZS_BIG_G + 4 * t;
                uint4 v = idx0 < V ? *reinterpret_cast<const uint4*>(pv + idx0) : make_uint4(0u, 0u, 0u, 0u);
                float tv[4] = {zs_u2f(v.x), zs_u2f(v.y), zs_u2f(v.z), zs_u2f(v.w)};
#pragma unroll
                for (int q = 0; q < 4; q++) tv[q] = (tv[q] < cut) ? 0.0f : tv[q];
                seq_group<ZS_BIG_NT, 4>(tv, 0, kept, NAN, sh.q);
            }
        }
    } else big_stream_z(R, ng, [&](uint32_t g, const float (&z)[4]) {
        float tv[4];
        const uint32_t idx0 = g * ZS_BIG_G + 4 * t;
        uint4 o;
        uint32_t* ob = reinterpret_cast<uint32_t*>(&o);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float p = idx0 + q < V ? big_term_e(z[q], use_thr, thr, m) / S : 0.0f;
            ob[q] = zs_f2u(p);
            tv[q] = (p < cut) ? 0.0f : p;
        }
        if (idx0 < V) *reinterpret_cast<uint4*>(pv + idx0) = o;
        if (minp) seq_group<ZS_BIG_NT, 4>(tv, 0, kept, NAN, sh.q);
        return false;
    });
    __threadfence_block();
    __syncthreads();
    auto p1_of = [&](uint32_t pb) -> float {
        float p = zs_u2f(pb);
        if (minp) {
            if (p < cut) p = 0.0f;
            else if (kept > 0.0f) p = p / kept;
        }
        return p;
    };
    // f(g, p1[4]) for every group in order, BK_U groups of loads in flight;
    // elements past V read 0 (pv holds 0 there); f returns true to stop
    auto stream_p1 = [&](auto&& f) {
        for (uint32_t g0 = 0; g0 < ng; g0 += BK_U) {
            uint4 v[BK_U];
#pragma unroll
            for (int u = 0; u < BK_U; u++) {
                const uint32_t idx0 = (g0 + u) * ZS_BIG_G + 4 * t;
                v[u] = (g0 + u < ng && idx0 < V) ? *reinterpret_cast<const uint4*>(pv + idx0) : make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int u = 0; u < BK_U; u++) {
                if (g0 + u >= ng) break;
                float p[4] = {p1_of(v[u].x), p1_of(v[u].y), p1_of(v[u].z), p1_of(v[u].w)};
                if (f(g0 + u, p)) return;
            }
        }
    };

    BK_T(2);
    // ---- top-p (sampler.rs:91-115)
    const bool topp = P.top_p < 1.0f && P.top_p > 0.0f;
    if (topp) {
        uint32_t* gv = a.pairs + (size_t)r * a.max_vocab * 2;  // level-0 layout
        uint32_t* tmp = gv + a.max_vocab;                       // level-1 refinement
        // The largest probability is p1 of exp(0) / S. When it reaches top_p
        // alone, the walk stops at the first element of the sorted order: the
        // lowest index holding that value.
        const uint32_t pmax1 = zs_f2u(p1_of(zs_f2u(1.0f / S)));
        const bool peak = zs_u2f(pmax1) >= P.top_p;
        // the walk on bucket totals (one wave) when zs_k_tp_* prepared it
        walk_out wo = {false, 0u, 0u};
        int fw = 0;
        if (!peak && (a.tp_cl[(size_t)r * ZS_TP_CL] & TP_ROW_FAST)) {
            if (t < 64) {
                walk_out w = {false, 0u, 0u};
                const int res = tp_walk(a, r, P.top_p, &w, reinterpret_cast<float*>(sh.sortbuf));

                if (t == 0) { sh.u[0] = (uint32_t)res; sh.u[1] = w.v; sh.u[2] = w.rank; }
            }
            __syncthreads();
            fw = (int)sh.u[0];
            wo = {fw == 1, sh.u[1], sh.u[2]};
            __syncthreads();
        }
        BK_T(3);
        if (fw == 0) {
#ifdef ZS_WALK_DEBUG
        if (threadIdx.x == 0) atomicAdd(&bk_dbg[7], 1ull);
#endif
        // counts per (rank, copy): 16 copies by lane keep same-address LDS
        // atomics (skewed histograms) at most 4-way
        uint32_t* cc = sh.sortbuf;
        for (int i = t; i < BK_NB * BK_NC; i += ZS_BIG_NT) cc[i] = 0;
        __syncthreads();
        const uint32_t cp = (uint32_t)t & (BK_NC - 1);
        if (!peak)
            stream_p1([&](uint32_t, const float (&p)[4]) {
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (p[q] > 0.0f) atomicAdd(&cc[bk_rank<0>(zs_f2u(p[q])) * BK_NC + cp], 1u);
                return false;
            });
        __syncthreads();
        // bucket starts by rank and the first candidate range: the ranks whose
        // guaranteed mass (count * bucket floor) reaches 1.02 * top_p
        static_assert(BK_NB == 2 * ZS_BIG_NT, "two ranks per thread");
        if (!peak) {
            uint32_t c2[2];
            double m2[2];
#pragma unroll
            for (int k2 = 0; k2 < 2; k2++) {
                const int rk = 2 * t + k2;
                uint32_t c = 0;
#pragma unroll
                for (int k = 0; k < BK_NC; k++) c += cc[rk * BK_NC + k];
                c2[k2] = c;
                m2[k2] = (double)c * (double)zs_u2f((uint32_t)(BK_NB - 1 - rk) << 19);
            }
            uint32_t ctot;
            double mtot;
            const uint32_t cex = block_excl_scan_u<ZS_BIG_NT>(c2[0] + c2[1], sh.hist2, &ctot);
            const double mex = block_excl_scan_d<ZS_BIG_NT>(m2[0] + m2[1], reinterpret_cast<double*>(sh.hist2), &mtot);
            sh.hist[2 * t] = cex;
            sh.hist[2 * t + 1] = cex + c2[0];
            if (t == 0) sh.hist[BK_NB] = ctot;
            const double lim = 1.02 * (double)P.top_p;
            int cand = ZS_BIGI;
            if (mex + m2[0] >= lim) cand = 2 * t;
            else if (mex + m2[0] + m2[1] >= lim) cand = 2 * t + 1;
            cand = block_min_i<ZS_BIG_NT>(cand, reinterpret_cast<int*>(sh.hist2));
            if (t == 0) sh.u[0] = cand == ZS_BIGI ? (uint32_t)(BK_NB - 1) : (uint32_t)cand;
        }
        __syncthreads();
        const uint32_t rlim = sh.u[0];
        float s = 0.0f;
        uint32_t done = 0;  // walked prefix of the level-0 layout
        for (int round = 0; round < 2 && !wo.stopped && !peak; round++) {
            const uint32_t rlo = round == 0 ? 0u : rlim + 1, rhi = round == 0 ? rlim : BK_NB - 1;
            if (rlo > rhi) break;
            // per (rank, copy) counts of the ranks gathered now (round 0 has
            // them from the histogram), turned into cursors inside each bucket
            uint32_t* cur = sh.sortbuf;
            if (round > 0) {
                for (int i = t; i < BK_NB * BK_NC; i += ZS_BIG_NT) cur[i] = 0;
                __syncthreads();
                stream_p1([&](uint32_t, const float (&p)[4]) {
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        const uint32_t rk = bk_rank<0>(zs_f2u(p[q]));
                        if (p[q] > 0.0f && rk >= rlo && rk <= rhi) atomicAdd(&cur[rk * BK_NC + cp], 1u);
                    }
                    return false;
                });
                __syncthreads();
            }
            for (uint32_t i = rlo + t; i <= rhi; i += ZS_BIG_NT) {
                uint32_t acc = sh.hist[i];
#pragma unroll
                for (int k = 0; k < BK_NC; k++) { uint32_t c = cur[i * BK_NC + k]; cur[i * BK_NC + k] = acc; acc += c; }
            }
            __syncthreads();
            stream_p1([&](uint32_t, const float (&p)[4]) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t pb = zs_f2u(p[q]);
                    const uint32_t rk = bk_rank<0>(pb);
                    if (p[q] > 0.0f && rk >= rlo && rk <= rhi) gv[atomicAdd(&cur[rk * BK_NC + cp], 1u)] = pb;
                }
                return false;
            });
            __threadfence_block();
            __syncthreads();
            const uint32_t upto = sh.hist[rhi + 1];
            wo = bk_walk<0>(gv, done, upto, sh.hist, s, P.top_p, tmp, sh);
            done = upto;
        }
        }  // fw == 0
        BK_T(4);
#ifdef ZS_WALK_DEBUG
        if (threadIdx.x == 0) atomicMax(&bk_dbg[8], wall_clock64() - bk_start);
#endif
        if (peak) wo = {true, pmax1, 0u};
        if (wo.stopped) {
            // The kept set is {p1 > v*} plus the first rank+1 elements equal to
            // v* in index order (the sort is stable); zs_k_kcount / zs_k_kwrite
            // compact {p1 >= v*} in index order over all CUs, and sum2 and the
            // draw run as rounds over that list.
            if (t == 0) {
                zs_row_state& o = a.rst[r];
                o.vstar = wo.v;
                o.krank = wo.rank;
                o.istar = 0xffffffffu;
                o.kminp = minp ? 1u : 0u;
                o.kcut = cut;
                o.kkept = kept;
                o.kpend = 1;
                o.knorm = 1;
            }
            return;
        }
    }
    BK_T(5);
    // ---- every positive p1 kept (no top-p, or a walk that never stopped): the
    // kept list is every positive p1 in index order (v* = 0: no value equals
    // it), with sum2 and the renormalised draw after a top-p walk, else the
    // draw on p1 itself (sampler.rs:118-127), as rounds over all CUs
    if (t == 0) {
        zs_row_state& o = a.rst[r];
        o.vstar = 0u;
        o.krank = 0u;
        o.istar = 0xffffffffu;
        o.kminp = minp ? 1u : 0u;
        o.kcut = cut;
        o.kkept = kept;
        o.kpend = 1;
        o.kident = minp ? 0u : 1u;
        o.knorm = topp ? 1u : 0u;
    }
}

// ===========================================================================
// Compaction of the kept set {p1 >= v*} in index order (every big row that
// reaches the draw; v* = 0 keeps every positive p1), over all CUs: zs_k_kcount counts per 4096-id group the values above
// and equal to v*; zs_k_kwrite places each group's elements after the groups
// before it, finds i* (the (rank+1)-th element equal to v*) and adds the
// approximate sums of the kept list per 1024-entry sub-chunk (the predictions
// of the kept-list rounds).
// ===========================================================================
__device__ __forceinline__ float kc_p1(const zs_row_state& st, uint32_t pb) {
    float p = zs_u2f(pb);
    if (st.kminp) {
        if (p < st.kcut) p = 0.0f;
        else if (st.kkept > 0.0f) p = p / st.kkept;
    }
    return p;
}

// (256-thread workgroups as zs_k_pv; so is zs_k_kwrite)
__global__ __launch_bounds__(PV_NT) void zs_k_kcount(zs_sargs a) {
    const uint32_t g = blockIdx.x, r = blockIdx.y;
    zs_row_state& st = a.rst[r];
    if (!st.kpend) return;
    const uint32_t t = threadIdx.x, V = a.b.V;
    const uint32_t vs = st.vstar;
    constexpr int NS = ZS_BIG_NT / PV_NT;
    uint4 v[NS];
#pragma unroll
    for (int u = 0; u < NS; u++) {
        const uint32_t idx0 = g * ZS_BIG_G + 4 * (t + u * PV_NT);
        v[u] = idx0 < V ? *reinterpret_cast<const uint4*>(a.pv + (size_t)r * a.max_vocab + idx0) : make_uint4(0u, 0u, 0u, 0u);
    }
    if (st.kident) {
        // the list is the row's p itself: its approximate sum per sub-chunk
        // (slot u of the threads holds sub-chunk u of the group)
        static_assert(ZS_BIG_G / ZS_SUB == NS && 4 * PV_NT == ZS_SUB, "slot u = sub-chunk u of the group");
        __shared__ double ssum[NS][PV_NT / 64];
#pragma unroll
        for (int u = 0; u < NS; u++) {
            const double d = wave_sum_d((double)zs_u2f(v[u].x) + (double)zs_u2f(v[u].y) + (double)zs_u2f(v[u].z) +
                                        (double)zs_u2f(v[u].w));
            if (zs_lane() == 0) ssum[u][zs_wid()] = d;
        }
        __syncthreads();
        const uint32_t sub = g * NS + t;
        if (t < NS && sub < (V + ZS_SUB - 1) / ZS_SUB)
            a.k_ap[(size_t)r * a.max_subs + sub] = ssum[t][0] + ssum[t][1] + ssum[t][2] + ssum[t][3];
        if (g == 0 && t == 0) {
            st.nk = V;
            st.klist = 1;
        }
        return;
    }
    uint32_t c = 0;  // (above << 16) | equal
#pragma unroll
    for (int u = 0; u < NS; u++) {
        const uint32_t pb[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float p = kc_p1(st, pb[q]);
            const uint32_t b = zs_f2u(p);
            if (p > 0.0f && b >= vs) c += b > vs ? 0x10000u : 1u;
        }
    }
    __shared__ uint32_t sh[PV_NT / 64];
    c = wave_sum_u(c);
    if (zs_lane() == 0) sh[zs_wid()] = c;
    __syncthreads();
    if (t == 0) {
        uint32_t tot = 0;
        for (int i = 0; i < PV_NT / 64; i++) tot += sh[i];
        a.kcnt[(size_t)r * a.nch * 2 + g] = tot;
    }
    // the kept-list sub-chunk sums are added by zs_k_kwrite
    if (t < ZS_BIG_G / ZS_SUB) a.k_ap[(size_t)r * a.max_subs + g * (ZS_BIG_G / ZS_SUB) + t] = 0.0;
}

__global__ __launch_bounds__(PV_NT) void zs_k_kwrite(zs_sargs a) {
    const uint32_t g = blockIdx.x, r = blockIdx.y;
    zs_row_state& st = a.rst[r];
    if (!st.kpend || st.kident) return;
    const uint32_t t = threadIdx.x, V = a.b.V;
    const uint32_t ng = (V + ZS_BIG_G - 1) / ZS_BIG_G;
    __shared__ uint32_t sh[PV_NT / 64];
    __shared__ uint32_t base_sh[3];
    __shared__ double lap[ZS_BIG_G / ZS_SUB + 1];
    const uint32_t* kc = a.kcnt + (size_t)r * a.nch * 2;
    if (t < 64) {
        // elements and equal elements before this group, and the totals
        uint32_t pre_all = 0, pre_eq = 0, tot_all = 0;
        for (uint32_t i = t; i < ng; i += 64) {
            const uint32_t c = kc[i];
            const uint32_t n = (c >> 16) + (c & 0xffffu);
            if (i < g) { pre_all += n; pre_eq += c & 0xffffu; }
            tot_all += n;
        }
        pre_all = wave_sum_u(pre_all);
        pre_eq = wave_sum_u(pre_eq);
        tot_all = wave_sum_u(tot_all);
        if (t == 0) { base_sh[0] = pre_all; base_sh[1] = pre_eq; base_sh[2] = tot_all; }
    }
    if (t <= ZS_BIG_G / ZS_SUB) lap[t] = 0.0;
    constexpr int NS = ZS_BIG_NT / PV_NT;
    uint4 v[NS];
#pragma unroll
    for (int u = 0; u < NS; u++) {
        const uint32_t idx0 = g * ZS_BIG_G + 4 * (t + u * PV_NT);
        v[u] = idx0 < V ? *reinterpret_cast<const uint4*>(a.pv + (size_t)r * a.max_vocab + idx0) : make_uint4(0u, 0u, 0u, 0u);
    }
    __syncthreads();
    uint32_t pos = base_sh[0], eq = base_sh[1];
    const uint32_t sub0 = pos / ZS_SUB;
    const uint32_t vs = st.vstar, rank = st.krank;
    uint32_t* kp = a.pairs + (size_t)r * a.max_vocab * 2;
    uint32_t* ki = kp + a.max_vocab;
    // the slots in index order: slot u of every thread, then slot u + 1
#pragma unroll
    for (int u = 0; u < NS; u++) {
        const uint32_t idx0 = g * ZS_BIG_G + 4 * (t + u * PV_NT);
        const uint32_t pb[4] = {v[u].x, v[u].y, v[u].z, v[u].w};
        uint32_t kb[4];
        uint32_t c = 0;  // (kept << 16) | equal
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const float p = kc_p1(st, pb[q]);
            kb[q] = zs_f2u(p);
            if (p > 0.0f && kb[q] >= vs) c += 0x10000u + (kb[q] == vs ? 1u : 0u);
        }
        uint32_t tot;
        const uint32_t ex = block_excl_scan_u<PV_NT>(c, sh, &tot);
        uint32_t ps = pos + (ex >> 16), e = eq + (ex & 0xffffu);
#pragma unroll
        for (int q = 0; q < 4; q++) {
            if (!(zs_u2f(kb[q]) > 0.0f && kb[q] >= vs)) continue;
            const uint32_t idx = idx0 + q;
            kp[ps] = kb[q];
            ki[ps] = idx;
            bool in = true;
            if (kb[q] == vs) {
                if (e == rank) st.istar = idx;
                in = e <= rank;
                e++;
            }
            if (in) atomicAdd(&lap[ps / ZS_SUB - sub0], (double)zs_u2f(kb[q]));
            ps++;
        }
        pos += tot >> 16;
        eq += tot & 0xffffu;
    }
    __syncthreads();
    if (t <= ZS_BIG_G / ZS_SUB && lap[t] != 0.0) atomicAdd(&a.k_ap[(size_t)r * a.max_subs + sub0 + t], lap[t]);
    if (g == 0 && t == 0) {
        st.nk = base_sh[2];
        st.klist = 1;
    }
}

// ===========================================================================
// Kept-list rounds: the sequential sums of the kept set in index order --
// sum2 (sampler.rs:107) and the draw's running sum of p / sum2 (:118-127) --
// spread over the GPU like the row sums above: every 1024-entry sub-chunk of a
// row's kept list adds its increments on the grid predicted from the
// approximate prefix, and one workgroup per row stitches the totals, redoing
// exactly the sub-chunks whose grid was not certain.
// ===========================================================================
struct klist_row {
    const uint32_t* kp;
    const uint32_t* ki;   // (null for a row whose list is its p in index order: entry i is id i)
    uint32_t nk, vstar, istar;
    float inv;  // 0: the kept p themselves (sum2, or the draw without top-p), else p / sum2 (draw)
    float sum2;
};
__device__ __forceinline__ klist_row make_klist(const zs_sargs& a, uint32_t r, const zs_row_state& st, int kind) {
    klist_row L;
    if (st.kident) {
        L.kp = a.pv + (size_t)r * a.max_vocab;
        L.ki = nullptr;
    } else {
        L.kp = a.pairs + (size_t)r * a.max_vocab * 2;
        L.ki = L.kp + a.max_vocab;
    }
    L.nk = st.nk;
    L.vstar = st.vstar;
    L.istar = st.istar;
    L.sum2 = kind && st.knorm ? st.sum2 : 1.0f;
    L.inv = kind && st.knorm ? 1.0f : 0.0f;
    return L;
}
// A wave's 16 terms of sub-chunk j (tv[q]: entry j * ZS_SUB + 64 q + lane),
// every load issued before the first is used. Term i of the list: the kept p
// (0 for the equal values after i*, and past the list), divided by sum2 for
// the draw.
__device__ __forceinline__ void klist_terms16(const klist_row& L, uint32_t j, float (&tv)[ZS_SUB / 64]) {
    // (unconditional loads at an index clamped into the list, L.nk >= 1: a
    // bounds test around each would become a branch that waits for it)
    uint32_t pb[ZS_SUB / 64], id[ZS_SUB / 64];
#pragma unroll
    for (int q = 0; q < ZS_SUB / 64; q++) {
        const uint32_t i = min(j * ZS_SUB + (uint32_t)q * 64u + (uint32_t)zs_lane(), L.nk - 1u);
        pb[q] = L.kp[i];
        id[q] = L.ki ? L.ki[i] : i;
    }
#pragma unroll
    for (int q = 0; q < ZS_SUB / 64; q++) {
        const uint32_t i = j * ZS_SUB + (uint32_t)q * 64u + (uint32_t)zs_lane();
        float p = 0.0f;
        if (i < L.nk && (pb[q] > L.vstar || id[q] <= L.istar)) {
            p = zs_u2f(pb[q]);
            if (L.inv != 0.0f) p = p / L.sum2;
        }
        tv[q] = p;
    }
}

// one wave per (sub-chunk, row): the increment pair of the sub-chunk on the
// grid predicted from the approximate prefix (terms in order: the q-th 64
// entries, lanes in order)
template <int KIND>
__global__ __launch_bounds__(256) void zs_k_roundK(zs_sargs a) {
    const uint32_t r = blockIdx.y;
    const uint32_t j = blockIdx.x * 4 + zs_wid();
    const zs_row_state& st = a.rst[r];
    if (!st.klist || (KIND == 0 && !st.knorm)) return;   // no sum2 without a top-p cut
    const uint32_t nks = (st.nk + ZS_SUB - 1) / ZS_SUB;
    if (j >= nks) return;
    const klist_row L = make_klist(a, r, st, KIND);
    const double* ap = a.k_ap + (size_t)r * a.max_subs;
    // approximate prefix before sub-chunk j and after it
    double pre = 0.0;
    for (uint32_t i = zs_lane(); i < j; i += 64) pre += ap[i];
    pre = wave_sum_d(pre);
    const double scale = KIND ? 1.0 / (double)L.sum2 : 1.0;
    const double lo = pre * scale, hi = (pre + ap[j]) * scale;
    const double delta = 1.0 / 256.0;
    const double lm = lo * (1.0 - delta), hm = hi * (1.0 + delta);
    sm_rec e = {0, 0u, 0u, 0u};
    float tv[ZS_SUB / 64];
    klist_terms16(L, j, tv);
    if (j == 0) {
        // sub-chunk 0 from the sum's start value, term by term (with the
        // draw's stop threshold, the uniform zs_k_stitchK compares with)
        __shared__ float k0buf[ZS_SUB];
#pragma unroll
        for (int q = 0; q < ZS_SUB / 64; q++) k0buf[q * 64 + zs_lane()] = tv[q];
        __builtin_amdgcn_s_waitcnt(0);
        __builtin_amdgcn_wave_barrier();
        const float thr = KIND == 1 ? zs_philox_uniform(a.b.d_seed[r], a.b.d_counter[r], 0u) : NAN;
        uint32_t sp;
        const float s0 = sm_serial(k0buf, ZS_SUB, KIND ? 0.0f : -0.0f, thr, &sp);
        if (zs_lane() == 0)
            reinterpret_cast<sm_rec*>(a.k_sum)[((size_t)r * 2 + KIND) * a.max_subs] = sm_rec{0, SM_EXACT, __float_as_uint(s0), sp};
        return;
    }
    // a sub-chunk where the sum surely starts in one binade and ends in the
    // next: its crossing record (zs_walk.h's sm_xrec), the exit term guessed
    // from the approximate start
    // (SM_ALT, the start estimate within the margin of the next binade: the
    // pair of all the terms on the next grid as well)
    const int bl = lm > 0x1p-99 ? ilogb(lm) : 0, bs = lm > 0x1p-99 ? ilogb(lo * (1.0 + delta)) : 0;
    if (j != 0 && lm > 0x1p-99 && hm < 0x1p100 && (bs == bl || bs == bl + 1) && ilogb(hm) == bl + 1) {
        const int eg = bl + 127;
        const bool alt = bs == bl + 1;
        const float sc = sm_scale(eg), sc2 = sm_scale(eg + 1);
        uint32_t carry = min((uint32_t)ldexp(lo, 150 - eg), ZS_BINADE - 1u), xpos = 0xffffffffu;
        seq_pair pre = {0u, 0u}, post = {0u, 0u}, all2 = {0u, 0u};
        float vx = 0.0f;
#pragma unroll
        for (int q = 0; q < ZS_SUB / 64; q++) {
            const float v = tv[q];
            const uint32_t pos = (uint32_t)q * 64u + (uint32_t)zs_lane();
            if (xpos == 0xffffffffu) {
                const float qv = fminf(v * sc, SM_QCAP);
                float rq = rintf(qv);
                const bool h = fabsf(qv - rq) == 0.5f;
                if (h) rq = floorf(qv);
                const uint32_t inc = (uint32_t)rq;
                const uint32_t incl = sm_wave_scan_sat(inc);
                const unsigned long long m = __ballot(zs_sat_add(carry, incl) >= ZS_BINADE);
                bool before = true;
                if (m) {
                    const int Lx = __ffsll((long long)m) - 1;
                    xpos = (uint32_t)q * 64u + (uint32_t)Lx;
                    vx = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(v), Lx));
                    before = pos < xpos;
                }
                const uint32_t ti = before ? inc : 0u;
                if (!__builtin_amdgcn_readfirstlane((int)(__ballot(h && before) != 0ull))) {
                    const uint32_t t = sm_wave_sum_sat(ti);
                    pre = seq_compose(pre, seq_pair{t, t});
                } else {
                    pre = seq_compose(pre, sm_wave_pair_reduce(!before ? seq_pair{0u, 0u}
                                                               : h ? sm_pair_tie(inc) : seq_pair{inc, inc}));
                }
                carry = zs_sat_add(carry, (uint32_t)__builtin_amdgcn_readlane((int)incl, 63));
            }
            if (xpos != 0xffffffffu || alt) {
                const float qv = fminf(v * sc2, SM_QCAP);
                float rq = rintf(qv);
                const bool hh = fabsf(qv - rq) == 0.5f;
                if (hh) rq = floorf(qv);
                const uint32_t inc2 = (uint32_t)rq;
                if (xpos != 0xffffffffu) {
                    const bool after = pos > xpos;
                    const bool h = hh && after;
                    const uint32_t inc = after ? inc2 : 0u;
                    if (!__builtin_amdgcn_readfirstlane((int)(__ballot(h) != 0ull))) {
                        const uint32_t t = sm_wave_sum_sat(inc);
                        post = seq_compose(post, seq_pair{t, t});
                    } else {
                        post = seq_compose(post, sm_wave_pair_reduce(h ? sm_pair_tie(inc) : seq_pair{inc, inc}));
                    }
                }
                if (alt) {
                    if (!__builtin_amdgcn_readfirstlane((int)(__ballot(hh) != 0ull))) {
                        const uint32_t t = sm_wave_sum_sat(inc2);
                        all2 = seq_compose(all2, seq_pair{t, t});
                    } else {
                        all2 = seq_compose(all2, sm_wave_pair_reduce(hh ? sm_pair_tie(inc2) : seq_pair{inc2, inc2}));
                    }
                }
            }
        }
        const uint32_t fl = (xpos != 0xffffffffu ? SM_CROSS : 0u) | (alt ? SM_ALT : 0u);
        if (fl) {
            e = sm_rec{eg, fl, pre.e, pre.o};
            if (zs_lane() == 0)
                reinterpret_cast<sm_xrec*>(a.k_xsum)[((size_t)r * 2 + KIND) * a.max_subs + j] =
                    sm_xrec{xpos, vx, post.e, post.o, all2.e, all2.o};
        }
    } else if (j != 0 && lm > 0x1p-99 && hm < 0x1p100 && ilogb(lm) == ilogb(hm)) {
        e.eg = ilogb(lm) + 127;
        const float sc = sm_scale(e.eg);
        uint32_t inc[ZS_SUB / 64], tie = 0u, tot = 0u;
#pragma unroll
        for (int q = 0; q < ZS_SUB / 64; q++) {
            const float qv = fminf(tv[q] * sc, SM_QCAP);
            float rq = rintf(qv);
            if (fabsf(qv - rq) == 0.5f) {
                tie |= 1u << q;
                rq = floorf(qv);
            }
            inc[q] = (uint32_t)rq;
            tot = zs_sat_add(tot, inc[q]);
        }
        seq_pair all;
        if (!__builtin_amdgcn_readfirstlane((int)(__ballot(tie != 0u) != 0ull))) {
            const uint32_t t = sm_wave_sum_sat(tot);
            all = seq_pair{t, t};
        } else {
            all = seq_pair{0u, 0u};
#pragma unroll
            for (int q = 0; q < ZS_SUB / 64; q++)
                all = seq_compose(all, sm_wave_pair_reduce(((tie >> q) & 1u) ? sm_pair_tie(inc[q])
                                                                              : seq_pair{inc[q], inc[q]}));
        }
        e.flags = SM_SAFE;
        e.d0 = all.e;
        e.d1 = all.o;
    }
    if (zs_lane() == 0) reinterpret_cast<sm_rec*>(a.k_sum)[((size_t)r * 2 + KIND) * a.max_subs + j] = e;
}

// Kept-list terms for sm_stitch: thread t's 4 consecutive entries.
struct klist_raw {
    uint4 p, i;
};
struct klist_tp {
    const klist_row& L;
    __device__ __forceinline__ uint32_t at(uint32_t j) const {
        return min(j * ZS_SUB + SW_TPT * threadIdx.x, (L.nk - 1u) & ~3u);
    }
    __device__ __forceinline__ void fetch(uint32_t j, klist_raw& raw) const {
        const uint32_t i = at(j);
        raw.p = *reinterpret_cast<const uint4*>(L.kp + i);
        raw.i = L.ki ? *reinterpret_cast<const uint4*>(L.ki + i) : make_uint4(i, i + 1u, i + 2u, i + 3u);
    }
    __device__ __forceinline__ void take(uint32_t j, const klist_raw& raw, float (&v)[SW_TPT]) const {
        const uint32_t i0 = j * ZS_SUB + SW_TPT * threadIdx.x;
        const uint32_t pb[4] = {raw.p.x, raw.p.y, raw.p.z, raw.p.w}, id[4] = {raw.i.x, raw.i.y, raw.i.z, raw.i.w};
#pragma unroll
        for (int e = 0; e < SW_TPT; e++) {
            float p = 0.0f;
            if (i0 + e < L.nk && (pb[e] > L.vstar || id[e] <= L.istar)) {
                p = zs_u2f(pb[e]);
                if (L.inv != 0.0f) p = p / L.sum2;
            }
            v[e] = p;
        }
    }
    __device__ __forceinline__ void direct(uint32_t j, float (&v)[SW_TPT]) const {
        klist_raw raw;
        fetch(j, raw);
        take(j, raw, v);
    }
};

// one workgroup per row: sum2 (KIND 0), or the draw (KIND 1) -- the first
// entry after which the running sum reaches the uniform (zs_walk.h)
template <int KIND>
__global__ __launch_bounds__(SW_NT) void zs_k_stitchK(zs_sargs a) {
    const uint32_t r = blockIdx.x;
    zs_row_state* stp = a.rst + r;
    if (!stp->klist || (KIND == 0 && !stp->knorm)) return;
    [[maybe_unused]] const unsigned long long k0 = SW_CLK();
    const zs_row_state st = *stp;
    const klist_row L = make_klist(a, r, st, KIND);
    const uint32_t nks = (L.nk + ZS_SUB - 1) / ZS_SUB;
    const sm_rec* ks = reinterpret_cast<const sm_rec*>(a.k_sum) + ((size_t)r * 2 + KIND) * a.max_subs;
    const sm_xrec* kx = reinterpret_cast<const sm_xrec*>(a.k_xsum) + ((size_t)r * 2 + KIND) * a.max_subs;
    for (uint32_t j = threadIdx.x; j < nks; j += SW_NT) {
        const sm_rec e = ks[j];
        sm_sh.rec[j] = e;
        if (e.flags & (SM_CROSS | SM_ALT)) sm_sh.xrec[j] = kx[j];
    }
    __syncthreads();
    float thresh = NAN;
    if (KIND == 1) {
        const float rr = zs_philox_uniform(a.b.d_seed[r], a.b.d_counter[r], 0u);
        if (rr <= 0.0f) {  // cumsum >= r at id 0 (sampler.rs:118-127)
            if (threadIdx.x == 0) {
                stp->token = 0;
                stp->mode = ZS_MODE_DONE;
            }
            return;
        }
        thresh = rr;
    }
    [[maybe_unused]] const unsigned long long k1 = SW_CLK();
    klist_tp tp{L};
    uint32_t stop;
    const float s = sm_stitch<klist_tp, klist_raw>(tp, nks, KIND ? 0.0f : -0.0f, thresh, &stop);
    SW_K(KIND, SW_CLK() - k0, k1 - k0);
    if (threadIdx.x == 0) {
        if (KIND == 0) {
            stp->sum2 = s;
        } else {
            stp->token = stop != 0xffffffffu ? (L.ki ? L.ki[stop] : stop) : a.b.V - 1;
            stp->mode = ZS_MODE_DONE;
        }
    }
}

// ===========================================================================
// zs_k_final: per-row outputs (logprobs.rs:34-54, hallucination.rs:129-154)
// ===========================================================================
__global__ __launch_bounds__(64) void zs_k_final(zs_sargs a) {
    // one wave per row; lane j handles observer candidate j
    const uint32_t r = blockIdx.x;
    const uint32_t lane = threadIdx.x;
    const zs_batch& b = a.b;
    if (r >= b.B) return;
    const zs_row_state& st = a.rst[r];
    const uint32_t tok = st.token;
    uint32_t status = st.status;
    const zs_row_params P = b.d_params[r];
    const bool want_lp = (P.flags & ZS_ROW_LOGPROBS) != 0;
    const bool want_unc = (P.flags & ZS_ROW_UNCERTAINTY) != 0;
    if (lane == 0) {
        b.d_token[r] = tok;
        b.d_top_n[r] = 0;
        b.d_logprob[r] = NAN;
        b.d_entropy[r] = NAN;
        b.d_max_prob[r] = NAN;
        b.d_margin[r] = NAN;
        b.d_chosen_lp[r] = NAN;
    }
    if (status & ZS_ST_LIMIT) {
        if (lane == 0) b.d_status[r] = status;
        return;
    }
    // x~ of the chosen token: the logit, the mask bit and a ban among the
    // patches of its 1024-id sub-chunk (lanes check them in parallel)
    float xc = -INFINITY;
    const bool in_range = tok < b.V;
    if (in_range) {
        xc = b.d_logits[(size_t)r * b.ld + tok];
        if ((P.flags & ZS_ROW_MASKED) && b.d_allow_bits && !zs_allowed_bit(b, r, tok)) xc = -INFINITY;
        const uint32_t* pid = a.p_id + (size_t)r * a.pstride;
        const uint32_t* psub = a.p_sub + (size_t)r * (a.max_subs + 1);
        const uint32_t nsub = (b.V + ZS_SUB - 1) / ZS_SUB;
        const uint32_t p0 = psub[tok / ZS_SUB], p1 = psub[min(tok / ZS_SUB + 1, nsub)];
        bool ban = false;
        for (uint32_t p = p0 + lane; p < p1; p += 64)
            if (pid[p] == tok && (a.p_flags[(size_t)r * a.pstride + p] & ZS_PF_BAN)) ban = true;
        if (__ballot(ban)) xc = -INFINITY;
    }
    const float M = st.obs_max;
    if (want_lp) {
        uint32_t ntl = P.top_logprobs > 20 ? 20 : P.top_logprobs;
        if (ntl > b.top_stride) ntl = b.top_stride;
        uint32_t* tid = b.d_top_ids + (size_t)r * b.top_stride;
        float* tlp = b.d_top_lps + (size_t)r * b.top_stride;
        if (st.obs_special) {
            // lse is NaN: every lp is NaN and partition_point(x >= NaN) == 0 inserts
            // each entry first, leaving ids n-1 .. 0 (logprobs.rs:41-51)
            const uint32_t n = ntl < b.V ? ntl : b.V;
            for (uint32_t j = lane; j < n; j += 64) { tid[j] = n - 1 - j; tlp[j] = NAN; }
            if (lane == 0) {
                b.d_top_n[r] = n;
                b.d_logprob[r] = in_range ? NAN : -INFINITY;
            }
        } else {
            const float lse = M + (float)log((double)st.obs_S);  // logprobs.rs:36
            if (lane == 0) b.d_logprob[r] = in_range ? xc - lse : -INFINITY;
            // the list the reference keeps by insertion (logprobs.rs:41-51):
            // lp desc, equal lp in id order; rank of candidate j in it
            const uint32_t nc = st.n_cand;
            const bool mine = lane < nc;
            const uint32_t id = mine ? st.cand_id[lane] : 0xffffffffu;
            const float xv = mine ? st.cand_x[lane] : -INFINITY;
            const float lp = xv - lse;
            uint32_t rank = 0;
            for (uint32_t i = 0; i < nc; i++) {
                const float li = zs_readlane_f(lp, i);
                const uint32_t ii = zs_readlane_u(id, i);
                rank += (li > lp || (li == lp && ii < id)) ? 1u : 0u;
            }
            // sorted x~ by rank, for the check below
            __shared__ float xs_sh[64];
            if (mine) xs_sh[rank] = xv;
            __syncthreads();
            // the order must not hinge on the last bit of lse (its logf may differ
            // from glibc's by one ulp)
            const float lo = nextafterf(lse, -INFINITY), hi = nextafterf(lse, INFINITY);
            const uint32_t lim = nc < ntl + 1 ? nc : ntl + 1;
            bool amb = false;
            if (lane + 1 < lim) {
                const float x0 = xs_sh[lane], x1 = xs_sh[lane + 1];
                const bool e0 = (x0 - lse) == (x1 - lse);
                const bool e1 = (x0 - lo) == (x1 - lo);
                const bool e2 = (x0 - hi) == (x1 - hi);
                amb = e0 != e1 || e0 != e2;
            }
            if (__ballot(amb)) status |= ZS_ST_TOPLP_AMBIG;
            const uint32_t n = ntl < nc ? ntl : nc;
            // Distinct x~ can round to one lp. When the list of candidates by
            // (x~ desc, id asc) was cut and its last candidate shares the lp
            // of the n-th entry, ids outside the list may hold that lp too and
            // rank before candidates by id: the entries above that lp are the
            // candidates', the rest are the smallest ids of the whole row at
            // that lp (found in id order by one scan of the row).
            bool fill = false;
            float lpn = -INFINITY;
            if (n > 0 && nc == ZS_OBS_CAND && nc < b.V) {
                const unsigned long long at = __ballot(mine && rank == n - 1);
                lpn = zs_readlane_f(lp, (uint32_t)__ffsll((long long)at) - 1u);
                float lmin = mine ? lp : INFINITY;
                for (int d = 32; d > 0; d >>= 1) lmin = fminf(lmin, __shfl_xor(lmin, d, 64));
                fill = lpn > -INFINITY && lmin == lpn;
            }
            if (!fill) {
                if (mine && rank < n) { tid[rank] = id; tlp[rank] = lp; }
            } else {
                if (mine && lp > lpn) { tid[rank] = id; tlp[rank] = lp; }
                uint32_t got = (uint32_t)__popcll(__ballot(mine && lp > lpn));
                const float* row = b.d_logits + (size_t)r * b.ld;
                const bool masked = (P.flags & ZS_ROW_MASKED) && b.d_allow_bits;
                const uint32_t* pid = a.p_id + (size_t)r * a.pstride;
                const uint32_t* pfl = a.p_flags + (size_t)r * a.pstride;
                const uint32_t* psub = a.p_sub + (size_t)r * (a.max_subs + 1);
                const uint32_t nsub = (b.V + ZS_SUB - 1) / ZS_SUB;
                for (uint32_t i0 = 0; i0 < b.V && got < n; i0 += 64) {
                    const uint32_t i = i0 + lane;
                    bool hit = false;
                    if (i < b.V) {
                        float xv = row[i];
                        if (masked && !zs_allowed_bit(b, r, i)) xv = -INFINITY;
                        hit = (xv - lse) == lpn;
                    }
                    unsigned long long hm = __ballot(hit);
                    while (hm && got < n) {
                        const uint32_t idh = i0 + (uint32_t)__ffsll((long long)hm) - 1u;
                        hm &= hm - 1ull;
                        // a banned id has x~ = -inf (its patches, lanes in parallel)
                        const uint32_t p0 = psub[idh / ZS_SUB], p1 = psub[min(idh / ZS_SUB + 1, nsub)];
                        bool ban = false;
                        for (uint32_t q = p0 + lane; q < p1; q += 64)
                            if (pid[q] == idh && (pfl[q] & ZS_PF_BAN)) ban = true;
                        if (__ballot(ban)) continue;
                        if (lane == 0) { tid[got] = idh; tlp[got] = lpn; }
                        got++;
                    }
                }
            }
            if (lane == 0) b.d_top_n[r] = n;
        }
    }
    if (want_unc && lane == 0) {
        if (st.obs_special) {
            // sum is NaN: no p > 0, top1 stays -inf (hallucination.rs:140-153)
            b.d_entropy[r] = 0.0f;
            b.d_max_prob[r] = 0.0f;
            b.d_margin[r] = 0.0f;
            b.d_chosen_lp[r] = -INFINITY;
        } else {
            const float inv = 1.0f / st.obs_S;
            const float top1 = inv;  // the max element has exp(0) = 1
            float top2 = -INFINITY;
            if (st.n_cand >= 2) top2 = zs_expf(st.cand_x[1] - M) * inv;
            b.d_entropy[r] = fmaxf(st.obs_H, 0.0f);
            b.d_max_prob[r] = fmaxf(top1, 0.0f);
            b.d_margin[r] = fmaxf(top1 - top2, 0.0f);
            float pc = in_range ? zs_expf(xc - M) * inv : 0.0f;
            b.d_chosen_lp[r] = pc > 0.0f ? (float)log((double)pc) : -INFINITY;
        }
    }
    if (lane == 0) b.d_status[r] = status;
}

// ===========================================================================
// host launcher
// ===========================================================================
#define ZS_LAUNCH_CHECK(call)                                                                   \
    do {                                                                                        \
        hipError_t e_ = (call);                                                                 \
        if (e_ != hipSuccess) return zs_set_error(ctx, ZS_EHIP, "zs_sample: %s", hipGetErrorString(e_)); \
    } while (0)

extern "C" int zs_sample_launch(zs_ctx* ctx, const zs_batch* bt, hipStream_t stream) {
    zs_sargs a;
    a.b = *bt;
    a.p_cnt = ctx->p_cnt;
    a.p_id = ctx->p_id;
    a.p_flags = ctx->p_flags;
    a.p_y = ctx->p_y;
    a.rst = ctx->rst;
    a.pairs = ctx->pairs;
    a.nch = ctx->max_chunks;
    a.max_vocab = ctx->max_vocab;
    a.pv = ctx->pv;
    a.p_sub = ctx->p_sub;
    a.max_subs = ctx->max_subs;
    a.k_ap = ctx->k_ap;
    a.k_sum = ctx->k_sum;
    a.k_xsum = ctx->k_sum + (size_t)ctx->max_rows * 2 * ctx->max_subs;
    a.tp_bk = ctx->tp_bk;
    a.tp_cl = ctx->tp_cl;
    a.tp_pre = ctx->tp_pre;
    a.kcnt = ctx->kcnt;
    a.tp_task = ctx->tp_task;
    a.rw_part = ctx->rw_part;
    a.rw_ctr = ctx->rw_ctr;
    // rows split their stream over two workgroups when the batch leaves the
    // second workgroups CUs of their own
    a.row_split = 2 * bt->B <= ctx->num_cus ? 1u : 0u;
    a.s_rec = ctx->s_rec;
    a.s_xrec = ctx->s_rec + (size_t)ctx->max_rows * ZS_NSUM * ctx->max_subs;
    a.s_apx = ctx->s_apx;
    a.gath = ctx->gath;
    a.pstride = ctx->max_vocab;
    a.s_hterm = ctx->s_hterm;
    const uint32_t B = bt->B;
    const bool prof = ctx->profiling != 0;
    int ev = 0;
    auto mark = [&](const char* name) {
        if (!prof) return;
        if (name) ctx->timed_names[ev] = name;
        (void)hipEventRecord((hipEvent_t)ctx->events[ev], stream);
        ev++;
    };
    mark(nullptr);
    if (a.b.pass_event && hipEventRecord((hipEvent_t)a.b.pass_event, stream) != hipSuccess) return -1;
    if (zs_row_launch(a, stream)) return zs_set_error(ctx, ZS_EHIP, "zs_sample: zs_k_row launch failed");
    mark("zs_k_row");
    // the row sums: the approximations and the big rows' sampler S here;
    // S_obs and the entropy (needed only by zs_k_final) on the context's side
    // stream beside the big-row kernels, unless profiling, which keeps every
    // kernel on the caller's stream
    {
        static const char* const names[8] = {"zs_k_sapx1", "zs_k_sround1", "zs_k_sstitch1", "zs_k_sapx2",
                                             "zs_k_sround2", "zs_k_sstitch2", "zs_k_sround3", "zs_k_sstitch3"};
        hipStream_t hs = stream;
        if (!prof) {
            hs = (hipStream_t)ctx->side_stream;
            ZS_LAUNCH_CHECK(hipEventRecord((hipEvent_t)ctx->fork_event, stream));
            ZS_LAUNCH_CHECK(hipStreamWaitEvent(hs, (hipEvent_t)ctx->fork_event, 0));
        }
        for (uint32_t w = 0; w < 3; w++) {
            if (zs_sums_launch(a, w, stream)) return zs_set_error(ctx, ZS_EHIP, "zs_sample: row sums launch failed");
            mark(names[w]);
        }
        for (uint32_t w = 3; w < 8; w++) {
            if (zs_sums_launch(a, w, hs)) return zs_set_error(ctx, ZS_EHIP, "zs_sample: observer sums launch failed");
            mark(names[w]);
        }
        if (!prof) ZS_LAUNCH_CHECK(hipEventRecord((hipEvent_t)ctx->join_event, hs));
    }
    hipLaunchKernelGGL(zs_k_pv, dim3((bt->V + ZS_BIG_G - 1) / ZS_BIG_G, B), dim3(PV_NT), 0, stream, a);
    mark("zs_k_pv");
    hipLaunchKernelGGL(zs_k_tp_plan, dim3(B), dim3(ZS_BIG_NT), 0, stream, a);
    mark("zs_k_tp_plan");
    hipLaunchKernelGGL(zs_k_tp_inc, dim3((bt->V + ZS_BIG_G - 1) / ZS_BIG_G, B), dim3(ZS_BIG_NT), 0, stream, a);
    mark("zs_k_tp_inc");
    hipLaunchKernelGGL(zs_k_tp_sort, dim3(std::min(512u, B * ZS_TP_CAND)), dim3(TP_SORT_NT), 0, stream, a);
    mark("zs_k_tp_sort");
    hipLaunchKernelGGL(zs_k_big, dim3(B), dim3(ZS_BIG_NT), 0, stream, a);
    mark("zs_k_big");
    hipLaunchKernelGGL(zs_k_kcount, dim3((bt->V + ZS_BIG_G - 1) / ZS_BIG_G, B), dim3(PV_NT), 0, stream, a);
    hipLaunchKernelGGL(zs_k_kwrite, dim3((bt->V + ZS_BIG_G - 1) / ZS_BIG_G, B), dim3(PV_NT), 0, stream, a);
    mark("zs_k_kcompact");
    const uint32_t nsubk = (bt->V + ZS_SUB - 1) / ZS_SUB;
    hipLaunchKernelGGL(zs_k_roundK<0>, dim3((nsubk + 3) / 4, B), dim3(256), 0, stream, a);
    mark("zs_k_roundK0");
    hipLaunchKernelGGL(zs_k_stitchK<0>, dim3(B), dim3(SW_NT), 0, stream, a);
    mark("zs_k_stitchK0");
    hipLaunchKernelGGL(zs_k_roundK<1>, dim3((nsubk + 3) / 4, B), dim3(256), 0, stream, a);
    mark("zs_k_roundK1");
    hipLaunchKernelGGL(zs_k_stitchK<1>, dim3(B), dim3(SW_NT), 0, stream, a);
    mark("zs_k_stitchK1");
    if (!prof) ZS_LAUNCH_CHECK(hipStreamWaitEvent(stream, (hipEvent_t)ctx->join_event, 0));
    hipLaunchKernelGGL(zs_k_final, dim3(B), dim3(64), 0, stream, a);
    mark("zs_k_final");
    if (prof) ctx->n_timed = ev - 1;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return zs_set_error(ctx, ZS_EHIP, "zs_sample launch: %s", hipGetErrorString(e));
    return ZS_OK;
}

#ifdef ZS_WALK_DEBUG
extern "C" int zs_dbg_walk_stats_k(unsigned long long* out) {
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(sw_dbg), 32 * sizeof(unsigned long long)) != hipSuccess) return -1;
    static unsigned long long zero[32];
    return hipMemcpyToSymbol(HIP_SYMBOL(sw_dbg), zero, sizeof(zero)) == hipSuccess ? 0 : -1;
}
#endif
