// zs_walk.h -- exact sequential f32 sums over sub-chunks of ZS_SUB terms:
// the stitch side of the GPU-wide sums (zs_sums.hip: the row sums;
// zs_sample.hip: the kept-list sums of the top-p draw).
//
// Inside one binade of the running sum s its values lie on the grid g = ulp(s)
// and adding a term t moves s by the integer round_half_even(t / g) (zs_math.h),
// except for an exact half-way term (its rounding follows the parity of s / g:
// an increment pair, total from an even start and from an odd start) and for
// the term that carries s out of its binade. A round kernel gives every
// sub-chunk whose grid it could predict its increment pair on that grid (a
// record); one 256-thread workgroup then walks the sub-chunks in order from
// the exact running sum (sm_stitch):
//   - runs of records whose grid is the sum's and whose totals keep the sum
//     inside its binade (and below the stop threshold) are applied 64 at a
//     time with a pair scan;
//   - any other sub-chunk is walked from its exact terms (sm_walk): per-thread
//     increment pairs prefix-scanned over the workgroup locate the first thread
//     whose terms leave the binade or reach the threshold; that thread steps
//     through its terms to that term, which it adds as a real f32 addition,
//     and the rest continues on the new grid (in the same step when no
//     half-way term of the next grid is in the way).
// Records are hints: a wrong grid or a total that would leave the binade sends
// the sub-chunk to the exact walk.
#pragma once
#include "zs_dev.h"
#include "zs_seq.h"

#define SM_SAFE 1u
#define SM_QCAP 33554432.0f     // increments clamp at 2^25 (any larger one leaves the binade)
#define SM_EG_MIN 28            // grids from 2^-122 up take the float-scaled increments
#define SM_HEAD 128             // terms added one by one from a sum's first nonzero term
#define SW_NT 256               // threads of a walk
#define SW_NW (SW_NT / 64)
#define SW_TPT 4                // terms per thread
static_assert(SW_NT * SW_TPT == ZS_SUB, "one workgroup per sub-chunk walk");

// Per (sum, sub-chunk) record of a round kernel.
struct sm_rec {
    int32_t eg;       // grid exponent the totals are on
    uint32_t flags;   // SM_SAFE: totals valid; SM_CROSS: a crossing record (below)
    uint32_t d0, d1;  // increments from an even / odd start (saturated at ZS_INC_CAP)
};
// A sub-chunk where the running sum is expected to leave its binade once, at
// term x: its sm_rec holds the start grid eg, SM_CROSS and the increment pair
// of terms 0 .. x-1 on grid eg; this record the exact term x and the pair of
// terms x+1 .. on grid eg + 1. The stitch checks the guess from the exact
// running sum (no exit before x, an exit at x into binade eg + 1, none after)
// and walks the sub-chunk when it fails.
// SM_ALT: the start may already be in binade eg + 1 (the crossing near the
// sub-chunk's start, on either side of it): the record also holds the pair
// of all the terms on grid eg + 1 (a0, a1), applied when the exact running
// sum is found there. (SM_ALT without SM_CROSS: only that pair is valid.)
#define SM_CROSS 2u
#define SM_ALT 4u
// SM_EXACT (sub-chunk 0 only): the round kernel, which knows the sum's start
// value, added the sub-chunk's terms one by one itself: d0 holds the bits of
// the sum after them, d1 the term where it reached the stop threshold (or
// 0xffffffff).
#define SM_EXACT 8u
struct sm_xrec {
    uint32_t x;
    float vx;
    uint32_t p0, p1;
    uint32_t a0, a1;
};

// 2^(150 - eg): the scale of grid eg (eg >= 24).
__device__ __forceinline__ float sm_scale(int eg) { return __uint_as_float((uint32_t)(277 - eg) << 23); }

// The pair of a half-way term m + 1/2: k + m goes to the even neighbour.
__device__ __forceinline__ seq_pair sm_pair_tie(uint32_t m) {
    seq_pair p;
    p.e = m + (m & 1u);
    p.o = m + ((m + 1u) & 1u);
    return p;
}

// Inclusive ordered scan of pairs over the wave: shifts by 1, 2, 4, 8 inside
// each row of 16 lanes, then the rows by broadcasts (DPP moves; a lane
// without a source receives the identity pair (0, 0)).
template <int CTRL, int ROWS, bool BC>
__device__ __forceinline__ seq_pair sm_pair_step(seq_pair p) {
    seq_pair o;
    o.e = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)p.e, CTRL, ROWS, 0xf, BC);
    o.o = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)p.o, CTRL, ROWS, 0xf, BC);
    return seq_compose(o, p);
}
__device__ __forceinline__ seq_pair sm_wave_pair_scan(seq_pair p) {
    p = sm_pair_step<0x111, 0xf, true>(p);    // row_shr:1
    p = sm_pair_step<0x112, 0xf, true>(p);    // row_shr:2
    p = sm_pair_step<0x114, 0xf, true>(p);    // row_shr:4
    p = sm_pair_step<0x118, 0xf, true>(p);    // row_shr:8
    p = sm_pair_step<0x142, 0xa, false>(p);   // row_bcast:15
    p = sm_pair_step<0x143, 0xc, false>(p);   // row_bcast:31
    return p;
}

// Inclusive saturating scan of a u32 over the wave, with the same DPP moves.
template <int CTRL, int ROWS, bool BC>
__device__ __forceinline__ uint32_t sm_sat_step(uint32_t x) {
    return zs_sat_add(x, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)x, CTRL, ROWS, 0xf, BC));
}
__device__ __forceinline__ uint32_t sm_wave_scan_sat(uint32_t x) {
    x = sm_sat_step<0x111, 0xf, true>(x);
    x = sm_sat_step<0x112, 0xf, true>(x);
    x = sm_sat_step<0x114, 0xf, true>(x);
    x = sm_sat_step<0x118, 0xf, true>(x);
    x = sm_sat_step<0x142, 0xa, false>(x);
    x = sm_sat_step<0x143, 0xc, false>(x);
    return x;
}

// Ordered reduction of pairs over the wave (lanes in increasing order; the
// result is uniform): the last lane of the DPP scan (the composition is
// associative), which keeps it off the LDS permute path of lane shuffles.
__device__ __forceinline__ seq_pair sm_wave_pair_reduce(seq_pair p) {
    p = sm_wave_pair_scan(p);
    p.e = (uint32_t)__builtin_amdgcn_readlane((int)p.e, 63);
    p.o = (uint32_t)__builtin_amdgcn_readlane((int)p.o, 63);
    return p;
}

// Saturating sum over the wave (uniform), the same way (the clamp at
// ZS_INC_CAP of non-negative terms is associative).
__device__ __forceinline__ uint32_t sm_wave_sum_sat(uint32_t v) {
    return (uint32_t)__builtin_amdgcn_readlane((int)sm_wave_scan_sat(v), 63);
}

__device__ __forceinline__ float sm_lane_f(float v, uint32_t l) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), (int)l));
}

// Workgroup barrier that orders LDS accesses only: __syncthreads() also waits
// for every outstanding global load of the calling wave, which would drain
// the loads the stitch keeps in flight for its next walks.
__device__ __forceinline__ void sm_bar() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// The walk's LDS: a file-scope object in each translation unit that includes
// this header, so that every access is an LDS instruction.
struct sm_wsh {
    uint32_t we[2][SW_NW], wo[2][SW_NW];   // per-wave pair totals on the grid (double buffered by step)
    uint32_t w2[2][SW_NW];                 // per-wave totals on the next grid
    uint32_t wt2[2][SW_NW];                // per wave: a half-way term on the next grid
    uint32_t cross[2][SW_NW];              // per wave: a thread of it leaves the binade or stops
    float s_new[2][SW_NW];
    uint32_t pos_new[2][SW_NW];            // the next term (ZS_SUB: done), | SW_STOP: stopped at pos - 1
    float tot_s[2];                        // the sum after the last thread (nothing met)
    uint32_t first[SW_NW];                 // zero sums: first nonzero term per wave
    float hs;
    uint32_t hstop;
    alignas(16) float hv[SW_TPT * 64];     // the head: one wave's terms, added one by one from here
    sm_rec rec[ZS_MAX_SUBS];               // the records of the sum being stitched
    sm_xrec xrec[ZS_MAX_SUBS];             // its crossing records (when the caller has them)
};
__shared__ sm_wsh sm_sh;
#define SW_STOP 0x80000000u

#ifdef ZS_WALK_DEBUG
// working diagnostics: cycles per walk phase (summed over workgroups)
__device__ unsigned long long sw_dbg[32];
__device__ unsigned long long sw_hist[64];
__shared__ unsigned long long sw_acc[16];
#define SW_T(i, c) do { if (threadIdx.x == 0) sw_acc[i] += (unsigned long long)(c); } while (0)
#define SW_CLK() clock64()
#define SW_K(k, tot, pre) do { if (threadIdx.x == 0) { atomicMax(&sw_dbg[16 + 3 * (k)], (unsigned long long)(tot)); \
    atomicAdd(&sw_dbg[17 + 3 * (k)], (unsigned long long)(tot)); atomicAdd(&sw_dbg[18 + 3 * (k)], (unsigned long long)(pre)); } } while (0)
#else
#define SW_K(k, tot, pre) ((void)0)
#define SW_T(i, c) ((void)0)
#define SW_CLK() 0ull
#endif

// Increments of a thread's 4 exact terms (those in `valid`) on grid eg, the
// half-way flags, and their pair.
__device__ __forceinline__ seq_pair sm_incs4(const float (&v)[SW_TPT], int eg, uint32_t valid,
                                             uint32_t (&inc)[SW_TPT], uint32_t& tie) {
    tie = 0u;
    if (eg >= SM_EG_MIN) {
        const float sc = sm_scale(eg);
#pragma unroll
        for (int q = 0; q < SW_TPT; q++) {
            const float qv = fminf(v[q] * sc, SM_QCAP);
            float rq = rintf(qv);
            const bool h = fabsf(qv - rq) == 0.5f && ((valid >> q) & 1u);
            if (h) rq = floorf(qv);
            tie |= (h ? 1u : 0u) << q;
            inc[q] = ((valid >> q) & 1u) ? (uint32_t)rq : 0u;
        }
    } else {
        // sums below 2^-99: integer increments
#pragma unroll
        for (int q = 0; q < SW_TPT; q++) {
            uint32_t tq = 0u;
            inc[q] = ((valid >> q) & 1u) ? zs_seq_inc(v[q], eg, &tq) : 0u;
            tie |= tq << q;
        }
    }
    seq_pair lp = {0u, 0u};
    if (tie) {
#pragma unroll
        for (int q = 0; q < SW_TPT; q++)
            lp = seq_compose(lp, ((tie >> q) & 1u) ? sm_pair_tie(inc[q]) : seq_pair{inc[q], inc[q]});
    } else {
        uint32_t tot = 0u;
#pragma unroll
        for (int q = 0; q < SW_TPT; q++) tot = zs_sat_add(tot, inc[q]);
        lp = seq_pair{tot, tot};
    }
    return lp;
}

// The exact walk of one sub-chunk over its exact terms v (thread t: terms
// 4t .. 4t+3) from running sum s, stopping after the first term where the
// sum reaches `thresh` (NaN: never): *stop = that term, else 0xffffffff.
// Called by the whole workgroup; the result is uniform.
__device__ __forceinline__ float sm_walk(const float (&v)[SW_TPT], float s, float thresh, uint32_t* stop) {
    sm_wsh& sh = sm_sh;
    const uint32_t t = threadIdx.x, lane = (uint32_t)zs_lane(), wid = (uint32_t)zs_wid();
    uint32_t pos = 0, par = 0;   // first term not yet added; LDS slot of this step
    *stop = 0xffffffffu;
    while (pos < ZS_SUB) {
        if (s == 0.0f) {
            // a zero sum takes its first nonzero term as it is (zero terms
            // before it leave a +0: -0 + +0 = +0); from there the sum climbs
            // through a binade at almost every doubling of the number of
            // terms: the next SM_HEAD terms are added one by one, in order
            uint32_t my = 0xffffffffu;
#pragma unroll
            for (int q = SW_TPT - 1; q >= 0; q--)
                if (SW_TPT * t + (uint32_t)q >= pos && v[q] != 0.0f) my = SW_TPT * t + (uint32_t)q;
            const unsigned long long m = __ballot(my != 0xffffffffu);
            if (lane == 0) sh.first[wid] = m ? (uint32_t)__builtin_amdgcn_readlane((int)my, __ffsll((long long)m) - 1) : 0xffffffffu;
            sm_bar();
            uint32_t first = 0xffffffffu;
#pragma unroll
            for (int w = 0; w < SW_NW; w++) first = min(first, sh.first[w]);
            // (zero terms leave a zero sum +0 and never reach a positive
            // threshold; a threshold of zero or less stops at term 0, which
            // callers handle before the walk)
            s = s + 0.0f;
            if (first == 0xffffffffu) return s;
            const uint32_t end = min(first + SM_HEAD, (uint32_t)ZS_SUB);
            [[maybe_unused]] const unsigned long long h0 = SW_CLK();
            // the head's terms lie in at most two waves: each wave adds the
            // ones it holds, in order, the first wave's before the second's
            const uint32_t w0 = first / (SW_TPT * 64), w1 = (end - 1) / (SW_TPT * 64);
            const bool thr = thresh == thresh;
            for (uint32_t w = w0; w <= w1; w++) {
                if (wid == w) {
                    // the wave's terms to LDS in term order, then every lane
                    // adds the same ones in order (broadcast reads, no lane
                    // reads); the terms are non-negative, so the running sum
                    // never decreases and one test per 4 terms finds the stop
                    float ss = w != w0 ? sh.hs : s;
                    uint32_t sp = w != w0 ? sh.hstop : 0xffffffffu;
                    const uint32_t base = SW_TPT * 64 * w;
                    *reinterpret_cast<float4*>(&sh.hv[SW_TPT * lane]) = make_float4(v[0], v[1], v[2], v[3]);
                    __builtin_amdgcn_s_waitcnt(0);
                    __builtin_amdgcn_wave_barrier();
                    const uint32_t e0 = first > base ? first - base : 0u, e1 = min(end - base, SW_TPT * 64u);
                    uint32_t e = sp == 0xffffffffu ? e0 : e1;   // (stopped in the wave before: nothing)
                    for (; e < e1 && (e & 3u); e++) {   // to a multiple of 4
                        ss = ss + sh.hv[e];
                        if (thr && ss >= thresh) { sp = base + e; break; }
                    }
                    // 32 terms per batch of LDS reads (their latency off the
                    // chain of additions); a batch that reaches the threshold
                    // is done again below, 4 terms at a time, to find the term
                    if (sp == 0xffffffffu) {
                        for (; e + 32 <= e1; e += 32) {
                            float4 q8[8];
#pragma unroll
                            for (int i = 0; i < 8; i++) q8[i] = *reinterpret_cast<const float4*>(&sh.hv[e + 4 * i]);
                            float c = ss;
#pragma unroll
                            for (int i = 0; i < 8; i++) c = (((c + q8[i].x) + q8[i].y) + q8[i].z) + q8[i].w;
                            if (thr && c >= thresh) break;
                            ss = c;
                        }
                    }
                    if (sp == 0xffffffffu) {
                        for (; e + 4 <= e1; e += 4) {
                            const float4 q4 = *reinterpret_cast<const float4*>(&sh.hv[e]);
                            const float c1 = ss + q4.x, c2 = c1 + q4.y, c3 = c2 + q4.z, c4 = c3 + q4.w;
                            if (thr && c4 >= thresh) {
                                const uint32_t k = c1 >= thresh ? 0u : c2 >= thresh ? 1u : c3 >= thresh ? 2u : 3u;
                                ss = k == 0u ? c1 : k == 1u ? c2 : k == 2u ? c3 : c4;
                                sp = base + e + k;
                                break;
                            }
                            ss = c4;
                        }
                    }
                    if (sp == 0xffffffffu) {
                        for (; e < e1; e++) {
                            ss = ss + sh.hv[e];
                            if (thr && ss >= thresh) { sp = base + e; break; }
                        }
                    }
                    if (lane == 0) { sh.hs = ss; sh.hstop = sp; }
                }
                sm_bar();
            }
            s = sh.hs;
            const uint32_t sp = sh.hstop;
            pos = end;
            sm_bar();
            SW_T(6, SW_CLK() - h0); SW_T(7, 1);
            if (sp != 0xffffffffu) { *stop = sp; return s; }
            continue;
        }
        [[maybe_unused]] const unsigned long long c0 = SW_CLK();
        const int eg = zs_grid_exp(s);
        const uint32_t k = zs_grid_k(s);
        const uint32_t kthr = zs_grid_thresh(thresh, eg);
        uint32_t valid = 0u;
#pragma unroll
        for (int q = 0; q < SW_TPT; q++) valid |= (SW_TPT * t + (uint32_t)q >= pos ? 1u : 0u) << q;
        uint32_t inc[SW_TPT], tie = 0u, inc2[SW_TPT], tie2 = 0u, tot = 0u, tot2 = 0u;
        // the next grid as well: after a crossing the rest of the sub-chunk
        // usually stays on it (its increments halve the scaled terms exactly)
        const bool two = eg >= SM_EG_MIN && eg + 1 < 254;
        if (eg >= SM_EG_MIN) {
            const float sc = sm_scale(eg);
#pragma unroll
            for (int q = 0; q < SW_TPT; q++) {
                const bool in = (valid >> q) & 1u;
                const float qv = fminf(v[q] * sc, SM_QCAP);
                float rq = rintf(qv);
                const bool h = fabsf(qv - rq) == 0.5f && in;
                if (h) rq = floorf(qv);
                tie |= (h ? 1u : 0u) << q;
                inc[q] = in ? (uint32_t)rq : 0u;
                const float qv2 = qv * 0.5f;
                const float rq2 = rintf(qv2);
                tie2 |= (fabsf(qv2 - rq2) == 0.5f && in ? 1u : 0u) << q;
                inc2[q] = in ? (uint32_t)rq2 : 0u;
                tot = zs_sat_add(tot, inc[q]);
                tot2 = zs_sat_add(tot2, inc2[q]);
            }
        } else {
            // sums below 2^-99: integer increments
#pragma unroll
            for (int q = 0; q < SW_TPT; q++) {
                uint32_t tq = 0u;
                inc[q] = ((valid >> q) & 1u) ? zs_seq_inc(v[q], eg, &tq) : 0u;
                tie |= tq << q;
                tot = zs_sat_add(tot, inc[q]);
                inc2[q] = 0u;
            }
            tie2 = 1u;
        }
        [[maybe_unused]] const unsigned long long c1 = SW_CLK();
        // inclusive scans over the wave: plain sums unless a half-way term
        // makes the increments depend on the parity
        const bool wtie = __builtin_amdgcn_readfirstlane((int)(__ballot(tie != 0u) != 0ull)) != 0;
        seq_pair wp;
        if (!wtie) {
            const uint32_t x = sm_wave_scan_sat(tot);
            wp = seq_pair{x, x};
        } else {
            seq_pair own = {0u, 0u};
#pragma unroll
            for (int q = 0; q < SW_TPT; q++)
                own = seq_compose(own, ((tie >> q) & 1u) ? sm_pair_tie(inc[q]) : seq_pair{inc[q], inc[q]});
            wp = sm_wave_pair_scan(own);
        }
        const uint32_t w2 = sm_wave_scan_sat(tot2);
        const bool anyt2w = __ballot(tie2 != 0u) != 0ull;
        if (lane == 63) {
            sh.we[par][wid] = wp.e;
            sh.wo[par][wid] = wp.o;
            sh.w2[par][wid] = w2;
            sh.wt2[par][wid] = anyt2w ? 1u : 0u;
        }
        [[maybe_unused]] const unsigned long long c2 = SW_CLK();
        sm_bar();
        [[maybe_unused]] const unsigned long long c3 = SW_CLK();
        seq_pair pre = {0u, 0u};   // the waves before this one
        uint32_t pre2 = 0u, all2 = 0u, anyt2 = 0u;
#pragma unroll
        for (int w = 0; w < SW_NW; w++) {
            if ((uint32_t)w < wid) {
                pre = seq_compose(pre, seq_pair{sh.we[par][w], sh.wo[par][w]});
                pre2 = zs_sat_add(pre2, sh.w2[par][w]);
            }
            all2 = zs_sat_add(all2, sh.w2[par][w]);
            anyt2 |= sh.wt2[par][w];
        }
        const seq_pair incl = seq_compose(pre, wp);
        const uint32_t kend = zs_sat_add(k, (k & 1u) ? incl.o : incl.e);
        const unsigned long long bad = __ballot(kend >= ZS_BINADE || kend >= kthr);
        // the exclusive prefix of the first thread that leaves the binade or
        // reaches the threshold
        seq_pair ex;
        ex.e = (uint32_t)__shfl_up((int)wp.e, 1, 64);
        ex.o = wtie ? (uint32_t)__shfl_up((int)wp.o, 1, 64) : ex.e;
        if (lane == 0) ex = seq_pair{0u, 0u};
        ex = seq_compose(pre, ex);
        const uint32_t L = bad ? (uint32_t)(__ffsll((long long)bad) - 1) : 64u;
        if (lane == L) {
            uint32_t kk = zs_sat_add(k, (k & 1u) ? ex.o : ex.e);
            int qx = SW_TPT - 1;
            bool found = false, at_thr = false;
#pragma unroll
            for (int q = 0; q < SW_TPT; q++) {
                if (found || !((valid >> q) & 1u)) continue;
                const uint32_t kn = zs_sat_add(kk, ((tie >> q) & 1u) ? inc[q] + ((kk + inc[q]) & 1u) : inc[q]);
                if (kn >= ZS_BINADE) { qx = q; found = true; }
                else if (kn >= kthr) { qx = q; found = true; at_thr = true; kk = kn; }
                else kk = kn;
            }
            float vx = 0.0f;
            uint32_t after2 = 0u;   // this thread's next-grid increments after term qx
#pragma unroll
            for (int q = 0; q < SW_TPT; q++) {
                if (q == qx) vx = v[q];
                if (q > qx) after2 = zs_sat_add(after2, inc2[q]);
            }
            float sn;
            uint32_t pn = SW_TPT * t + (uint32_t)qx + 1u;
            if (at_thr) {
                sn = zs_grid_value(kk, eg);   // the sum through term qx, on this grid
                pn |= SW_STOP;
            } else {
                const float sx = zs_grid_value(kk, eg) + vx;   // the term that leaves the binade
                sn = sx;
                if (sx >= thresh) {
                    pn |= SW_STOP;
                } else if (two && !anyt2 && zs_grid_exp(sx) == eg + 1) {
                    // the rest on the next grid: its total minus the terms
                    // through qx (no half-way term there: plain sums)
                    const uint32_t rest = zs_sat_add(all2 - min(all2, zs_sat_add(pre2, w2)), after2);
                    const uint32_t k2 = zs_sat_add(zs_grid_k(sx), rest);
                    if (all2 < ZS_INC_CAP && k2 < ZS_BINADE && k2 < zs_grid_thresh(thresh, eg + 1)) {
                        sn = zs_grid_value(k2, eg + 1);
                        pn = ZS_SUB;
                    }
                }
            }
            sh.s_new[par][wid] = sn;
            sh.pos_new[par][wid] = pn;
        }
        if (lane == 0) sh.cross[par][wid] = bad ? 1u : 0u;
        if (t == SW_NT - 1) sh.tot_s[par] = (kend < ZS_BINADE && kend < kthr) ? zs_grid_value(kend, eg) : 0.0f;
        [[maybe_unused]] const unsigned long long c4 = SW_CLK();
        sm_bar();
        [[maybe_unused]] const unsigned long long c5 = SW_CLK();
        SW_T(0, c1 - c0); SW_T(1, c2 - c1); SW_T(2, c3 - c2); SW_T(3, c4 - c3); SW_T(4, c5 - c4); SW_T(5, 1);
        int cw = -1;
#pragma unroll
        for (int w = SW_NW - 1; w >= 0; w--)
            if (sh.cross[par][w]) cw = w;
        if (cw < 0) return sh.tot_s[par];
        s = sh.s_new[par][cw];
        pos = sh.pos_new[par][cw];
        par ^= 1u;
        if (pos & SW_STOP) {
            *stop = (pos & ~SW_STOP) - 1u;
            return s;
        }
    }
    return s;
}

// The sequential f32 sum of buf[0 .. n-1] (LDS, n a multiple of 32) from s,
// one addition per term in order, stopping at the first term where it
// reaches thresh (NaN: never): *stop = that term, else 0xffffffff. The terms
// are read 32 at a time, so their loads stay off the chain of additions; a
// batch that reaches the threshold is added again term by term.
__device__ __forceinline__ float sm_serial(const float* buf, uint32_t n, float s, float thresh, uint32_t* stop) {
    *stop = 0xffffffffu;
    const bool thr = thresh == thresh;
    for (uint32_t e = 0; e < n; e += 32) {
        float4 q8[8];
#pragma unroll
        for (int i = 0; i < 8; i++) q8[i] = *reinterpret_cast<const float4*>(buf + e + 4 * i);
        float c = s;
#pragma unroll
        for (int i = 0; i < 8; i++) c = (((c + q8[i].x) + q8[i].y) + q8[i].z) + q8[i].w;
        if (thr && c >= thresh) {
            for (uint32_t i = e; i < e + 32; i++) {
                s = s + buf[i];
                if (s >= thresh) {
                    *stop = i;
                    return s;
                }
            }
        }
        s = c;
    }
    return s;
}

// First sub-chunk from j whose record is neither safe nor a crossing record
// (nsub: none): the next one whose terms the stitch will surely need; uniform.
__device__ __forceinline__ uint32_t sm_next_fragile(uint32_t j, uint32_t nsub) {
    for (uint32_t i0 = j; i0 < nsub; i0 += 64) {
        const uint32_t i = i0 + (uint32_t)zs_lane();
        const unsigned long long m = __ballot(i < nsub && !(sm_sh.rec[i].flags & (SM_SAFE | SM_CROSS | SM_ALT | SM_EXACT)));
        if (m) return i0 + (uint32_t)(__ffsll((long long)m) - 1);
    }
    return nsub;
}

// The sum over nsub sub-chunks whose records are in sm_sh.rec (crossing
// records in sm_sh.xrec), from s, with the stop threshold `thresh` (NaN:
// none): *stop = the global index of the term where the sum reaches it, else
// 0xffffffff. The term provider TP gives the thread's 4 exact terms of a
// sub-chunk: tp.fetch(j, raw) issues the loads of the stored exact terms of
// a sub-chunk the round kernel left without a safe record (those with neither
// a safe nor a crossing record two walks ahead; a crossing record's terms
// only when it does not hold), tp.take(j, raw, v) turns them into terms,
// tp.direct(j, v) computes them for a sub-chunk whose record was safe but
// whose total did not apply.
// A crossing record of sub-chunk j applied to the exact running sum s
// (uniform): true with the new sum, or with *stop set when the threshold is
// reached at its term x; false when its guess does not hold.
__device__ __forceinline__ bool sm_cross(uint32_t j, float& s, float thresh, uint32_t* stop) {
    const sm_rec e = sm_sh.rec[j];
    const sm_xrec xr = sm_sh.xrec[j];   // (read with the record: meaningful only with SM_CROSS / SM_ALT)
    if (!(e.flags & (SM_CROSS | SM_ALT)) || s == 0.0f) return false;
    const int eg = zs_grid_exp(s);
    const uint32_t k = zs_grid_k(s);
    if ((e.flags & SM_ALT) && eg == e.eg + 1) {
        // already past the crossing: every term on this grid
        const uint32_t ka = zs_sat_add(k, (k & 1u) ? xr.a1 : xr.a0);
        if (ka >= ZS_BINADE || ka >= zs_grid_thresh(thresh, eg)) return false;
        s = zs_grid_value(ka, eg);
        return true;
    }
    if (e.eg != eg || !(e.flags & SM_CROSS)) {
#ifdef ZS_WALK_DEBUG
        if (threadIdx.x == 0) atomicAdd(&sw_dbg[30], 1ull);
#endif
        return false;
    }
    const uint32_t k1 = zs_sat_add(k, (k & 1u) ? e.d1 : e.d0);
    if (k1 >= ZS_BINADE || k1 >= zs_grid_thresh(thresh, eg)) { SW_T(15, 1); return false; }
    const float sx = zs_grid_value(k1, eg) + xr.vx;   // the term that leaves the binade
    if (zs_grid_exp(sx) != eg + 1) {
#ifdef ZS_WALK_DEBUG
        if (threadIdx.x == 0) atomicAdd(&sw_dbg[31], 1ull);
#endif
        return false;
    }
    if (sx >= thresh) {
        *stop = j * ZS_SUB + xr.x;
        s = sx;
        return true;
    }
    const uint32_t kx = zs_grid_k(sx);
    const uint32_t k2 = zs_sat_add(kx, (kx & 1u) ? xr.p1 : xr.p0);
    if (k2 >= ZS_BINADE || k2 >= zs_grid_thresh(thresh, eg + 1)) return false;
    s = zs_grid_value(k2, eg + 1);
    return true;
}

template <class TP, class RAW>
__device__ __forceinline__ float sm_stitch(TP& tp, uint32_t nsub, float s, float thresh, uint32_t* stop) {
    const uint32_t lane = (uint32_t)zs_lane();
    *stop = 0xffffffffu;
    uint32_t nf0 = sm_next_fragile(0, nsub);
    uint32_t nf1 = nf0 < nsub ? sm_next_fragile(nf0 + 1, nsub) : nsub;
    RAW q0, q1;
#ifdef ZS_WALK_DEBUG
    if (threadIdx.x < 16) sw_acc[threadIdx.x] = 0ull;
#endif
    if (nf0 < nsub) tp.fetch(nf0, q0);
    if (nf1 < nsub) tp.fetch(nf1, q1);
    uint32_t j = 0;
    if (nsub && (sm_sh.rec[0].flags & SM_EXACT)) {
        s = __uint_as_float(sm_sh.rec[0].d0);
        if (sm_sh.rec[0].d1 != 0xffffffffu) {
            *stop = sm_sh.rec[0].d1;
            return s;
        }
        j = 1;
    }
    while (j < nsub) {
        [[maybe_unused]] const unsigned long long g0 = SW_CLK();
        const uint32_t fj = sm_sh.rec[j].flags;
        if (s != 0.0f && (fj & SM_SAFE)) {
            // sub-chunks j .. j+63 on the grid of s, applied up to the first
            // one that is not safe, is on another grid, leaves the binade or
            // reaches the threshold
            const int eg = zs_grid_exp(s);
            const uint32_t k = zs_grid_k(s);
            const uint32_t kthr = zs_grid_thresh(thresh, eg);
            const uint32_t i = j + lane;
            const sm_rec e = i < nsub ? sm_sh.rec[i] : sm_rec{0, 0u, 0u, 0u};
            const bool ok = (e.flags & SM_SAFE) && e.eg == eg;
            const seq_pair p = sm_wave_pair_scan(ok ? seq_pair{e.d0, e.d1} : seq_pair{ZS_INC_CAP, ZS_INC_CAP});
            const uint32_t kend = zs_sat_add(k, (k & 1u) ? p.o : p.e);
            const unsigned long long bad = __ballot(!(ok && kend < ZS_BINADE && kend < kthr));
            const uint32_t n_ok = bad ? (uint32_t)(__ffsll((long long)bad) - 1) : 64u;
            if (n_ok) {
                SW_T(11, 1); SW_T(14, SW_CLK() - g0);
                s = zs_grid_value((uint32_t)__builtin_amdgcn_readlane((int)kend, (int)n_ok - 1), eg);
                j += n_ok;
                continue;
            }
        }
        const bool xr = (fj & (SM_CROSS | SM_ALT)) != 0u;
        if (xr) {
            uint32_t sp = 0xffffffffu;
            if (sm_cross(j, s, thresh, &sp)) {
                SW_T(13, 1);
                if (sp != 0xffffffffu) {
                    *stop = sp;
                    break;
                }
                j++;
                SW_T(12, SW_CLK() - g0);
                continue;
            }
        }
        float v[SW_TPT];
        [[maybe_unused]] const unsigned long long l0 = SW_CLK();
        if (xr) {
            // a crossing record that did not hold: its stored terms
            RAW qx;
            tp.fetch(j, qx);
            tp.take(j, qx, v);
        } else if (j == nf0) {
#ifdef ZS_WALK_DEBUG
            if (threadIdx.x == 0 && !(sm_sh.rec[j].flags & SM_CROSS)) atomicAdd(&sw_dbg[28], 1ull);
#endif
            tp.take(j, q0, v);
            nf0 = nf1;
            q0 = q1;
            nf1 = nf0 < nsub ? sm_next_fragile(nf0 + 1, nsub) : nsub;
            if (nf1 < nsub) tp.fetch(nf1, q1);
        } else {
#ifdef ZS_WALK_DEBUG
            if (threadIdx.x == 0) atomicAdd(&sw_dbg[27], 1ull);
#endif
            tp.direct(j, v);
        }
        uint32_t sp;
#ifdef ZS_WALK_DEBUG
        if (threadIdx.x == 0) atomicAdd(&sw_hist[j < 31u ? j : (j + 32u >= nsub ? 63u - (nsub - 1u - j) : 31u)], 1ull);
#endif
        [[maybe_unused]] const unsigned long long l1 = SW_CLK();
        SW_T(8, l1 - l0); SW_T(9, 1);
        s = sm_walk(v, s, thresh, &sp);
        sm_bar();
        SW_T(10, SW_CLK() - l1);
        if (sp != 0xffffffffu) {
            *stop = j * ZS_SUB + sp;
            break;
        }
        j++;
    }
#ifdef ZS_WALK_DEBUG
    if (threadIdx.x < 16) atomicAdd(&sw_dbg[threadIdx.x], sw_acc[threadIdx.x]);
#endif
    return s;
}
