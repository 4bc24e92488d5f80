// zs_row.hip -- the front of the sampler step, one 512-thread workgroup per
// row: everything of a row that needs the whole row, with no other workgroup
// involved and therefore no device-scope synchronisation and no launch
// boundary between the phases.
//
// Reference semantics (per row, in the order of rest.rs:2594-2624):
//   x~ = apply_mask(x)                    logit_fsm.rs:247-270 (bans, allow bits)
//   y  = adjust_logits(x~)                decode_ctrl.rs:107-126
//   token = sample_with_rng(y, cfg, r)    sampler.rs:31-128
//   logprobs / token_uncertainty on x~    logprobs.rs:34-54, hallucination.rs:129-154
//
// Phases of zs_k_row:
//   P0  patches: the row's ban / bias / count-map entries merged into one list
//       sorted by id with the exact patched y of every listed id
//       (decode_ctrl.rs:107-126 operation order; lists of any length: the
//       first ZS_PATCH_LDS entries in LDS, the rest in row scratch), ranked by
//       a bitmap of the patched ids with per-word prefix counts, and stored
//       for the later kernels;
//   P1  one read of the logits: observer maximum / NaN / +inf, sampler maximum,
//       finite count and flags, greedy argmax (last maximal element, a NaN
//       restarts the fold: sampler.rs:35-43), and candidate lists kept in LDS
//       behind a rising threshold: the observers' top entries by (x~ desc, id
//       asc) for top_logprobs / margin, the sampler's top-k by (z desc, id asc)
//       (sampler.rs:53-64: its k-th key is the threshold), or every finite z
//       when no top-k applies and at most ZS_SMALL_CAP are finite;
//   decisions: greedy / non-finite rows get their token; rows whose survivors
//       fit ZS_SMALL_CAP are sampled exactly by one wave (small_path_wave);
//       other rows are "big" and continue in zs_sample.hip;
//   state: which exact sums the row needs (zs_sums.hip: the observers' S and
//       entropy, a big row's sampler S), over the whole row or over the
//       allowed ids a masked row gathered to row scratch.
#include <hip/hip_runtime.h>
#ifdef ZS_WALK_DEBUG
// Debug builds: wall-clock time of zs_k_row's phases (0-5, row count in 7)
// and of the small path's (8-15), summed over rows (zs_dbg_row_stats).
__device__ unsigned long long rw_dbg[16];
#define ZS_SP_T(i)                                               \
    do {                                                         \
        if (zs_lane() == 0) {                                    \
            const unsigned long long c_ = wall_clock64();        \
            atomicAdd(&rw_dbg[8 + (i)], c_ - sp_t0);             \
            sp_t0 = c_;                                          \
        }                                                        \
    } while (0)
#endif
#include "zs_sampler.h"

#define RW_NT 512
#define RW_NW (RW_NT / 64)
#define RW_G 2048          // ids per tile: one float4 per thread
#define RW_BUF 2048        // candidate buffer entries (per list)
#define RW_KEEP 1024       // a list above this is compacted to its top K
// per (row, half) slot of a split row: statistics, then the observers' and
// the sampler's list entries
#define RW_PART_O 16
#define RW_PART_S (RW_PART_O + 32)
#define RW_PART (RW_PART_S + ZS_SMALL_CAP)

struct rw_shared {
    uint32_t pid[4096];             // the patch list's head (ZS_PATCH_LDS): ids (sorted) | flags << 30
    float py[4096];                 // their y
    union {
        struct {
            unsigned long long o[RW_BUF];         // P1: observer candidates
            unsigned long long s[RW_BUF];         // P1: sampler candidates
        } b;
    } u;
    alignas(16) float sval[ZS_SMALL_CAP];   // also the small path's scratch
    uint32_t sidx[ZS_SMALL_CAP];
    uint32_t cand_id[ZS_OBS_CAND];
    float cand_x[ZS_OBS_CAND];
    uint32_t ru[6][RW_NW];
    float rf[3][RW_NW];
    float fthr[2];                  // candidate thresholds as values
    float fcut[2];                  // largest values cut from the lists
    unsigned long long rl[RW_NW];
    uint32_t n_surv, tok;
    uint32_t merge;                 // split rows: the halves that finished before this one
    uint32_t ovf[3];                // first tile that lost a list entry, per group slot
    uint32_t thr_o, thr_s;          // candidate admission thresholds (keys)
    float fsh;
    uint32_t sel_hist[2][256];      // list selection: digit histogram (double buffered)
    uint32_t sel_mm[3][RW_NW];      // list selection: per-wave member count, key min / max
    uint32_t sel_n;                 // list selection: places taken by the gather
    uint32_t inf_lim;               // observers: largest id whose -inf can enter the list
    uint32_t g_n, g_done;           // masked rows: allowed ids gathered to row scratch, gather done
    uint32_t sel_st[4];             // list selection: chosen digit, count before it, its count, places
};
// The workgroup's LDS (one object, so that functions outside the kernel
// address it directly).
__shared__ rw_shared rw_sh;
// Bitmap of the row's patched ids, ceil(V / 32) words, followed by the number
// of patched ids before each word (dynamic LDS).
extern __shared__ uint32_t rw_pbits[];

#define RW_PF_SHIFT 30u

#ifdef ZS_WALK_DEBUG
#define RW_T(i)                                                  \
    do {                                                         \
        if (threadIdx.x == 0) {                                  \
            const unsigned long long c_ = wall_clock64();        \
            atomicAdd(&rw_dbg[i], c_ - rw_t0);                   \
            rw_t0 = c_;                                          \
        }                                                        \
    } while (0)
#else
#define RW_T(i) do { } while (0)
#endif

// A value every lane holds equally (read from LDS after a barrier), moved to
// a scalar register so that the compiler branches on it without exec masks.
__device__ __forceinline__ uint32_t rw_uni(uint32_t v) { return __builtin_amdgcn_readfirstlane(v); }
__device__ __forceinline__ float rw_unif(float v) { return __uint_as_float(__builtin_amdgcn_readfirstlane(__float_as_uint(v))); }
// Sum of a u32 over the wave (no overflow check), uniform: pairs, quads,
// eights and rows of 16 by DPP permutations, then the rows by broadcasts;
// lane 63 ends with the total.
__device__ __forceinline__ uint32_t rw_wave_sum(uint32_t v) {
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0xB1, 0xf, 0xf, false);    // quad_perm [1,0,3,2]
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x4E, 0xf, 0xf, false);    // quad_perm [2,3,0,1]
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false);   // row_half_mirror
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x140, 0xf, 0xf, false);   // row_mirror
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);   // row_bcast:15
    v += (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);   // row_bcast:31
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Workgroup barrier that orders LDS accesses only. __syncthreads() also waits
// for every outstanding global load of the calling wave, which would drain the
// loads the tile loops keep in flight ahead of the tile being processed.
__device__ __forceinline__ void rw_bar() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

// Ascending sort of the m <= 256 entries at buf by one wave (called by the 64
// lanes of one wave; no barrier).
template <int E>
__device__ __forceinline__ void rw_wave_sort_e(unsigned long long* buf, uint32_t m) {
    const uint32_t lane = (uint32_t)zs_lane();
    unsigned long long k[E];
#pragma unroll
    for (int e = 0; e < E; e++) k[e] = lane * E + e < m ? buf[lane * E + e] : ~0ull;
    wave_sort_u64_e<E>(k);
#pragma unroll
    for (int e = 0; e < E; e++) if (lane * E + e < m) buf[lane * E + e] = k[e];
}
__device__ __forceinline__ void rw_wave_sort(unsigned long long* buf, uint32_t m) {
    if (m <= 64) rw_wave_sort_e<1>(buf, m);
    else if (m <= 128) rw_wave_sort_e<2>(buf, m);
    else rw_wave_sort_e<4>(buf, m);
}

// ---------------------------------------------------------------------------
// P0: merged patch list. The row's ban / bias / count entries (any number)
// are merged into one entry per patched id, in id order, with the exact
// patched y of the reference's per-token operation sequence: bans first
// (logit_fsm.rs:248-252), then the logit_bias entries in list order, then the
// penalty of the count map (decode_ctrl.rs:107-126). The ids' bitmap and its
// per-word prefix counts (dynamic LDS) give every patched id its rank in the
// list; the list itself is in row scratch (a.pstride entries per row), its
// first ZS_PATCH_LDS entries also in LDS for the row kernel's phases.
// Returns the number of patched ids.
// ---------------------------------------------------------------------------
#define ZS_PATCH_LDS 4096
__device__ __forceinline__ uint32_t rw_rank(uint32_t id, uint32_t words) {
    const uint32_t wd = rw_pbits[id >> 5];
    return rw_pbits[words + (id >> 5)] + __popc(wd & ((1u << (id & 31)) - 1u));
}

__device__ __forceinline__ int rw_patches(const zs_sargs& a, uint32_t r, const zs_row_params& P, uint32_t& has_y, rw_shared& sh,
                                          bool wr = true) {
    const zs_batch& b = a.b;
    const uint32_t t = threadIdx.x, V = b.V;
    const uint32_t words = (V + 31) / 32;
    uint32_t* seen = rw_pbits + 2 * words;   // bias ids met once, and more than once
    uint32_t* dup = rw_pbits + 3 * words;
    const uint32_t ban0 = b.d_ban_off ? b.d_ban_off[r] : 0, ban1 = b.d_ban_off ? b.d_ban_off[r + 1] : 0;
    const uint32_t bi0 = b.d_bias_off ? b.d_bias_off[r] : 0, bi1 = b.d_bias_off ? b.d_bias_off[r + 1] : 0;
    for (uint32_t i = t; i < words; i += RW_NT) {
        rw_pbits[i] = 0u;
        if (bi1 != bi0) { seen[i] = 0u; dup[i] = 0u; }
    }
    uint32_t c0 = b.d_cnt_off ? b.d_cnt_off[r] : 0, c1 = b.d_cnt_off ? b.d_cnt_off[r + 1] : 0;
    if (!zs_penalty_active(P)) c1 = c0;  // counts only matter when penalties are active
    const uint32_t nb = ban1 - ban0, nbi = bi1 - bi0, nc = c1 - c0;
    const uint32_t nsub = (V + ZS_SUB - 1) / ZS_SUB;
    uint32_t* psub = a.p_sub + (size_t)r * (a.max_subs + 1);
    uint32_t* out_id = a.p_id + (size_t)r * a.pstride;
    uint32_t* out_fl = a.p_flags + (size_t)r * a.pstride;
    float* out_y = a.p_y + (size_t)r * a.pstride;
    // entry k: in LDS (ids and flags in sh.pid, y in sh.py) for the list's
    // head, in row scratch past it; the head is copied out at the end
    auto FL = [&](uint32_t k) -> uint32_t { return k < ZS_PATCH_LDS ? sh.pid[k] >> RW_PF_SHIFT : out_fl[k]; };
    auto SET_FL = [&](uint32_t k, uint32_t f) {
        if (k < ZS_PATCH_LDS) sh.pid[k] = (sh.pid[k] & ((1u << RW_PF_SHIFT) - 1u)) | (f << RW_PF_SHIFT);
        else out_fl[k] = f;
    };
    auto Y = [&](uint32_t k) -> float { return k < ZS_PATCH_LDS ? sh.py[k] : out_y[k]; };
    auto SET_Y = [&](uint32_t k, float y) {
        if (k < ZS_PATCH_LDS) sh.py[k] = y;
        else out_y[k] = y;
    };
    __syncthreads();
    // the patched ids, and the bias ids that occur more than once
    for (uint32_t i = t; i < nb + nbi + nc; i += RW_NT) {
        uint32_t id;
        if (i < nb) id = b.d_ban_ids[ban0 + i];
        else if (i < nb + nbi) id = b.d_bias_ids[bi0 + i - nb];
        else id = b.d_cnt_ids[c0 + i - nb - nbi];
        if (id >= V) continue;
        const uint32_t bit = 1u << (id & 31);
        atomicOr(&rw_pbits[id >> 5], bit);
        if (i >= nb && i < nb + nbi && (atomicOr(&seen[id >> 5], bit) & bit)) atomicOr(&dup[id >> 5], bit);
    }
    __syncthreads();
    // per-word prefix counts of the bitmap (words / RW_NT words per thread at most 8)
    uint32_t np;
    {
        const uint32_t per = (words + RW_NT - 1) / RW_NT;
        const uint32_t w0 = t * per;
        uint32_t c = 0;
        for (uint32_t w = w0; w < min(w0 + per, words); w++) c += __popc(rw_pbits[w]);
        uint32_t run = block_excl_scan_u<RW_NT>(c, sh.ru[2], &np);
        for (uint32_t w = w0; w < min(w0 + per, words); w++) {
            rw_pbits[words + w] = run;
            // the list in id order: every patched id with its masked logit
            uint32_t m = rw_pbits[w];
            while (m) {
                const uint32_t id = w * 32 + (uint32_t)__builtin_ctz(m);
                m &= m - 1u;
                float x = b.d_logits[(size_t)r * b.ld + id];
                if ((P.flags & ZS_ROW_MASKED) && b.d_allow_bits && !zs_allowed_bit(b, r, id)) x = -INFINITY;
                if (run < ZS_PATCH_LDS) {
                    sh.pid[run] = id;
                    sh.py[run] = x;
                } else {
                    out_id[run] = id;
                    out_fl[run] = 0u;
                    out_y[run] = x;
                }
                run++;
            }
        }
    }
    np = rw_uni(np);
    __syncthreads();
    // bans (a banned x~ and y are -inf)
    for (uint32_t i = t; i < nb; i += RW_NT) {
        const uint32_t id = b.d_ban_ids[ban0 + i];
        if (id >= V) continue;
        const uint32_t k = rw_rank(id, words);
        SET_FL(k, ZS_PF_BAN);
        SET_Y(k, -INFINITY);
    }
    __syncthreads();
    // logit_bias (decode_ctrl.rs:108-112): an id met once takes its bias in
    // parallel; the entries of an id met more than once are added by one
    // thread in list order
    for (uint32_t i = t; i < nbi; i += RW_NT) {
        const uint32_t id = b.d_bias_ids[bi0 + i];
        if (id >= V || ((dup[id >> 5] >> (id & 31)) & 1u)) continue;
        const uint32_t k = rw_rank(id, words);
        SET_Y(k, Y(k) + b.d_bias_vals[bi0 + i]);
        SET_FL(k, FL(k) | ZS_PF_Y);
    }
    if (t == 0) {
        for (uint32_t i = 0; i < nbi; i++) {
            const uint32_t id = b.d_bias_ids[bi0 + i];
            if (id >= V || !((dup[id >> 5] >> (id & 31)) & 1u)) continue;
            const uint32_t k = rw_rank(id, words);
            SET_Y(k, Y(k) + b.d_bias_vals[bi0 + i]);
            SET_FL(k, FL(k) | ZS_PF_Y);
        }
    }
    __syncthreads();
    // penalty (decode_ctrl.rs:113-125): repeat, then frequency * count + presence
    // (the count map holds each id once)
    for (uint32_t i = t; i < nc; i += RW_NT) {
        const uint32_t id = b.d_cnt_ids[c0 + i];
        if (id >= V) continue;
        const uint32_t k = rw_rank(id, words);
        const uint32_t cnt = b.d_cnt_vals[c0 + i];
        float y = Y(k);
        if (P.repeat != 1.0f) {
            if (y > 0.0f) y = y / P.repeat;
            else y = y * P.repeat;
        }
        float pen_v = __fmul_rn(P.frequency, (float)cnt);
        pen_v = __fadd_rn(pen_v, P.presence);
        y = __fsub_rn(y, pen_v);
        SET_Y(k, y);
        SET_FL(k, FL(k) | ZS_PF_Y);
    }
    __syncthreads();
    // the list's head out to row scratch (the later kernels read it there)
    uint32_t hy = 0;
    for (uint32_t k = t; k < np; k += RW_NT) {
        const uint32_t fl = FL(k);
        hy |= (fl & ZS_PF_Y) ? 1u : 0u;
        if (wr && k < ZS_PATCH_LDS) {
            out_id[k] = sh.pid[k] & ((1u << RW_PF_SHIFT) - 1u);
            out_fl[k] = fl;
            out_y[k] = sh.py[k];
        }
    }
    has_y = block_or_u<RW_NT>(hy, sh.ru[1]);
    if (wr && t == 0) a.p_cnt[r] = np;
    // first patch of every 1024-id sub-chunk (read by the sum, big-row and
    // output kernels): the bitmap's prefix count at the sub-chunk start
    for (uint32_t j = t; wr && j <= nsub; j += RW_NT) psub[j] = j * (ZS_SUB / 32) < words ? rw_pbits[words + j * (ZS_SUB / 32)] : np;
    __syncthreads();
    return (int)np;
}

// ---------------------------------------------------------------------------
// Element access: x~ (observers: mask and bans) and z (sampler: patched y,
// divided by T) of the 4 ids g*RW_G + 4t .. +3.
// ---------------------------------------------------------------------------
struct rw_row {
    const uint32_t* gfl;            // the patch list in row scratch (entries past its LDS head)
    const float* gy;
    const float* row;
    const uint32_t* allow;
    const uint32_t* allow_or_row;   // allow bits, or any readable words when unmasked
    uint32_t V, np, words;
    uint32_t ldm4, wmax;            // last float4 of the row, last readable word
    uint32_t amask;                 // 15 for an unmasked row, else 0
    uint32_t glast;                 // the last tile of the streamed range
    uint32_t vend, gend;            // the streamed range's end: id (its ids >= vend read -inf) and tile
};
struct rw_raw {
    float4 v;
    uint32_t w;   // the allow word holding the 4 ids
    uint32_t pw;  // the patch bitmap word holding them (rows with patches)
};
// A load through a global-address-space pointer (the host pass of the
// compiler only parses device code, and has no such address space).
template <class T>
__device__ __forceinline__ T rw_gload(const T* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return *(const __attribute__((address_space(1))) T*)p;
#else
    return *p;
#endif
}
// Loads of tile g for this thread, as global-memory loads (a generic pointer
// would be loaded with flat instructions, whose completion every LDS wait
// also waits for). Unconditional, from addresses clamped into the row (rows
// are ld >= V floats, ld a multiple of 4) and into the allow bitset, so that
// nothing waits for them before their data is used.
__device__ __forceinline__ rw_raw rw_fetch(const rw_row& R, uint32_t g) {
    const uint32_t idx0 = min(g * RW_G + 4 * threadIdx.x, R.ldm4);
    rw_raw o;
    typedef float rw_f4 __attribute__((ext_vector_type(4)));
    const rw_f4 v = rw_gload(reinterpret_cast<const rw_f4*>(R.row + idx0));
    o.v = make_float4(v.x, v.y, v.z, v.w);
    o.w = rw_gload(R.allow_or_row + min(idx0 >> 5, R.wmax));
    // read with the loads, long before its use
    o.pw = R.np ? rw_pbits[min((g * RW_G + 4 * threadIdx.x) >> 5, R.words - 1)] : 0u;
    return o;
}
// The patched ids among the 4 ids from idx0 (bits of pb): bans set x~ and
// y to -inf, biased or counted ids take their y from the patch list. Their
// rank in the sorted list is the number of bitmap bits before them (per-word
// prefix counts follow the bitmap). GP: the list is longer than its LDS head,
// and ranks past it read the row's copy in global memory (a load that the
// streaming loops must not contain otherwise: the compiler then waits for
// every load in flight after each tile).
template <bool GP>
__device__ __forceinline__ void rw_patch4(const rw_row& R, uint32_t idx0, uint32_t pb, uint32_t wd, float (&x)[4],
                                          float (&y)[4], const rw_shared& sh) {
    uint32_t rank = rw_pbits[R.words + (idx0 >> 5)] + __popc(wd & ((1u << (idx0 & 31)) - 1u));
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if (!((pb >> q) & 1u)) continue;
        uint32_t fl;
        float py;
        if (!GP || rank < ZS_PATCH_LDS) { fl = sh.pid[rank] >> RW_PF_SHIFT; py = sh.py[rank]; }
        else { fl = R.gfl[rank]; py = R.gy[rank]; }
        if (fl & ZS_PF_BAN) { x[q] = -INFINITY; y[q] = -INFINITY; }
        if (fl & ZS_PF_Y) y[q] = py;
        rank++;
    }
}
// x~ (observers: mask and bans) and y (sampler: patched, before the
// temperature) of the 4 ids g*RW_G + 4t .. +3; ids >= V read -inf. Branch
// free but for two uniform tests (the row's last tile, patches in the row)
// and the rare threads holding a patched id.
template <bool GP>
__device__ __forceinline__ void rw_elems(const rw_row& R, uint32_t g, const rw_raw& raw, float (&x)[4], float (&y)[4],
                                         const rw_shared& sh) {
    const uint32_t idx0 = g * RW_G + 4 * threadIdx.x;
    const uint32_t aw = (raw.w >> (idx0 & 31)) | R.amask;   // amask: 15 when unmasked
    x[0] = (aw & 1u) ? raw.v.x : -INFINITY;
    x[1] = (aw & 2u) ? raw.v.y : -INFINITY;
    x[2] = (aw & 4u) ? raw.v.z : -INFINITY;
    x[3] = (aw & 8u) ? raw.v.w : -INFINITY;
    const bool last = g >= R.glast;   // uniform
    if (last) {
#pragma unroll
        for (int q = 0; q < 4; q++) x[q] = idx0 + q < R.vend ? x[q] : -INFINITY;
    }
#pragma unroll
    for (int q = 0; q < 4; q++) y[q] = x[q];
    if (R.np) {
        const uint32_t wd = raw.pw;
        uint32_t pb = (wd >> (idx0 & 31)) & 15u;
        if (last) pb = idx0 < R.vend ? pb : 0u;
        if (pb) rw_patch4<GP>(R, idx0, pb, wd, x, y, sh);
    }
}

// Calls f(g, u, x, y) for the tiles from g_begin up to R.gend in order, in
// groups of four (u = 0..3, a constant in each unrolled copy: per-tile state
// of a group can live in registers indexed by u), with four tiles of loads in
// flight: unrolled by four so that each load stays in its own registers until
// used (copying a register whose load is outstanding waits for every load). f
// returns true (uniformly) to stop; rw_stream then returns that tile's index,
// else R.gend. The last group is padded with tiles past the range (ids >=
// R.vend, read as -inf), which f must treat as neutral. f must not call functions: a call inside the
// loop saves the registers of the loads in flight, which waits for them.
template <bool GP, class F>
__device__ __forceinline__ uint32_t rw_stream(const rw_row& R, const rw_shared& sh, uint32_t g_begin, const F& f) {
    const uint32_t ng = R.gend;
    rw_raw raw[4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        raw[u] = rw_fetch(R, min(g_begin + (uint32_t)u, ng - 1));
        // issued in slot order, as in the loop: the wait before a slot's use
        // then covers only that slot's loads
        __asm__ volatile("" ::: "memory");
    }
    for (uint32_t g0 = g_begin; g0 < ng; g0 += 4) {
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const uint32_t g = g0 + u;
            float x[4], y[4];
            rw_elems<GP>(R, g, raw[u], x, y, sh);
            raw[u] = rw_fetch(R, min(g + 4, ng - 1));
            __asm__ volatile("" ::: "memory");   // keep the loads issued here, ahead of their use
            if (rw_uni(f(g, u, x, y) ? 1u : 0u)) return g;
        }
    }
    return ng;
}

// The elements of one tile (the tile a stream stopped at).
__device__ __forceinline__ void rw_tile(const rw_row& R, const rw_shared& sh, uint32_t g, float (&x)[4], float (&y)[4]) {
    const rw_raw raw = rw_fetch(R, g);
    rw_elems<true>(R, g, raw, x, y, sh);
}

// ---------------------------------------------------------------------------
// Candidate lists (P1). Entries are ((~key) << 32) | id: ascending order is
// key descending, id ascending (Rust's stable descending sort on total_cmp).
// A list admits the elements whose key exceeds its threshold (the key of its
// K-th entry once known); when it holds more than RW_KEEP entries it is
// sorted and cut to its first K, raising the threshold. Elements equal to the
// threshold that arrive later have larger ids than the K entries at or above
// it, so they can never enter the first K.
// ---------------------------------------------------------------------------
struct rw_list {
    unsigned long long* buf;
    uint32_t* cnt;      // [3] per-tile reservation counters (rotating)
    long long* thr;     // admission threshold: keys > thr enter
    uint32_t* flag;     // bit 0: the last compaction cut entries equal to its K-th key
};

// Selection on a list (list 0: observers, 1: sampler): of its first n
// entries, those of ids < idlim are the list's members; the K1 smallest
// members (all of them when fewer) are brought to the front of the buffer in
// ascending order. Returns the number of members. Called by every thread.
//
// An MSB radix selection on the 64-bit entries, 8-bit digits: the digits
// above the first bit where the members' keys differ are skipped; each pass
// histograms one digit of the members that share the bits above it with the
// K1-th smallest, and one wave picks the digit where the count reaches K1. It stops once the members up to and including the chosen digit
// number at most RW_SEL_CAP (always by the last digit: entries are
// distinct); those are gathered to the front and sorted by one wave.
#define RW_SEL_CAP 256
#define RW_SEL_E (RW_BUF / RW_NT)   // list entries per thread
static_assert(RW_BUF % RW_NT == 0, "the list is spread evenly over the threads");
static_assert(RW_PART == ZS_ROW_PART && ZS_OBS_CAND <= RW_PART_S - RW_PART_O && ZS_KS + 1 <= ZS_SMALL_CAP,
              "the split rows' slots hold the lists");

__device__ __noinline__ uint32_t rw_select(int which, uint32_t n, uint32_t K1, uint32_t idlim) {
    rw_shared& sh = rw_sh;
    unsigned long long* buf = which ? sh.u.b.s : sh.u.b.o;
    const uint32_t t = threadIdx.x, lane = (uint32_t)zs_lane(), wid = (uint32_t)zs_wid();
    const unsigned long long NONE = ~0ull;   // no member: ids are below 2^32 - 1
    unsigned long long v[RW_SEL_E];
    uint32_t lo = 0xffffffffu, hi = 0;       // keys (high words) of the members
    uint32_t c = 0;
#pragma unroll
    for (int e = 0; e < RW_SEL_E; e++) {
        const uint32_t i = t + (uint32_t)e * RW_NT;
        v[e] = NONE;
        if (i < n) {
            const unsigned long long w = buf[i];
            if ((uint32_t)w < idlim) v[e] = w;
        }
        const bool mem = v[e] != NONE;
        c += (uint32_t)__popcll(__ballot(mem));
        if (mem) {
            lo = min(lo, (uint32_t)(v[e] >> 32));
            hi = max(hi, (uint32_t)(v[e] >> 32));
        }
    }
    for (int d = 32; d > 0; d >>= 1) {
        lo = min(lo, (uint32_t)__shfl_xor(lo, d, 64));
        hi = max(hi, (uint32_t)__shfl_xor(hi, d, 64));
    }
    if (lane == 0) { sh.sel_mm[0][wid] = c; sh.sel_mm[1][wid] = lo; sh.sel_mm[2][wid] = hi; }
    __syncthreads();
    c = 0; lo = 0xffffffffu; hi = 0;
#pragma unroll
    for (int w = 0; w < RW_NW; w++) {
        c += sh.sel_mm[0][w];
        lo = min(lo, sh.sel_mm[1][w]);
        hi = max(hi, sh.sel_mm[2][w]);
    }
    c = rw_uni(c);
    if (c == 0) return 0;   // every thread read buf before the barrier above
    const uint32_t need = min(c, K1);
    // the selected members: (v >> shift) <= (pre >> shift)
    int shift = 0;
    unsigned long long pre = NONE - 1ull;   // every member (ids < 2^32 - 1)
    if (c > RW_SEL_CAP) {
        lo = rw_uni(lo); hi = rw_uni(hi);
        shift = lo != hi ? 32 + ((31 - __clz(lo ^ hi)) & ~7) : 24;
        pre = ((unsigned long long)lo << 32) & ~((2ull << (shift + 7)) - 1ull);   // the bits above the digit
        uint32_t below = 0;   // members with a smaller prefix
        if (t < 256) sh.sel_hist[0][t] = 0;
        for (int pass = 0;; pass ^= 1) {
            // histogram pass-parity buffer; the other one is cleared for the
            // next pass (its last reader finished before this pass's first barrier)
            if (t < 256) sh.sel_hist[pass ^ 1][t] = 0;
            __syncthreads();
            const int up = shift + 8;
#pragma unroll
            for (int e = 0; e < RW_SEL_E; e++) {
                const bool in = v[e] != NONE && (up >= 64 || (v[e] >> up) == (pre >> up));
                const uint32_t dg = (uint32_t)(v[e] >> shift) & 255u;
                if (in) atomicAdd(&sh.sel_hist[pass][dg], 1u);
            }
            __syncthreads();
            if (wid == 0) {
                // the digit where the running count reaches need
                uint32_t h[4], s4 = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) { h[q] = sh.sel_hist[pass][lane * 4 + q]; s4 += h[q]; }
                const uint32_t inc = wave_incl_scan_u(s4);
                const unsigned long long hit = __ballot(below + inc >= need);
                const uint32_t L = (uint32_t)__ffsll((long long)hit) - 1u;   // one exists
                if (lane == L) {
                    uint32_t run = below + inc - s4;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        if (run + h[q] >= need) {
                            sh.sel_mm[0][0] = lane * 4 + q;
                            sh.sel_mm[1][0] = run;
                            sh.sel_mm[2][0] = h[q];
                            break;
                        }
                        run += h[q];
                    }
                }
            }
            __syncthreads();
            const uint32_t dg = rw_uni(sh.sel_mm[0][0]), cb = rw_uni(sh.sel_mm[2][0]);
            below = rw_uni(sh.sel_mm[1][0]);
            pre |= (unsigned long long)dg << shift;
            if (below + cb <= RW_SEL_CAP || shift == 0) break;
            shift -= 8;
        }
    }
    // gather the selected members to the front (every read of buf is done)
    if (t == 0) sh.sel_n = 0;
    __syncthreads();
#pragma unroll
    for (int e = 0; e < RW_SEL_E; e++) {
        if (v[e] == NONE || (v[e] >> shift) > (pre >> shift)) continue;
        buf[atomicAdd(&sh.sel_n, 1u)] = v[e];
    }
    __syncthreads();
    const uint32_t m = rw_uni(sh.sel_n);
    if (wid == 0) rw_wave_sort(buf, m);
    __syncthreads();
    return c;
}

// Cuts a list to its K smallest members (rw_select); the K-th key becomes the
// threshold (below K members: every id is admitted). Also records the value
// of the threshold, whether entries equal to the K-th key were cut, and the
// largest value cut (into *cutmax).
// Returns the new entry count. Called by every thread.
__device__ uint32_t rw_compact(int which, const rw_list& L, uint32_t n, uint32_t K, uint32_t idlim, float* fthr,
                               float* cutmax) {
    const uint32_t c = rw_select(which, n, K + 1, idlim);
    const uint32_t keep = min(c, K);
    if (threadIdx.x == 0) {
        if (c >= K) {
            const uint32_t kk = ~(uint32_t)(L.buf[K - 1] >> 32);
            *L.thr = (long long)kk;
            *fthr = zs_key_to_float(kk);
            *L.flag = (c > K && ~(uint32_t)(L.buf[K] >> 32) == kk) ? 1u : 0u;
            if (c > K) *cutmax = fmaxf(*cutmax, zs_key_to_float(~(uint32_t)(L.buf[K] >> 32)));
        } else {
            *L.thr = -1;
            *fthr = -INFINITY;
            *L.flag = 0u;
        }
    }
    __syncthreads();
    return keep;
}

// Writes the admitted elements (bit q of m = element q: key kk[q], id idx0 +
// q) at base + their reservation on counter ctr; an element whose place is
// past the buffer is not written and its tile is reported in *ovf (the lowest
// such tile is streamed again after a compaction).
__device__ __forceinline__ void rw_admit(const rw_list& L, uint32_t* ctr, uint32_t base, uint32_t m,
                                         const uint32_t (&kk)[4], uint32_t idx0, uint32_t g, uint32_t* ovf) {
    const uint32_t n = __popc(m);
    uint32_t p = base + atomicAdd(ctr, n);
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if (!((m >> q) & 1u)) continue;
        if (p < RW_BUF) L.buf[p] = ((unsigned long long)(~kk[q]) << 32) | (idx0 + q);
        else atomicMin(ovf, g);
        p++;
    }
}

// Row scratch of a masked row's gathered values, 16-byte aligned.
__device__ __forceinline__ float* rw_scratch(const zs_sargs& a, uint32_t r) {
    float* cx = a.gath + (size_t)r * (2 * (size_t)a.max_vocab + 16);
    return cx + ((4u - (uint32_t)((reinterpret_cast<uintptr_t>(cx) >> 2) & 3u)) & 3u);
}

// A masked row's allowed ids in index order, with their x~ (cx) and y (cy)
// written to row scratch: the sums then run over these values only (a
// masked id's term is zero, which leaves a running sum unchanged). cx, cy
// hold round_up(n, 4) values each (the tail padded with -inf); cy = cx +
// round_up(n, 4); the ids follow at cy + round_up(n, 4). Returns n, or 0
// when no id, more than RW_BUF ids or more than a quarter of the row is
// allowed (then the sums run over the whole row with its allow bits: each
// thread's loop over its allowed ids, with a dependent load per id, took 29 us
// on rows with tens of thousands of them, more than P1's whole stream saves).
// Uniform.
__device__ __noinline__ uint32_t rw_gather_allowed(const float* row, const uint32_t* allow, uint32_t V, uint32_t np,
                                                   float* cx, const uint32_t* gfl, const float* gy) {
    rw_shared& sh = rw_sh;
    const uint32_t t = threadIdx.x, words = (V + 31) / 32;
    const uint32_t per = (words + RW_NT - 1) / RW_NT, w0 = t * per, w1 = min(w0 + per, words);
    auto word = [&](uint32_t w) {
        uint32_t a = allow[w];
        if (w == words - 1 && (V & 31)) a &= (1u << (V & 31)) - 1u;
        return a;
    };
    uint32_t c = 0;
    for (uint32_t w = w0; w < w1; w++) c += __popc(word(w));
    uint32_t n;
    uint32_t pos = block_excl_scan_u<RW_NT>(c, sh.ru[4], &n);
    n = rw_uni(n);
    if (n == 0 || n > RW_BUF || n > V / 4 || V < 16) return 0;   // V >= 16: 3 round_up(n, 4) + 3 values fit 2 V
    const uint32_t n4 = (n + 3) & ~3u;
    float* cy = cx + n4;
    for (uint32_t w = w0; w < w1; w++) {
        uint32_t a = word(w);
        while (a) {
            const uint32_t id = w * 32 + (uint32_t)__builtin_ctz(a);
            a &= a - 1u;
            float x = row[id], y = x;
            if (np) {
                const uint32_t wd = rw_pbits[id >> 5];
                if ((wd >> (id & 31)) & 1u) {
                    const uint32_t rank = rw_pbits[words + (id >> 5)] + __popc(wd & ((1u << (id & 31)) - 1u));
                    const uint32_t fl = rank < ZS_PATCH_LDS ? sh.pid[rank] >> RW_PF_SHIFT : gfl[rank];
                    if (fl & ZS_PF_BAN) { x = -INFINITY; y = -INFINITY; }
                    if (fl & ZS_PF_Y) y = rank < ZS_PATCH_LDS ? sh.py[rank] : gy[rank];
                }
            }
            cx[pos] = x;
            cy[pos] = y;
            reinterpret_cast<uint32_t*>(cy + n4)[pos] = id;
            pos++;
        }
    }
    if (t < n4 - n) { cx[n + t] = -INFINITY; cy[n + t] = -INFINITY; }
    __syncthreads();
    return n;
}

// Exact sampling of a small survivor set by wave 0 (token to sh.tok).
__device__ __noinline__ void rw_small(uint64_t seed, uint64_t counter, uint32_t V, const zs_row_params& P, uint32_t nsv,
                                      float zmax, rw_shared& sh) {
    const uint32_t tk = nsv <= 64 ? small_path_wave<1>(seed, counter, V, P, nsv, zmax, sh.sval, sh.sidx)
                                  : small_path_wave<ZS_SMALL_CAP / 64>(seed, counter, V, P, nsv, zmax, sh.sval, sh.sidx);
    if (threadIdx.x == 0) sh.tok = tk;
}

// The row of the j-th row workgroup: the unmasked rows in index order, then
// the masked ones. Uniform.
__device__ __forceinline__ uint32_t rw_block_row(const zs_batch& b, uint32_t j) {
    if (!b.d_allow_bits || b.B > 4 * RW_NT) return j;
    rw_shared& sh = rw_sh;
    const uint32_t t = threadIdx.x, lane = (uint32_t)zs_lane(), wid = (uint32_t)zs_wid();
    const uint32_t nchunk = (b.B + RW_NT - 1) / RW_NT;
    uint32_t rank[4], um = 0;      // rank among the rows of its kind; bit c: unmasked
    uint32_t carry = 0;            // unmasked rows in the chunks before
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) {
        rank[c] = 0;
        if (c >= nchunk) continue;
        const uint32_t i = c * RW_NT + t;
        const bool in = i < b.B;
        const bool u = in && !(b.d_params[i].flags & ZS_ROW_MASKED);
        const unsigned long long m = __ballot(u);
        if (lane == 0) sh.sel_mm[0][wid] = (uint32_t)__popcll(m);
        __syncthreads();
        uint32_t before = carry, tot = 0;
#pragma unroll
        for (int w = 0; w < RW_NW; w++) {
            const uint32_t k = sh.sel_mm[0][w];
            before += (uint32_t)w < wid ? k : 0u;
            tot += k;
        }
        __syncthreads();
        before += (uint32_t)__popcll(m & ((1ull << lane) - 1ull));
        rank[c] = u ? before : i - before;   // masked: rows before it minus unmasked before it
        um |= u ? (1u << c) : 0u;
        carry += tot;
    }
    const uint32_t nu = carry;
    if (t == 0) sh.sel_n = j;   // fallback (not reached: every j < B has a row)
    __syncthreads();
#pragma unroll
    for (uint32_t c = 0; c < 4; c++) {
        const uint32_t i = c * RW_NT + t;
        if (c >= nchunk || i >= b.B) continue;
        const uint32_t pos = ((um >> c) & 1u) ? rank[c] : nu + rank[c];
        if (pos == j) sh.sel_n = i;
    }
    __syncthreads();
    const uint32_t r = rw_uni(sh.sel_n);
    __syncthreads();
    return r;
}

// ---------------------------------------------------------------------------
// zs_k_row
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(RW_NT) void zs_k_row(zs_sargs a) {
    const zs_batch& b = a.b;
    // with a.row_split, workgroups B .. 2B - 1 take the second half of their
    // row's stream (below)
    const uint32_t half = (a.row_split && blockIdx.x >= b.B) ? 1u : 0u;
    const uint32_t r = rw_block_row(b, blockIdx.x - half * b.B);
    const uint32_t t = threadIdx.x;
    const uint32_t V = b.V;
    rw_shared& sh = rw_sh;
    __shared__ uint32_t cnt_o[3], cnt_s[3], flag_o, flag_s;
    __shared__ long long thr_o, thr_s;
    const zs_row_params P = b.d_params[r];
    zs_row_state& st = a.rst[r];
    const float T = P.temperature;
    const bool want_lp = (P.flags & ZS_ROW_LOGPROBS) != 0;
    const bool want_unc = (P.flags & ZS_ROW_UNCERTAINTY) != 0;
    const bool want_obs = want_lp || want_unc;
#ifdef ZS_WALK_DEBUG
    unsigned long long rw_t0 = wall_clock64();
#endif
    const bool greedy = T <= 0.0f;
    const bool tinf = T == INFINITY;   // y / inf is NaN for y = +-inf: checked per element
    const uint32_t* allow = ((P.flags & ZS_ROW_MASKED) && b.d_allow_bits) ? b.d_allow_bits + (size_t)r * b.allow_words
                                                                          : nullptr;
    // A row that streams the whole row (not a masked row taking its lists from
    // at most RW_BUF gathered ids) may split the stream over two workgroups
    // when the batch leaves CUs free (a.row_split), unless its patch list may
    // pass the LDS head (both workgroups build it). Both halves decide alike.
    const uint32_t ngt = (V + RW_G - 1) / RW_G;
    bool split = false;
    if (a.row_split && ngt >= 8) {
        const uint32_t nb = b.d_ban_off ? b.d_ban_off[r + 1] - b.d_ban_off[r] : 0u;
        const uint32_t nbi = b.d_bias_off ? b.d_bias_off[r + 1] - b.d_bias_off[r] : 0u;
        const uint32_t nc = (b.d_cnt_off && zs_penalty_active(P)) ? b.d_cnt_off[r + 1] - b.d_cnt_off[r] : 0u;
        if (nb + nbi + nc <= ZS_PATCH_LDS) {
            if (!allow || greedy || tinf) {
                split = true;
            } else {
                const uint32_t words = (V + 31) / 32;
                uint32_t c = 0;
                for (uint32_t w = t; w < words; w += RW_NT) {
                    uint32_t aw = allow[w];
                    if (w == words - 1 && (V & 31)) aw &= (1u << (V & 31)) - 1u;
                    c += (uint32_t)__popc(aw);
                }
                split = rw_uni(block_sum_u<RW_NT>(c, sh.ru[4])) > RW_BUF;
            }
        }
    }
    if (half && !split) return;

    // ---------------- P0: patches (the second half builds its own LDS copy
    // only: the first writes the row's list out)
    uint32_t has_y = 0;
    const int np = rw_patches(a, r, P, has_y, sh, half == 0);
    RW_T(0);
    rw_row R;
    R.gfl = a.p_flags + (size_t)r * a.pstride;
    R.gy = a.p_y + (size_t)r * a.pstride;
    R.row = b.d_logits + (size_t)r * b.ld;
    R.allow = allow;
    R.V = V;
    R.np = rw_uni((uint32_t)np);
    R.words = (V + 31) / 32;
    R.ldm4 = (uint32_t)min((uint64_t)b.ld - 4, (uint64_t)0xfffffff0u);
    R.allow_or_row = R.allow ? R.allow : reinterpret_cast<const uint32_t*>(R.row);
    R.wmax = R.allow ? R.words - 1 : R.ldm4;
    R.amask = R.allow ? 0u : 15u;
    // the streamed range: the whole row, or this workgroup's half
    const uint32_t gmid = ngt / 2;
    const uint32_t gbeg = (split && half) ? gmid : 0u;
    R.gend = (split && !half) ? gmid : ngt;
    R.vend = R.gend == ngt ? V : R.gend * RW_G;
    R.glast = (R.vend - 1) / RW_G;

    // ---------------- P1: statistics and candidate lists
    // The sampler's z = y / T (sampler.rs:47-51) is not formed per element
    // here: division by T > 0 is monotone, so the maximum, the order and the
    // top-k of z follow from those of y (ties created by the rounding are
    // checked when the threshold is set).
    const bool has_topk = P.top_k > 0 && P.top_k < V;
    // sampler list: 1 = top-k by y (k <= ZS_KS), 2 = every y > -inf (the
    // small-survivor check when no top-k applies), 0 = none
    const uint32_t smode = greedy ? 0u : (has_topk ? (P.top_k <= ZS_KS ? 1u : 0u) : 2u);
    const uint32_t Ks = smode == 1 ? P.top_k : 0u;
    const uint32_t Ko = want_obs ? (ZS_OBS_CAND < V ? ZS_OBS_CAND : V) : 0u;
    rw_list LO, LS;
    LO.buf = sh.u.b.o; LO.cnt = cnt_o; LO.thr = &thr_o; LO.flag = &flag_o;
    LS.buf = sh.u.b.s; LS.cnt = cnt_s; LS.thr = &thr_s; LS.flag = &flag_s;
    if (t < 3) { cnt_o[t] = 0; cnt_s[t] = 0; }
    if (t == 0) { thr_o = -1; thr_s = -1; flag_o = 0; flag_s = 0; }
    float omax = -INFINITY, ymax = -INFINITY;
    uint32_t fl = 0;                // ZS_CF_OBS_NAN, ZS_CF_Z_NAN
    float rejf = -INFINITY;         // largest y turned away from the top-k list
    int last_nan = -1;
    unsigned long long gbest = 0;   // greedy: (key << 32) | (id + 1); ties -> larger id
    uint32_t n_o = 0, n_s = 0;      // entries in the lists (uniform)
    bool s_over = false;            // smode 2: more than ZS_SMALL_CAP values above -inf
    __syncthreads();
    // keys of one element set (observers: -0 and +0 share one key, as equal
    // logprobs rank by id, logprobs.rs:41-51)
    auto keys = [&](const float (&x)[4], const float (&y)[4], uint32_t (&kx)[4], uint32_t (&ky)[4]) {
#pragma unroll
        for (int q = 0; q < 4; q++) {
            kx[q] = zs_total_key(x[q] + 0.0f);
            ky[q] = zs_total_key(y[q]);
        }
    };
    // The lists are synchronised once per group of four tiles: admissions
    // reserve places with a counter slot that rotates over three groups, so a
    // single barrier per group separates its use, its read and its reset.
    uint32_t grp = 0, lastslot = 0;
    bool thr_init = false, p1stop = false;
    if (t < 3) sh.ovf[t] = 0xffffffffu;
    if (t == 0) {
        sh.fthr[0] = sh.fthr[1] = -INFINITY;
        sh.fcut[0] = sh.fcut[1] = -INFINITY;
        sh.inf_lim = 0xffffffffu;
    }
    __syncthreads();
    // A masked row with at most RW_BUF allowed ids (every other x~ and y is
    // -inf) takes its statistics and lists from the allowed ids alone,
    // gathered in index order to row scratch (which the sums reuse): the
    // lists then hold every allowed id (observers) and every y above -inf
    // (sampler), of which the selections take the same first entries as from
    // the whole row. Not for greedy rows (the last maximal element may be a
    // masked -inf), T = inf (a masked y / T is NaN) or rows with fewer than
    // Ko finite x~ (their observers' list ends with -inf ids of the whole
    // row).
    // (the gathered count and whether the gather ran are kept in LDS: few
    // values stay live across the stream below)
    bool gath = false;
    if (t == 0) { sh.g_n = 0; sh.g_done = 0; }
    if (R.allow && !greedy && !tinf && !split) {
        const float* gcx = rw_scratch(a, r);
        const uint32_t gn = rw_gather_allowed(R.row, R.allow, V, R.np, rw_scratch(a, r), R.gfl, R.gy);
        if (t == 0) { sh.g_n = gn; sh.g_done = 1; }
        if (gn && gn <= RW_BUF) {
            uint32_t nf = 0;
            for (uint32_t i = t; i < gn; i += RW_NT) nf += gcx[i] > -INFINITY ? 1u : 0u;
            nf = block_sum_u<RW_NT>(nf, sh.ru[4]);
            gath = rw_uni(nf) >= Ko;
        }
    }
    RW_T(1);
    uint32_t g = gbeg;
    const uint32_t ng = gath ? 0u : R.gend;
    const uint32_t Vend = R.vend;
    // the admission thresholds in scalar registers: they change only where
    // the lists are set up (first tile) and compacted (outside the stream)
    float r_tfo = -INFINITY, r_tfs = -INFINITY;
    bool r_allo = true, r_alls = true;
    uint32_t r_ilim = 0xffffffffu;
    auto load_thr = [&]() {
        r_tfo = rw_unif(sh.fthr[0]);
        r_tfs = rw_unif(sh.fthr[1]);
        r_allo = rw_uni(thr_o < 0 ? 1u : 0u) != 0u;
        r_alls = rw_uni(thr_s < 0 ? 1u : 0u) != 0u;
        r_ilim = rw_uni(sh.inf_lim);
    };
    if (gath) {
        const float* gcx = rw_scratch(a, r);
        const uint32_t gn = rw_uni(sh.g_n);
        const uint32_t gn4 = (gn + 3) & ~3u;
        const float* gy = gcx + gn4;
        const uint32_t* gid = reinterpret_cast<const uint32_t*>(gy + gn4);
        for (uint32_t i = t; i < gn; i += RW_NT) {
            const float x = gcx[i], y = gy[i];
            const uint32_t id = gid[i];
            omax = fmaxf(omax, x);
            ymax = fmaxf(ymax, y);
            if (x != x) fl |= ZS_CF_OBS_NAN;
            if (y != y) {
                fl |= ZS_CF_Z_NAN;
                last_nan = max(last_nan, (int)id);
            }
            if (Ko) LO.buf[i] = ((unsigned long long)(~zs_total_key(x + 0.0f)) << 32) | id;
            if (smode != 0 && y > -INFINITY) {
                const uint32_t p = atomicAdd(&cnt_s[0], 1u);
                if (smode == 1 || p < ZS_SMALL_CAP) LS.buf[p] = ((unsigned long long)(~zs_total_key(y)) << 32) | id;
            }
        }
        __syncthreads();
        n_o = Ko ? gn : 0u;
        n_s = rw_uni(cnt_s[0]);
        if (smode == 2 && n_s > ZS_SMALL_CAP) s_over = true;
    }
    while (g < ng) {
        auto tile = [&](uint32_t g, int u, const float (&x)[4], const float (&y)[4]) {
            const uint32_t idx0 = g * RW_G + 4 * t;
            // branch-free statistics (ids >= V read -inf: neutral here)
            omax = fmaxf(omax, fmaxf(fmaxf(x[0], x[1]), fmaxf(x[2], x[3])));
            ymax = fmaxf(ymax, fmaxf(fmaxf(y[0], y[1]), fmaxf(y[2], y[3])));
            uint32_t nx = 0, ny = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                nx |= (x[q] != x[q]) ? 1u : 0u;
                ny |= (y[q] != y[q]) ? (1u << q) : 0u;
            }
            if (nx) fl |= ZS_CF_OBS_NAN;
            if (ny) {
                fl |= ZS_CF_Z_NAN;
                last_nan = max(last_nan, (int)(idx0 + 31 - __clz(ny)));
            }
            // valid ids of the thread (the last tile only is partial)
            const uint32_t vm = idx0 + 4 <= Vend ? 15u : (idx0 >= Vend ? 0u : (1u << (Vend - idx0)) - 1u);
            if (tinf) {
                // y / inf is NaN for a real y = +-inf (ids past the range read
                // -inf and are no elements)
#pragma unroll
                for (int q = 0; q < 4; q++)
                    if (((vm >> q) & 1u) && (y[q] == INFINITY || y[q] == -INFINITY)) fl |= ZS_CF_Z_NAN;
            }
            if (greedy) {
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    if (y[q] != y[q] || idx0 + q >= Vend) continue;
                    // -0.0 and +0.0 compare equal in the reference (partial_cmp)
                    const uint32_t k = zs_total_key(y[q] == 0.0f ? 0.0f : y[q]);
                    const unsigned long long c = ((unsigned long long)k << 32) | (idx0 + q + 1);
                    gbest = c > gbest ? c : gbest;
                }
            }
            if (!thr_init) {
                // initial thresholds (first tile): in every wave the c-th largest
                // thread maximum has at least c elements of that wave at or above
                // it, so the smallest of the waves' values, with c = ceil(K / 16),
                // has at least K elements of this tile at or above it (ids >= V
                // hold key 0)
                thr_init = true;
                if (Ko || Ks) {
                    uint32_t kx[4], ky[4];
                    keys(x, y, kx, ky);
                    uint32_t mo = 0, ms = 0;
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        if (!((vm >> q) & 1u)) continue;
                        mo = max(mo, kx[q]);
                        ms = max(ms, ky[q]);
                    }
                    const uint32_t so = wave_sort_u32(mo), ss = wave_sort_u32(ms);
                    const int co = max((int)((Ko + RW_NW - 1) / RW_NW), 1), cs = max((int)((Ks + RW_NW - 1) / RW_NW), 1);
                    const uint32_t wo = __shfl(so, 64 - co, 64), ws = __shfl(ss, 64 - cs, 64);
                    // observers: -inf values rank by id, so once this tile holds
                    // Ko of them, a -inf of a larger id than the Ko-th can never
                    // be among the first Ko (masked rows are mostly -inf)
                    uint32_t minf = 0;
#pragma unroll
                    for (int q = 0; q < 4; q++) minf |= (((vm >> q) & 1u) && x[q] == -INFINITY) ? (1u << q) : 0u;
                    const uint32_t ninf = (uint32_t)__popc(minf), winf = wave_incl_scan_u(ninf);
                    if (zs_lane() == 63) sh.ru[4][zs_wid()] = winf;
                    if (zs_lane() == 0) { sh.ru[2][zs_wid()] = wo; sh.ru[3][zs_wid()] = ws; }
                    rw_bar();
                    uint32_t a0 = 0xffffffffu, a1 = 0xffffffffu, ibefore = 0;
#pragma unroll
                    for (int w = 0; w < RW_NW; w++) {
                        a0 = min(a0, sh.ru[2][w]); a1 = min(a1, sh.ru[3][w]);
                        ibefore += (uint32_t)w < (uint32_t)zs_wid() ? sh.ru[4][w] : 0u;
                    }
                    ibefore += winf - ninf;
                    if (Ko && ibefore < Ko && Ko <= ibefore + ninf) {
                        // the (Ko - ibefore)-th set bit of minf
                        uint32_t mm = minf;
                        for (uint32_t k = Ko - ibefore; k > 1; k--) mm &= mm - 1u;
                        sh.inf_lim = idx0 + (uint32_t)(__ffs(mm) - 1);
                    }
                    rw_bar();
                    if (t == 0) {
                        // observers: a bound at or below the key of -inf admits
                        // every id (equal -inf logprobs rank by id). Sampler:
                        // the values above -inf (a k-th value of -inf makes
                        // every finite value a survivor; -inf ids never are)
                        const uint32_t kmin = zs_total_key(-INFINITY);
                        thr_o = a0 > kmin ? (long long)a0 - 1 : -1;
                        thr_s = a1 > kmin ? (long long)a1 - 1 : (long long)kmin;
                        sh.fthr[0] = a0 > kmin ? zs_key_to_float(a0 - 1u) : -INFINITY;
                        sh.fthr[1] = a1 > kmin ? zs_key_to_float(a1 - 1u) : -INFINITY;
                    }
                    rw_bar();
                    load_thr();
                }
            }
            // admissions, compared as values: a key above the threshold key is a
            // value above the threshold value, -0 and +0 aside (they compare
            // equal: only the value of the k-th entry matters, and observers
            // rank equal values by id) and NaN aside (a NaN row takes no list);
            // a threshold below every key (-1) admits every valid id
            const uint32_t slot = grp % 3;
            uint32_t po = 0, ps = 0;
            {
                const float tfo = r_tfo, tfs = r_tfs;
                const bool allo = r_allo, alls = r_alls;
                const uint32_t ilim = r_ilim;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    po |= ((x[q] > tfo || allo) && (x[q] != -INFINITY || idx0 + q <= ilim)) ? (1u << q) : 0u;
                    if (smode == 1) {
                        const bool in = y[q] > tfs || alls;
                        ps |= in ? (1u << q) : 0u;
                        if (!in) rejf = fmaxf(rejf, y[q]);
                    }
                }
                po &= Ko ? vm : 0u;
                ps &= vm;
            }
            if (smode == 2 && !s_over) {
                // every value above -inf: one reservation per wave (places past
                // ZS_SMALL_CAP are not written; the count ends the list)
                uint32_t m = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) m |= (y[q] > -INFINITY) ? (1u << q) : 0u;
                m &= vm;
                const uint32_t c = __popc(m);
                uint32_t inc = c;
                for (int d = 1; d < 64; d <<= 1) {
                    const uint32_t o = __shfl_up(inc, d, 64);
                    if (zs_lane() >= d) inc += o;
                }
                const uint32_t wtot = __shfl(inc, 63, 64);
                uint32_t base = 0;
                if (wtot) {
                    if (zs_lane() == 0) base = atomicAdd(&cnt_s[slot], wtot);
                    base = __shfl(base, 0, 64);
                }
                uint32_t p = n_s + base + inc - c;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    if (!((m >> q) & 1u)) continue;
                    if (p < ZS_SMALL_CAP) LS.buf[p] = ((unsigned long long)(~zs_total_key(y[q])) << 32) | (idx0 + q);
                    p++;
                }
            }
            if (po | ps) {
                uint32_t kx[4], ky[4];
                keys(x, y, kx, ky);
                if (po) rw_admit(LO, &cnt_o[slot], n_o, po, kx, idx0, g, &sh.ovf[slot]);
                if (ps) rw_admit(LS, &cnt_s[slot], n_s, ps, ky, idx0, g, &sh.ovf[slot]);
            }
            if (u != 3) return false;
            // end of the group: counts, overflow, compaction need
            if (t == 0) {
                const uint32_t nx = (grp + 1) % 3;
                cnt_o[nx] = 0;
                cnt_s[nx] = 0;
                sh.ovf[nx] = 0xffffffffu;
            }
            rw_bar();
            n_o += rw_uni(cnt_o[slot]);
            n_s += rw_uni(cnt_s[slot]);
            const uint32_t ovf = rw_uni(sh.ovf[slot]);
            lastslot = slot;
            grp++;
            // more than ZS_SMALL_CAP finite values: the small-survivor list
            // is dropped (its count ended it; nothing to compact)
            if (smode == 2 && !s_over && n_s > ZS_SMALL_CAP) s_over = true;
            p1stop = ovf != 0xffffffffu || n_o > RW_KEEP || (smode == 1 && n_s > RW_KEEP);
            return p1stop;
        };
        // (rows with more patches than the LDS head take the loop that can
        // read the rest from global memory)
        load_thr();
        g = R.np > ZS_PATCH_LDS ? rw_stream<true>(R, sh, g, tile) : rw_stream<false>(R, sh, g, tile);
        if (!p1stop) break;
        p1stop = false;
        // compactions (rare): a list past RW_KEEP is cut to its first K. After
        // an overflow, the entries of the tiles from the first one that lost
        // an entry are dropped; that tile is admitted again element by element
        // with compactions as needed (every round places at least
        // RW_BUF - RW_KEEP entries), and the stream resumes after it (the
        // statistics are maxima and flags, which a second visit does not
        // change).
        __syncthreads();
        const uint32_t ovf = sh.ovf[lastslot];
        const uint32_t idlim = ovf != 0xffffffffu ? ovf * RW_G : 0xffffffffu;
        if (smode == 2 && !s_over && (n_s > ZS_SMALL_CAP || ovf != 0xffffffffu)) s_over = true;
        auto compact_lists = [&](uint32_t lim) {
            if (Ko && (n_o > RW_KEEP || lim != 0xffffffffu))
                n_o = rw_compact(0, LO, min(n_o, (uint32_t)RW_BUF), Ko, lim, &sh.fthr[0], &sh.fcut[0]);
            if (smode == 1 && (n_s > RW_KEEP || lim != 0xffffffffu)) {
                n_s = rw_compact(1, LS, min(n_s, (uint32_t)RW_BUF), Ks, lim, &sh.fthr[1], &sh.fcut[1]);
                rejf = fmaxf(rejf, sh.fcut[1]);   // entries cut count as turned away
            }
        };
        compact_lists(idlim);
        if (t < 3) { cnt_o[t] = 0; cnt_s[t] = 0; sh.ovf[t] = 0xffffffffu; }
        __syncthreads();
        if (ovf != 0xffffffffu && ovf < ng) {
            float x[4], y[4];
            rw_tile(R, sh, ovf, x, y);
            uint32_t kx[4], ky[4];
            keys(x, y, kx, ky);
            const uint32_t idx0 = ovf * RW_G + 4 * t;
            const uint32_t vm = idx0 + 4 <= Vend ? 15u : (idx0 >= Vend ? 0u : (1u << (Vend - idx0)) - 1u);
            uint32_t po = 0, ps = 0;
            for (int round = 0; ; round++) {
                // the tile's elements above the current thresholds, minus those placed
                const float tfo = sh.fthr[0], tfs = sh.fthr[1];
                const bool allo = thr_o < 0, alls = thr_s < 0;
                uint32_t wo = 0, ws = 0;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    wo |= ((x[q] > tfo || allo) && (x[q] != -INFINITY || idx0 + q <= sh.inf_lim)) ? (1u << q) : 0u;
                    if (smode == 1) {
                        const bool in = y[q] > tfs || alls;
                        ws |= in ? (1u << q) : 0u;
                        if (!in) rejf = fmaxf(rejf, y[q]);
                    }
                }
                wo &= Ko ? vm : 0u;
                ws &= vm;
                if (round == 0) { po = wo; ps = ws; }
                else { po &= wo; ps &= ws; }
                // place what fits (the rest stays in po / ps)
                uint32_t lo = 0, ls = 0;
                {
                    const uint32_t n1 = __popc(po), n2 = __popc(ps);
                    uint32_t p1 = n_o + (n1 ? atomicAdd(&cnt_o[0], n1) : 0u);
                    uint32_t p2 = n_s + (n2 ? atomicAdd(&cnt_s[0], n2) : 0u);
#pragma unroll
                    for (int q = 0; q < 4; q++) {
                        if ((po >> q) & 1u) {
                            if (p1 < RW_BUF) LO.buf[p1] = ((unsigned long long)(~kx[q]) << 32) | (idx0 + q);
                            else lo |= 1u << q;
                            p1++;
                        }
                        if ((ps >> q) & 1u) {
                            if (p2 < RW_BUF) LS.buf[p2] = ((unsigned long long)(~ky[q]) << 32) | (idx0 + q);
                            else ls |= 1u << q;
                            p2++;
                        }
                    }
                }
                po = lo;
                ps = ls;
                __syncthreads();
                n_o = min(n_o + cnt_o[0], (uint32_t)RW_BUF);
                n_s = min(n_s + cnt_s[0], (uint32_t)RW_BUF);
                const bool more = __syncthreads_or((po | ps) != 0u);
                if (t == 0) { cnt_o[0] = 0; cnt_s[0] = 0; }
                if (!more) break;
                compact_lists(0xffffffffu);
                __syncthreads();
            }
            compact_lists(0xffffffffu);   // back below RW_KEEP for the stream
            __syncthreads();
            grp = 0;
            g = ovf + 1;
        } else {
            grp = 0;
            g = g + 1;
        }
    }
    RW_T(2);
    // ---- row statistics (one workgroup reduction)
    {
        for (int d = 32; d > 0; d >>= 1) {
            omax = fmaxf(omax, __shfl_xor(omax, d, 64));
            ymax = fmaxf(ymax, __shfl_xor(ymax, d, 64));
            fl |= __shfl_xor(fl, d, 64);
            last_nan = max(last_nan, __shfl_xor(last_nan, d, 64));
            rejf = fmaxf(rejf, __shfl_xor(rejf, d, 64));
            const unsigned long long og = __shfl_xor(gbest, d, 64);
            gbest = og > gbest ? og : gbest;
        }
        if (zs_lane() == 0) {
            sh.rf[0][zs_wid()] = omax; sh.rf[1][zs_wid()] = ymax;
            sh.ru[0][zs_wid()] = fl; sh.rf[2][zs_wid()] = rejf;
            sh.ru[2][zs_wid()] = (uint32_t)last_nan;
            sh.rl[zs_wid()] = gbest;
        }
        __syncthreads();
        omax = -INFINITY; ymax = -INFINITY; fl = 0; rejf = -INFINITY; last_nan = -1; gbest = 0;
#pragma unroll
        for (int w = 0; w < RW_NW; w++) {
            omax = fmaxf(omax, sh.rf[0][w]); ymax = fmaxf(ymax, sh.rf[1][w]);
            fl |= sh.ru[0][w]; rejf = fmaxf(rejf, sh.rf[2][w]);
            last_nan = max(last_nan, (int)sh.ru[2][w]);
            gbest = sh.rl[w] > gbest ? sh.rl[w] : gbest;
        }
        __syncthreads();
    }
    if (split) {
        // This half's lists cut to what the row can need from it: the first
        // Ko observers, the sampler's first Ks + 1 (the next one counts as
        // turned away), or its small-survivor list. They go to the half's
        // slot with its statistics; the half that finishes second merges the
        // other's slot into its own and goes on alone (no waiting: the first
        // to finish leaves).
        uint32_t no = 0, ns = 0;
        if (Ko) no = min(rw_select(0, min(n_o, (uint32_t)RW_BUF), Ko, 0xffffffffu), Ko);
        if (smode == 1) {
            const uint32_t c = rw_select(1, min(n_s, (uint32_t)RW_BUF), Ks + 2, 0xffffffffu);
            if (c > Ks + 1) rejf = fmaxf(rejf, zs_key_to_float(~(uint32_t)(sh.u.b.s[Ks + 1] >> 32)));
            ns = min(c, Ks + 1);
        } else if (smode == 2 && !s_over) {
            ns = n_s;   // at most ZS_SMALL_CAP
        }
        RW_T(15);
        unsigned long long* mine = a.rw_part + ((size_t)r * 2 + half) * RW_PART;
        if (t == 0) {
            mine[0] = (unsigned long long)__float_as_uint(omax) | ((unsigned long long)__float_as_uint(ymax) << 32);
            mine[1] = (unsigned long long)fl | ((unsigned long long)(uint32_t)last_nan << 32);
            mine[2] = (unsigned long long)__float_as_uint(rejf) | ((unsigned long long)(s_over ? 1u : 0u) << 32);
            mine[3] = gbest;
            mine[4] = (unsigned long long)no | ((unsigned long long)ns << 32);
        }
        for (uint32_t i = t; i < no; i += RW_NT) mine[RW_PART_O + i] = sh.u.b.o[i];
        for (uint32_t i = t; i < ns; i += RW_NT) mine[RW_PART_S + i] = sh.u.b.s[i];
        // (the barrier completes every wave's stores; one device-scope fence
        // then publishes them before the count, and one makes the other
        // half's visible after it)
        __syncthreads();
        if (t == 0) {
            __threadfence();
            const uint32_t m = atomicAdd(&a.rw_ctr[r], 1u);
            if (m) {
                a.rw_ctr[r] = 0u;   // for the next call
                __threadfence();
            }
            sh.merge = m;
        }
        __syncthreads();
        RW_T(6);
        if (rw_uni(sh.merge) == 0u) return;   // the other half merges
        const unsigned long long* oth = a.rw_part + ((size_t)r * 2 + (1u - half)) * RW_PART;
        const unsigned long long h0 = oth[0], h1 = oth[1], h2 = oth[2], h3 = oth[3], h4 = oth[4];
        omax = fmaxf(omax, __uint_as_float((uint32_t)h0));
        ymax = fmaxf(ymax, __uint_as_float((uint32_t)(h0 >> 32)));
        fl |= (uint32_t)h1;
        last_nan = max(last_nan, (int)(uint32_t)(h1 >> 32));
        rejf = fmaxf(rejf, __uint_as_float((uint32_t)h2));
        const bool o_over = (h2 >> 32) != 0ull;
        gbest = h3 > gbest ? h3 : gbest;
        const uint32_t ono = (uint32_t)h4, ons = (uint32_t)(h4 >> 32);
        for (uint32_t i = t; i < ono; i += RW_NT) sh.u.b.o[no + i] = oth[RW_PART_O + i];
        n_o = no + ono;
        if (smode == 1) {
            for (uint32_t i = t; i < ons; i += RW_NT) sh.u.b.s[ns + i] = oth[RW_PART_S + i];
            n_s = ns + ons;
        } else if (smode == 2) {
            s_over = s_over || o_over || ns + ons > ZS_SMALL_CAP;
            if (!s_over)
                for (uint32_t i = t; i < ons; i += RW_NT) sh.u.b.s[ns + i] = oth[RW_PART_S + i];
            n_s = ns + ons;
        }
        __syncthreads();
        // later streams (the greedy fold after a NaN) cover the whole row
        R.gend = ngt;
        R.vend = V;
        R.glast = (V - 1) / RW_G;
    }
    const float M = rw_unif(omax);
    const float zmax = rw_unif(zs_temper(ymax, T));   // max z = temper(max y): monotone
    const bool special = (fl & ZS_CF_OBS_NAN) || M == INFINITY || M == -INFINITY;
    uint32_t obs_need = 0;
    if (!special && want_obs) obs_need |= ZS_OBS_S;
    if (!special && want_unc) obs_need |= ZS_OBS_H;
    // observer candidates: the first Ko entries of the sorted list
    uint32_t n_cand = 0;
    if (Ko) {
        const uint32_t n = rw_select(0, min(n_o, (uint32_t)RW_BUF), Ko, 0xffffffffu);
        n_cand = min(n, Ko);
        if (t < n_cand) {
            sh.cand_id[t] = (uint32_t)sh.u.b.o[t];
            sh.cand_x[t] = zs_key_to_float(~(uint32_t)(sh.u.b.o[t] >> 32));
        }
    }
    RW_T(3);

    // ---------------- sampler decisions
    uint32_t token = 0, mode = ZS_MODE_DONE, status = 0, has_thr = 0, thr_key = 0;
    float thr = -INFINITY;
    if (greedy) {
        // sampler.rs:35-42, max_by over partial_cmp: the last maximal element;
        // a NaN compares Equal, so the fold restarts after the last NaN
        status |= ZS_ST_GREEDY;
        if (last_nan < 0) {
            token = gbest ? (uint32_t)(gbest & 0xffffffffull) - 1u : 0u;
        } else {
            const uint32_t L = (uint32_t)last_nan;
            unsigned long long gb = 0;
            rw_stream<true>(R, sh, 0, [&](uint32_t g, int, const float (&x)[4], const float (&y)[4]) {
                const uint32_t idx0 = g * RW_G + 4 * t;
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    const uint32_t id = idx0 + q;
                    if (id >= V || id <= L || y[q] != y[q]) continue;
                    const uint32_t k = zs_total_key(y[q] == 0.0f ? 0.0f : y[q]);
                    const unsigned long long c = ((unsigned long long)k << 32) | (id + 1);
                    gb = c > gb ? c : gb;
                }
                return false;
            });
            for (int d = 32; d > 0; d >>= 1) {
                const unsigned long long o = __shfl_xor(gb, d, 64);
                gb = o > gb ? o : gb;
            }
            if (zs_lane() == 0) sh.rl[zs_wid()] = gb;
            __syncthreads();
            gb = 0;
#pragma unroll
            for (int w = 0; w < RW_NW; w++) gb = sh.rl[w] > gb ? sh.rl[w] : gb;
            __syncthreads();
            token = gb ? (uint32_t)(gb & 0xffffffffull) - 1u : L;
        }
    } else if ((fl & ZS_CF_Z_NAN) || zmax == INFINITY || zmax == -INFINITY) {
        // exp_sum is NaN: every comparison in the draw fails -> V-1 (sampler.rs:127)
        status |= ZS_ST_NONFINITE;
        token = V - 1;
    } else {
        bool small = false;
        uint32_t nsv = 0;
        if (smode == 1) {
            const uint32_t n = rw_select(1, min(n_s, (uint32_t)RW_BUF), Ks + 1, 0xffffffffu);
            // the k-th largest z is temper(the k-th largest y); a list of
            // fewer than k holds every y above -inf, so the k-th is -inf
            const float yk = n >= Ks ? zs_key_to_float(~(uint32_t)(sh.u.b.s[Ks - 1] >> 32)) : -INFINITY;
            thr = zs_temper(yk, T);
            thr_key = zs_total_key(thr);
            has_thr = 1;
            // every element at the threshold must be listed: after the first
            // k, the next listed y and the largest y turned away must map
            // below it (or the threshold is -inf: every finite value listed)
            bool complete = thr == -INFINITY;
            if (!complete) {
                const float ynext = n > Ks ? zs_key_to_float(~(uint32_t)(sh.u.b.s[Ks] >> 32)) : -INFINITY;
                const float yrej = rejf;
                complete = zs_temper(ynext, T) < thr && zs_temper(yrej, T) < thr;
            }
            if (thr == 0.0f) complete = false;  // the other zero also survives
            if (complete) {
                // survivors: !(z < thr) (sampler.rs:59-63) and above -inf
                if (t < 64) {
                    uint32_t c = 0;
                    for (uint32_t i0 = 0; i0 < Ks; i0 += 64) {
                        const uint32_t i = i0 + t;
                        float zi = -INFINITY;
                        if (i < Ks && i < n) zi = zs_temper(zs_key_to_float(~(uint32_t)(sh.u.b.s[i] >> 32)), T);
                        const bool sv = zi > -INFINITY;
                        const unsigned long long m = __ballot(sv);
                        if (sv) {
                            const uint32_t p = c + __popcll(m & ((1ull << t) - 1ull));
                            sh.sval[p] = zi;
                            sh.sidx[p] = (uint32_t)sh.u.b.s[i];
                        }
                        c += __popcll(m);
                    }
                    if (t == 0) sh.n_surv = c;
                }
                __syncthreads();
                nsv = sh.n_surv;
                small = true;
            }
        } else if (smode == 2 && !s_over) {
            // every y above -inf, unordered (<= ZS_SMALL_CAP); their z
            if (t < 64) {
                uint32_t c = 0;
                for (uint32_t i0 = 0; i0 < n_s; i0 += 64) {
                    const uint32_t i = i0 + t;
                    float zi = -INFINITY;
                    if (i < n_s) zi = zs_temper(zs_key_to_float(~(uint32_t)(sh.u.b.s[i] >> 32)), T);
                    const bool sv = zi > -INFINITY;
                    const unsigned long long m = __ballot(sv);
                    if (sv) {
                        const uint32_t p = c + __popcll(m & ((1ull << t) - 1ull));
                        sh.sval[p] = zi;
                        sh.sidx[p] = (uint32_t)sh.u.b.s[i];
                    }
                    c += __popcll(m);
                }
                if (t == 0) sh.n_surv = c;
            }
            __syncthreads();
            nsv = sh.n_surv;
            small = true;
        } else if (has_topk) {
            has_thr = 2;   // top_k > ZS_KS: zs_k_big selects the threshold
        }
        if (small) {
            __syncthreads();
            if (t < 64) rw_small(b.d_seed[r], b.d_counter[r], V, P, nsv, zmax, sh);
            __syncthreads();
            token = sh.tok;
            status |= ZS_ST_SMALL;
        } else {
            mode = ZS_MODE_BIG;
        }
    }
    __syncthreads();
    RW_T(4);

    // ---------------- the row sums, left to zs_sums.hip: the sampler's S of a
    // big row (on the caller's stream, before the big-row kernels), S_obs
    // (logprobs and uncertainty) and the entropy (on the side stream). A
    // masked row's sums run over its allowed ids, gathered to row scratch
    // (when at most RW_BUF and a quarter of the row are allowed), else over
    // the whole row with its allow bits.
    const bool doA = (obs_need & ZS_OBS_S) != 0;
    const bool doB = mode == ZS_MODE_BIG && has_thr != 2;
    const bool doH = (obs_need & ZS_OBS_H) != 0;
    uint32_t gn = 0;
    if (R.allow && (doA || doB || doH))
        gn = rw_uni(sh.g_done) ? rw_uni(sh.g_n) : rw_gather_allowed(R.row, R.allow, V, R.np, rw_scratch(a, r), R.gfl, R.gy);

    // ---------------- row state for the sums, the big-row kernels and zs_k_final
    if (t == 0) {
        st.rounds = (doB ? (1u << ZS_SUM_SAMP_S) : 0u) | (doA ? (1u << ZS_SUM_OBS_S) : 0u) |
                    (doH ? (1u << ZS_SUM_OBS_H) : 0u);
        st.g_n = gn;
        st.z_max = zmax;
        st.has_thr = has_thr;
        st.thr_key = thr_key;
        st.mode = mode;
        st.token = token;
        st.status = status;
        st.obs_max = M;
        st.obs_special = special ? 1u : 0u;
        st.obs_need = obs_need;
        st.n_cand = n_cand;
        st.klist = 0;
        st.kpend = 0;
        st.kident = 0;
        st.knorm = 0;
        st.samp_S = -0.0f;
        st.obs_S = -0.0f;
        st.obs_H = 0.0f;
    }
    if (t < n_cand) { st.cand_id[t] = sh.cand_id[t]; st.cand_x[t] = sh.cand_x[t]; }
    if (mode == ZS_MODE_BIG) {
        // bucket counts and masses of the top-p walk, accumulated by zs_k_pv
        zs_tp_bucket* bk = a.tp_bk + (size_t)r * ZS_TP_NB;
        for (uint32_t i = t; i < ZS_TP_NB; i += RW_NT) { bk[i].cnt = 0u; bk[i].mass = 0.0f; }
    }
    RW_T(5);
#ifdef ZS_WALK_DEBUG
    if (t == 0) atomicAdd(&rw_dbg[7], 1ull);
#endif
}

#ifdef ZS_WALK_DEBUG
extern "C" int zs_dbg_row_stats(unsigned long long* out) {
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(rw_dbg), 16 * sizeof(unsigned long long)) != hipSuccess) return -1;
    static unsigned long long zero[16];
    return hipMemcpyToSymbol(HIP_SYMBOL(rw_dbg), zero, sizeof(zero)) == hipSuccess ? 0 : -1;
}
#endif

extern "C" int zs_row_launch(const zs_sargs& a, hipStream_t stream) {
    const size_t dyn = 4 * ((a.b.V + 31) / 32) * sizeof(uint32_t);
    hipLaunchKernelGGL(zs_k_row, dim3(a.row_split ? 2 * a.b.B : a.b.B), dim3(RW_NT), dyn, stream, a);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
