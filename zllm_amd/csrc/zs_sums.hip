// zs_sums.hip -- the row sums of the sampler step, spread over the whole GPU.
//
// Three sequential f32 sums per row are reproduced exactly, in index order:
//   S_obs = sum expf(x~ - M)                 logprobs.rs:36, hallucination.rs:134-135
//   S     = sum expf(z - zmax), z = y / T    sampler.rs:68 (0 below a top-k cut)
//   H     = sum -(p ((x~ - M) - ln S_obs)),  p = expf(x~ - M) / S_obs, p > 0
//                                            hallucination.rs:139-144
// Inside one binade of the running sum s its values lie on the grid g = ulp(s)
// and adding a term t moves s by the integer round_half_even(t / g) (zs_math.h),
// except for an exact half-way term (its rounding follows the parity of s / g)
// and for the term that carries s out of its binade. A row is cut into
// sub-chunks of ZS_SUB ids, each taken by one wave:
//   zs_k_sapx    approximate sums of every sub-chunk (v_exp_f32 terms), from
//                which the grid of the running sum at each sub-chunk is
//                predicted (prefix sums, with a margin for the f32 rounding);
//   zs_k_sround  every sub-chunk whose predicted interval stays inside one
//                binade adds its increments on that grid: a pair (total from
//                an even start, total from an odd start), which makes the
//                half-way terms exact whatever the start;
//   zs_k_sstitch one wave per (row, sum) walks the sub-chunks in order from
//                the exact running sum: a sub-chunk whose grid was predicted
//                right and whose total stays inside the binade moves the sum
//                by its total; any other (a crossing, a wrong prediction) is
//                added exactly from its terms: per-lane increment pairs
//                prefix-scanned over the wave locate the lane where the sum
//                leaves its binade, whose terms are added as real f32
//                additions, and the walk resumes on the new grid.
// A wrong prediction costs time, never exactness: the stitch checks the grid
// and the binade end of every sub-chunk total it applies.
//
// Terms of S_obs and S are exact glibc expf values: a fast exp (relative
// error below ZS_EXP_EPS) decides an increment unless its scaled value lies
// within the error band of a half-integer, where zs_expf recomputes it
// (certified increments); H's terms are certified the same way with a band
// that covers the two extra f32 roundings of p and of the product.
#include <hip/hip_runtime.h>
#include "zs_sampler.h"
#include "zs_walk.h"

#define SM_EPT 16                       // terms per lane of a sub-chunk
#define SM_NT 256                       // threads of the approx / round kernels (4 sub-chunks)
#define SM_BAND_S 0x1p-21f              // certification band of the exp terms (ZS_EXP_EPS)
#define SM_BAND_H 0x1p-19f              // of the entropy terms (ZS_EXP_EPS + two roundings)
#define SM_MARGIN 0x1p-9                // relative margin of the grid prediction

static_assert(ZS_SUB == SM_EPT * 64, "one wave per sub-chunk");


static_assert(sizeof(sm_rec) == sizeof(zs_sub_sum), "sm_rec lives in the zs_sub_sum scratch");

// ---------------------------------------------------------------------------
// The terms' source: the row's logits (with the allow bits of a masked row and
// the merged patch list of zs_k_row), or the allowed ids a masked row gathered
// to row scratch (x~ and y already patched).
// ---------------------------------------------------------------------------
struct sm_src {
    const float* px;
    const float* py;
    const uint32_t* allow;   // row source of a masked row, else null
    const uint32_t* pid;     // patches (row source), else null
    const uint32_t* pfl;
    const float* pyv;
    const uint32_t* psub;
    uint32_t n;              // terms
    uint32_t lim4;           // last float4 start inside px / py
};

__device__ __forceinline__ const float* sm_gather_base(const zs_sargs& a, uint32_t r) {
    const float* cx = a.gath + (size_t)r * (2 * (size_t)a.max_vocab + 16);
    return cx + ((4u - (uint32_t)((reinterpret_cast<uintptr_t>(cx) >> 2) & 3u)) & 3u);
}

__device__ __forceinline__ sm_src sm_src_of(const zs_sargs& a, uint32_t r, const zs_row_state& st,
                                            const zs_row_params& P) {
    const zs_batch& b = a.b;
    sm_src s;
    if (st.g_n) {
        const uint32_t n4 = (st.g_n + 3u) & ~3u;
        s.px = sm_gather_base(a, r);
        s.py = s.px + n4;
        s.allow = nullptr;
        s.pid = nullptr;
        s.pfl = nullptr;
        s.pyv = nullptr;
        s.psub = nullptr;
        s.n = st.g_n;
        s.lim4 = n4 - 4u;
    } else {
        s.px = b.d_logits + (size_t)r * b.ld;
        s.py = s.px;
        s.allow = ((P.flags & ZS_ROW_MASKED) && b.d_allow_bits) ? b.d_allow_bits + (size_t)r * b.allow_words : nullptr;
        const bool patched = a.p_cnt[r] != 0u;
        s.pid = patched ? a.p_id + (size_t)r * a.pstride : nullptr;
        s.pfl = a.p_flags + (size_t)r * a.pstride;
        s.pyv = a.p_y + (size_t)r * a.pstride;
        s.psub = a.p_sub + (size_t)r * (a.max_subs + 1);
        s.n = b.V;
        s.lim4 = (uint32_t)min((uint64_t)b.ld - 4u, (uint64_t)0xfffffff0u);
    }
    return s;
}

// Exact terms of the sub-chunks that are not safe, per (row, sum), max_vocab
// floats: the sampler's S (caller's stream, finished before the big-row
// kernels reuse it) in the top-p prefix area; S_obs and then the entropy, in
// turn on the side stream beside the big-row kernels, in an area of their own.
__device__ __forceinline__ float* sm_darea(const zs_sargs& a, uint32_t r, int kind) {
    if (kind == ZS_SUM_SAMP_S) return reinterpret_cast<float*>(a.tp_pre + (size_t)r * a.max_vocab * 2);
    return a.s_hterm + (size_t)r * ((size_t)a.max_vocab + 8);
}

// Position (in the sub-chunk) of term e of float4 i of this lane: interleaved
// (i-th quarter of the sub-chunk, coalesced loads: the approx and round
// kernels) or contiguous (the lane's 16 consecutive terms: the stitch, which
// needs each lane's terms in summation order).
template <bool CONTIG>
__device__ __forceinline__ uint32_t sm_pos(uint32_t lane, int i) {
    return CONTIG ? 16u * lane + 4u * (uint32_t)i : 256u * (uint32_t)i + 4u * lane;
}

// A sub-chunk's loads for this lane, issued ahead of their use: the logits
// (or a masked row's gathered x~), the allow words and up to 64 of the
// sub-chunk's patches, one per lane.
typedef float sm_f4 __attribute__((ext_vector_type(4)));
struct sm_raw {
    sm_f4 vx[4];
    uint32_t w[4];
    uint32_t pid, pfl;
    float pyv;
    uint32_t p0, p1;    // the sub-chunk's patch range (uniform)
};

template <bool CONTIG>
__device__ __forceinline__ void sm_fetch(const sm_src& S, uint32_t j, sm_raw& R) {
    const uint32_t lane = (uint32_t)zs_lane();
    const uint32_t base = j * ZS_SUB;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t id0 = base + sm_pos<CONTIG>(lane, i);
        const uint32_t ia = min(id0, S.lim4);
        R.vx[i] = *reinterpret_cast<const sm_f4*>(S.px + ia);
        R.w[i] = S.allow ? S.allow[min(id0, S.n - 1u) >> 5] : 0xffffffffu;
    }
    R.p0 = R.p1 = 0u;
    if (S.pid) {
        R.p0 = S.psub[j];
        R.p1 = S.psub[j + 1];
        const uint32_t p = R.p0 + lane;
        if (p < R.p1) {
            R.pid = S.pid[p];
            R.pfl = S.pfl[p];
            R.pyv = S.pyv[p];
        }
    }
}

// x~ and y of the lane's terms from the fetched data: masked-out ids and
// terms past n read -inf (a zero term); bans set x~ and y to -inf, biased /
// counted ids take their y from the patch list.
template <bool CONTIG>
__device__ __forceinline__ void sm_finish(const sm_src& S, uint32_t j, const sm_raw& R, float (&x)[SM_EPT],
                                          float (&y)[SM_EPT]) {
    const uint32_t lane = (uint32_t)zs_lane();
    const uint32_t base = j * ZS_SUB;
    const bool gy = S.py != S.px;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t id0 = base + sm_pos<CONTIG>(lane, i);
        const uint32_t w = R.w[i] >> (id0 & 31u);
        const float xv[4] = {R.vx[i].x, R.vx[i].y, R.vx[i].z, R.vx[i].w};
        float yv[4] = {xv[0], xv[1], xv[2], xv[3]};
        if (gy) {
            // (gathered rows: y follows the x values; loaded here, not ahead)
            const sm_f4 vy = *reinterpret_cast<const sm_f4*>(S.py + min(id0, S.lim4));
            yv[0] = vy.x; yv[1] = vy.y; yv[2] = vy.z; yv[3] = vy.w;
        }
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const bool in = ((w >> e) & 1u) && id0 + e < S.n;
            x[4 * i + e] = in ? xv[e] : -INFINITY;
            y[4 * i + e] = in ? yv[e] : -INFINITY;
        }
    }
    // patches: each lane holds one of the first 64 (the rest are loaded here)
    for (uint32_t pb = R.p0; pb < R.p1; pb += 64) {
        uint32_t pid = R.pid, pfl = R.pfl;
        float pyv = R.pyv;
        if (pb != R.p0 && pb + lane < R.p1) {
            pid = S.pid[pb + lane];
            pfl = S.pfl[pb + lane];
            pyv = S.pyv[pb + lane];
        }
        const uint32_t cnt = min(R.p1 - pb, 64u);
        for (uint32_t u = 0; u < cnt; u++) {
            const uint32_t loc = (uint32_t)__builtin_amdgcn_readlane((int)pid, (int)u) - base;
            const uint32_t fl = (uint32_t)__builtin_amdgcn_readlane((int)pfl, (int)u);
            const float yp = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pyv), (int)u));
            const uint32_t owner = CONTIG ? (loc >> 4) : ((loc >> 2) & 63u);
            const int slot = CONTIG ? (int)(loc & 15u) : (int)(4u * (loc >> 8) + (loc & 3u));
            if (owner == lane) {
#pragma unroll
                for (int q = 0; q < SM_EPT; q++) {
                    if (q != slot) continue;
                    if (fl & ZS_PF_BAN) { x[q] = -INFINITY; y[q] = -INFINITY; }
                    if (fl & ZS_PF_Y) y[q] = yp;
                }
            }
        }
    }
}

template <bool CONTIG>
__device__ __forceinline__ void sm_load(const sm_src& S, uint32_t j, float (&x)[SM_EPT], float (&y)[SM_EPT]) {
    sm_raw R;
    sm_fetch<CONTIG>(S, j, R);
    sm_finish<CONTIG>(S, j, R, x, y);
}

// The glibc expf table in LDS (zs_expf_tab): the exact recomputations read it
// with a short LDS latency instead of a constant-memory load. File-scope LDS
// objects, so that every access is an LDS instruction (a generic pointer
// would give flat loads, which also wait for the outstanding global loads).
__shared__ uint64_t sm_tab[32];
__device__ __forceinline__ void sm_tab_fill() {
    const uint64_t T[32] = ZS_EXP2F_TAB;
    if (threadIdx.x < 32) {
#pragma unroll
        for (int i = 0; i < 32; i++)
            if ((int)threadIdx.x == i) sm_tab[i] = T[i];
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------
// Terms of the three sums: the argument d, a fast approximate value (-1: use
// the exact value) and the exact value.
// ---------------------------------------------------------------------------
struct sm_terms {
    int kind;            // ZS_SUM_*
    float M;             // observers: the row maximum of x~
    float T, rT, zmax, thr;
    uint32_t div;        // sampler: 0 no division, 1 Markstein, 2 IEEE
    bool use_thr;
    float inv, lns;      // entropy: 1 / S_obs, ln S_obs
};

__device__ __forceinline__ sm_terms sm_terms_of(int kind, const zs_row_state& st, const zs_row_params& P) {
    sm_terms f;
    f.kind = kind;
    f.M = st.obs_max;
    const float T = P.temperature;
    f.T = T;
    f.rT = 1.0f / T;
    f.div = !(T > 0.0f && T != 1.0f) ? 0u : ((T >= 0x1p-20f && T <= 0x1p20f) ? 1u : 2u);
    f.zmax = st.z_max;
    f.use_thr = st.has_thr != 0u;
    f.thr = zs_key_to_float(st.thr_key);
    f.inv = 1.0f / st.obs_S;
    f.lns = (float)log((double)st.obs_S);
    return f;
}

// z = y / T correctly rounded (sampler.rs:47-51): Markstein's sequence
// q0 = RN(y rT), q1 = RN(q0 + RN(y - q0 T) rT) is RN(y / T) for 2^-100 <= |y|
// <= 2^100 and 2^-20 <= T <= 2^20; zeros and infinities divide exactly as
// y rT; other y (and other T) divide the IEEE way.
__device__ __forceinline__ float sm_temper(const sm_terms& f, float y) {
    if (f.div == 0u) return y;
    // (-inf / inf is NaN; a row with T = inf and a real -inf element is
    // non-finite and sums nothing, so its -inf terms here are ids past the
    // row: no term)
    if (f.div == 2u) return y == -INFINITY ? -INFINITY : y / f.T;
    const float q0 = y * f.rT;
    const float q1 = fmaf(fmaf(-q0, f.T, y), f.rT, q0);
    const float a = fabsf(y);
    if (a >= 0x1p-100f && a <= 0x1p100f) return q1;
    if (a == 0.0f || a == INFINITY) return q0;
    return y / f.T;
}

__device__ __forceinline__ float sm_arg(const sm_terms& f, float x, float y) {
    if (f.kind == ZS_SUM_SAMP_S) {
        float z = sm_temper(f, y);
        if (f.use_thr && z < f.thr) z = -INFINITY;
        return z - f.zmax;
    }
    return x - f.M;
}

__device__ __forceinline__ float sm_exact(const sm_terms& f, float d) {
    const float e = zs_expf_tab(d, sm_tab);
    if (f.kind != ZS_SUM_OBS_H) return e;
    const float p = e * f.inv;
    return p > 0.0f ? -(p * (d - f.lns)) : 0.0f;
}

// -1 where only the exact value decides (subnormal results)
__device__ __forceinline__ float sm_fast(const sm_terms& f, float d) {
    const float e = zs_exp_fast(fmaxf(d, ZS_EXP_FAST_MIN));
    float v = e;
    if (f.kind == ZS_SUM_OBS_H) v = -((e * f.inv) * (d - f.lns));
    return d >= ZS_EXP_FAST_MIN ? v : (d < ZS_EXP_ZERO ? 0.0f : -1.0f);
}

// Increments of the lane's 16 terms on the grid of scale sc = 2^(150 - eg),
// eg >= SM_EG_MIN, from their fast values a, certified: where the band
// around a scaled value reaches a half-integer (or a is -1) the exact value
// decides (the recomputation is a branch taken only by the lanes that need
// it, skipped by the wave when none does). Terms outside `valid` count 0.
// *tie: bit q set for an exact half-way increment (then inc[q] is
// floor(t / g)).
__device__ __forceinline__ void sm_incs(const sm_terms& f, const float (&a)[SM_EPT], const float (&d)[SM_EPT], float sc,
                                        uint32_t valid, uint32_t (&inc)[SM_EPT], uint32_t* tie) {
    const float band = f.kind == ZS_SUM_OBS_H ? SM_BAND_H : SM_BAND_S;
    uint32_t unc = 0u;
#pragma unroll
    for (int q = 0; q < SM_EPT; q++) {
        const float qv = fminf(a[q] * sc, SM_QCAP);
        const float rq = rintf(qv);
        inc[q] = ((valid >> q) & 1u) ? (uint32_t)rq : 0u;
        const bool u = a[q] < 0.0f || (fmaf(qv, band, fabsf(qv - rq)) >= 0.5f && qv < SM_QCAP);
        unc |= (u ? 1u : 0u) << q;
    }
    unc &= valid;
    *tie = 0u;
    if (__builtin_amdgcn_readfirstlane((int)(__ballot(unc != 0u) != 0ull))) {
        if (unc) {
            uint32_t tb = 0u;
#pragma unroll
            for (int q = 0; q < SM_EPT; q++) {
                if (!((unc >> q) & 1u)) continue;
                const float qe = fminf(sm_exact(f, d[q]) * sc, SM_QCAP);
                float rq = rintf(qe);
                if (fabsf(qe - rq) == 0.5f) {
                    tb |= 1u << q;
                    rq = floorf(qe);
                }
                inc[q] = (uint32_t)rq;
            }
            *tie = tb;
        }
    }
}

__device__ __forceinline__ float sm_wave_sum_f(float v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    return __uint_as_float((uint32_t)__builtin_amdgcn_readfirstlane((int)__float_as_uint(v)));
}

// ---------------------------------------------------------------------------
// zs_k_sapx / zs_k_sround: each wave takes SM_SPW sub-chunks of one row (a
// workgroup SM_SPB consecutive ones), with the row's set-up done once and the
// next sub-chunk's loads issued before the current one is computed.
// ---------------------------------------------------------------------------
#define SM_SPW 1
#define SM_SPB (SM_SPW * (SM_NT / 64))

// Sub-chunk i of this wave in its workgroup's range.
__device__ __forceinline__ uint32_t sm_sub_of(uint32_t i) {
    return blockIdx.x * SM_SPB + (uint32_t)zs_wid() + (SM_NT / 64) * i;
}

// ---------------------------------------------------------------------------
// zs_k_sapx: approximate sums per sub-chunk. Record per sub-chunk: S_obs
// part, sampler S part, sum of e (x~ - M) for the entropy (v_exp_f32 terms),
// the largest x~ and the largest y.
// ---------------------------------------------------------------------------
#define SM_APX 8   // floats per sub-chunk record
// WHICH 1: the sampler's S (caller's stream); 2: S_obs and the entropy (side
// stream). Each writes only its own fields of the record.
template <int WHICH>
__global__ __launch_bounds__(SM_NT) void zs_k_sapx(zs_sargs a) {
    const uint32_t r = blockIdx.y;
    const zs_row_state& st = a.rst[r];
    const uint32_t jobs = st.rounds & (WHICH == 1 ? (1u << ZS_SUM_SAMP_S) : ((1u << ZS_SUM_OBS_S) | (1u << ZS_SUM_OBS_H)));
    if (!jobs) return;
    const zs_row_params P = a.b.d_params[r];
    const sm_src S = sm_src_of(a, r, st, P);
    const uint32_t nsub = (S.n + ZS_SUB - 1) / ZS_SUB;
    if (sm_sub_of(0) >= nsub) return;
    const float M = st.obs_max, zmax = st.z_max;
    const float T = P.temperature, rT = 1.0f / T;
    const bool divide = T > 0.0f && T != 1.0f;
    const bool use_thr = st.has_thr != 0u;
    const float thr = zs_key_to_float(st.thr_key);
    const bool obs = (jobs & ((1u << ZS_SUM_OBS_S) | (1u << ZS_SUM_OBS_H))) != 0u;
    const bool samp = (jobs & (1u << ZS_SUM_SAMP_S)) != 0u;
    // (a rolled loop: the copy of the next sub-chunk's loads at its end waits
    // for them after this sub-chunk's arithmetic)
    sm_raw Rc, Rn;
    sm_fetch<false>(S, sm_sub_of(0), Rc);
#pragma unroll 1
    for (int i = 0; i < SM_SPW; i++) {
        const uint32_t j = sm_sub_of(i);
        if (j >= nsub) break;
        const bool more = i + 1 < SM_SPW && sm_sub_of(i + 1) < nsub;
        if (more) sm_fetch<false>(S, sm_sub_of(i + 1), Rn);
        float x[SM_EPT], y[SM_EPT];
        sm_finish<false>(S, j, Rc, x, y);
        float so = 0.0f, ss = 0.0f, sd = 0.0f, mo = -INFINITY, ms = -INFINITY;
#pragma unroll
        for (int q = 0; q < SM_EPT; q++) {
            if (obs) {
                const float d = x[q] - M;
                const float e = d >= ZS_EXP_FAST_MIN ? zs_exp_hw(d) : 0.0f;
                so += e;
                mo = fmaxf(mo, x[q]);
                sd += d >= ZS_EXP_FAST_MIN ? e * d : 0.0f;
            }
            if (samp) {
                float z = divide ? y[q] * rT : y[q];
                if (use_thr && z < thr) z = -INFINITY;
                const float d = z - zmax;
                const float e = d >= ZS_EXP_FAST_MIN ? zs_exp_hw(d) : 0.0f;
                ss += e;
                ms = fmaxf(ms, y[q]);
            }
        }
        float* o = a.s_apx + ((size_t)r * a.max_subs + j) * SM_APX;
        if (WHICH == 1) {
            ss = sm_wave_sum_f(ss);
            ms = wave_max_f(ms);
            if (zs_lane() == 0) { o[1] = ss; o[4] = ms; }
        } else {
            so = sm_wave_sum_f(so);
            sd = sm_wave_sum_f(sd);
            mo = wave_max_f(mo);
            if (zs_lane() == 0) { o[0] = so; o[2] = sd; o[3] = mo; }
        }
        if (more) Rc = Rn;
    }
}

// Prefix data of the predictions of sub-chunk j (uniform): the sums of the
// approximate S_obs, sampler S and entropy parts of the sub-chunks before j
// and the largest x~ and y there.
struct sm_pre {
    double so, ss, sd;
    float mo, ms;
};
__device__ __forceinline__ sm_pre sm_pre_of(const zs_sargs& a, uint32_t r, uint32_t j) {
    const float* ap = a.s_apx + (size_t)r * a.max_subs * SM_APX;
    sm_pre P = {0.0, 0.0, 0.0, -INFINITY, -INFINITY};
    for (uint32_t i = (uint32_t)zs_lane(); i < j; i += 64) {
        const float4 v0 = *reinterpret_cast<const float4*>(ap + (size_t)i * SM_APX);
        const float v4 = ap[(size_t)i * SM_APX + 4];
        P.so += (double)v0.x;
        P.ss += (double)v0.y;
        P.sd += (double)v0.z;
        P.mo = fmaxf(P.mo, v0.w);
        P.ms = fmaxf(P.ms, v4);
    }
    P.so = wave_sum_d(P.so);
    P.ss = wave_sum_d(P.ss);
    P.sd = wave_sum_d(P.sd);
    P.mo = wave_max_f(P.mo);
    P.ms = wave_max_f(P.ms);
    return P;
}

// The approximate range of sum `kind` over sub-chunk j: lo below its start,
// mid the start's estimate, hi above its end (hi widened by the margin).
__device__ __forceinline__ void sm_range(const zs_sargs& a, uint32_t r, uint32_t j, int kind, const sm_terms& f,
                                         const sm_pre& P, double& lo, double& mid, double& hi) {
    const float* own = a.s_apx + ((size_t)r * a.max_subs + j) * SM_APX;
    if (kind == ZS_SUM_OBS_H) {
        const double inv = (double)f.inv, lns = (double)f.lns;
        mid = inv * (lns * P.so - P.sd);
        hi = inv * (lns * (P.so + (double)own[0]) - (P.sd + (double)own[2]));
        lo = mid * (1.0 - SM_MARGIN);
    } else {
        // the largest term before j, exactly: expf(max x~ - M), or expf(z -
        // zmax) of the largest y (z = y / T is monotone in y; not under a
        // top-k cut, which the approximate sums apply only approximately)
        const double pre = kind == ZS_SUM_SAMP_S ? P.ss : P.so;
        float tmax = 0.0f;
        if (kind == ZS_SUM_OBS_S) tmax = sm_exact(f, P.mo - f.M);
        else if (!f.use_thr) tmax = sm_exact(f, sm_temper(f, P.ms) - f.zmax);
        mid = pre;
        lo = fmax(pre * (1.0 - SM_MARGIN), (double)tmax);
        hi = pre + (double)(kind == ZS_SUM_SAMP_S ? own[1] : own[0]);
    }
    hi *= 1.0 + SM_MARGIN;
}
// Predicted grid of sub-chunk j of a sum from its approximate range
// (sm_range): the range widened by the margin must stay in one binade of
// grids >= SM_EG_MIN. The running sum is never below the
// largest term added so far (the f32 additions of non-negative terms are
// monotone), which bounds it from below where the margin would reach under
// a power of two (a sum resting just above one after its largest term).
// Returns the grid exponent, or 0.
__device__ __forceinline__ int sm_predict(uint32_t j, double lo, double hi) {
    if (j == 0 || !(lo > 0x1p-99) || !(hi < 0x1p100)) return 0;
    const int blo = ilogb(lo), bhi = ilogb(hi);
    if (blo != bhi) return 0;
    return blo + 127;   // zs_grid_exp of a normal float in that binade
}

// Crossing records of unpredictable sub-chunks (zs_walk.h's sm_xrec): when
// the approximate range puts the start surely in one binade and the end in
// the next, the exit term x is guessed from the start's estimate, and the
// pairs of the terms before x (grid eg) and after it (grid eg + 1) are taken
// over the exact terms, a quarter (4 terms a lane) at a time in summation
// order (quarter, lane, element). sm_cross_grid: the start grid, or 0 (no
// record), the estimated start on that grid (below the binade's end), and
// whether the start may already be in the next binade (SM_ALT: the pair of
// all the terms on the next grid as well).
__device__ __forceinline__ int sm_cross_grid(uint32_t j, double lo, double mid, double hi, uint32_t* kt,
                                             bool* alt) {
    if (j == 0 || !(lo > 0x1p-99) || !(hi < 0x1p100)) return 0;
    const int b = ilogb(lo), bm = ilogb(mid * (1.0 + SM_MARGIN));
    if (ilogb(hi) != b + 1 || (bm != b && bm != b + 1)) return 0;
    *alt = bm == b + 1;
    *kt = min((uint32_t)ldexp(mid, 23 - b), ZS_BINADE - 1u);
    return b + 127;
}
// Increments of 4 exact terms on the grid of scale sc (those in `valid`) and
// their half-way flags: the walk's rule (zs_walk.h).
__device__ __forceinline__ void sm_exact_incs4(const float (&v)[4], float sc, uint32_t valid, uint32_t (&inc)[4],
                                               uint32_t& tie) {
    tie = 0u;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        const float qe = fminf(v[e] * sc, SM_QCAP);
        float rq = rintf(qe);
        const bool h = fabsf(qe - rq) == 0.5f && ((valid >> e) & 1u);
        if (h) rq = floorf(qe);
        tie |= (h ? 1u : 0u) << e;
        inc[e] = ((valid >> e) & 1u) ? (uint32_t)rq : 0u;
    }
}
// The ordered pair of the wave's increments (lanes in order, elements in
// `valid` in order): a plain sum unless a half-way term is among them.
__device__ __forceinline__ seq_pair sm_wave_pair4(const uint32_t (&inc)[4], uint32_t tie, uint32_t valid) {
    if (!__builtin_amdgcn_readfirstlane((int)(__ballot(tie != 0u) != 0ull))) {
        uint32_t t = 0u;
#pragma unroll
        for (int e = 0; e < 4; e++) t = zs_sat_add(t, ((valid >> e) & 1u) ? inc[e] : 0u);
        const uint32_t w = sm_wave_sum_sat(t);
        return seq_pair{w, w};
    }
    seq_pair lp = {0u, 0u};
#pragma unroll
    for (int e = 0; e < 4; e++)
        if ((valid >> e) & 1u) lp = seq_compose(lp, ((tie >> e) & 1u) ? sm_pair_tie(inc[e]) : seq_pair{inc[e], inc[e]});
    return sm_wave_pair_reduce(lp);
}
struct sm_xstate {
    uint32_t carry, xpos;
    seq_pair pre, post, alt;
    float vx;
};
// One quarter qi of exact terms (this lane's 4 of it, dv); alt: the pair of
// all of them on grid eg + 1 as well.
__device__ __forceinline__ void sm_cross_quarter(sm_xstate& X, const float (&dv)[4], int qi, int eg, bool alt) {
    const uint32_t lane = (uint32_t)zs_lane();
    const uint32_t p0 = 256u * (uint32_t)qi + 4u * lane;   // this lane's first position in the quarter
    if (X.xpos == 0xffffffffu) {
        uint32_t inc[4], tie;
        sm_exact_incs4(dv, sm_scale(eg), 0xfu, inc, tie);
        uint32_t lt = 0u;
#pragma unroll
        for (int e = 0; e < 4; e++) lt = zs_sat_add(lt, inc[e]);
        const uint32_t incl = sm_wave_scan_sat(lt);
        const unsigned long long m = __ballot(zs_sat_add(X.carry, incl) >= ZS_BINADE);
        uint32_t vm = 0xfu;   // this lane's terms before the exit
        if (m) {
            const int L = __ffsll((long long)m) - 1;
            uint32_t kk = zs_sat_add(X.carry, incl - lt), ex = 3u;
            bool found = false;
#pragma unroll
            for (int e = 0; e < 4; e++) {
                kk = zs_sat_add(kk, inc[e]);
                if (!found && kk >= ZS_BINADE) { ex = (uint32_t)e; found = true; }
            }
            ex = (uint32_t)__builtin_amdgcn_readlane((int)ex, L);
            X.xpos = 256u * (uint32_t)qi + 4u * (uint32_t)L + ex;
            const float dq = ex == 0u ? dv[0] : ex == 1u ? dv[1] : ex == 2u ? dv[2] : dv[3];
            X.vx = __uint_as_float((uint32_t)__builtin_amdgcn_readlane((int)__float_as_uint(dq), L));
            vm = 0u;
#pragma unroll
            for (int e = 0; e < 4; e++) vm |= (p0 + (uint32_t)e < X.xpos ? 1u : 0u) << e;
        }
        X.pre = seq_compose(X.pre, sm_wave_pair4(inc, tie & vm, vm));
        X.carry = zs_sat_add(X.carry, (uint32_t)__builtin_amdgcn_readlane((int)incl, 63));
    }
    if (X.xpos != 0xffffffffu || alt) {
        uint32_t inc2[4], tie2;
        sm_exact_incs4(dv, sm_scale(eg + 1), 0xfu, inc2, tie2);
        if (X.xpos != 0xffffffffu) {
            uint32_t vm = 0u;
#pragma unroll
            for (int e = 0; e < 4; e++) vm |= (p0 + (uint32_t)e > X.xpos ? 1u : 0u) << e;
            X.post = seq_compose(X.post, sm_wave_pair4(inc2, tie2 & vm, vm));
        }
        if (alt) X.alt = seq_compose(X.alt, sm_wave_pair4(inc2, tie2, 0xfu));
    }
}

// Sub-chunk total on grid eg (uniform): the increment pair of the wave's
// terms in summation order (interleaved layout: quarter i, lane, element).
__device__ __forceinline__ seq_pair sm_total(const sm_terms& f, const float (&x)[SM_EPT], const float (&y)[SM_EPT],
                                             int eg) {
    float dd[SM_EPT], av[SM_EPT];
#pragma unroll
    for (int q = 0; q < SM_EPT; q++) {
        dd[q] = sm_arg(f, x[q], y[q]);
        av[q] = sm_fast(f, dd[q]);
    }
    uint32_t inc[SM_EPT], tie, tot = 0u;
    sm_incs(f, av, dd, sm_scale(eg), 0xffffu, inc, &tie);
#pragma unroll
    for (int q = 0; q < SM_EPT; q++) tot = zs_sat_add(tot, inc[q]);
    if (!__builtin_amdgcn_readfirstlane((int)(__ballot(tie != 0u) != 0ull))) {
        const uint32_t s = sm_wave_sum_sat(tot);
        return seq_pair{s, s};
    }
    // half-way terms: ordered pairs, quarter by quarter
    seq_pair all = {0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        seq_pair lp = {0u, 0u};
#pragma unroll
        for (int e = 0; e < 4; e++) {
            const int q = 4 * i + e;
            const seq_pair t = ((tie >> q) & 1u) ? sm_pair_tie(inc[q]) : seq_pair{inc[q], inc[q]};
            lp = seq_compose(lp, t);
        }
        all = seq_compose(all, sm_wave_pair_reduce(lp));
    }
    return all;
}

// ---------------------------------------------------------------------------
// zs_k_sround<STAGE>: one sum per stage: 1 the sampler's S of the big rows
// (the big-row kernels wait for it), 2 S_obs and 3 the entropy (which needs
// the exact S_obs), both on the side stream.
// ---------------------------------------------------------------------------
template <int STAGE>
__device__ __forceinline__ constexpr int sm_stage_kind() {
    return STAGE == 1 ? ZS_SUM_SAMP_S : STAGE == 2 ? ZS_SUM_OBS_S : ZS_SUM_OBS_H;
}
// exact terms of a wave's sub-chunk for its crossing record
__shared__ float sm_xbuf[SM_NT / 64][ZS_SUB];
template <int STAGE>
__global__ __launch_bounds__(SM_NT) void zs_k_sround(zs_sargs a) {
    const uint32_t r = blockIdx.y;
    const zs_row_state& st = a.rst[r];
    const uint32_t mine = 1u << sm_stage_kind<STAGE>();
    const uint32_t jobs = st.rounds & mine;
    if (!jobs) return;
    const zs_row_params P = a.b.d_params[r];
    const sm_src S = sm_src_of(a, r, st, P);
    const uint32_t nsub = (S.n + ZS_SUB - 1) / ZS_SUB;
    if (blockIdx.x * SM_SPB >= nsub) return;
    sm_tab_fill();
    const int kinds[1] = {sm_stage_kind<STAGE>()};
    constexpr int NK = 1;
    sm_terms F[NK];
#pragma unroll
    for (int u = 0; u < NK; u++) F[u] = sm_terms_of(kinds[u], st, P);
    if (sm_sub_of(0) >= nsub) return;
    sm_raw Rc, Rn;
    sm_fetch<false>(S, sm_sub_of(0), Rc);
#pragma unroll 1
    for (int i = 0; i < SM_SPW; i++) {
        const uint32_t j = sm_sub_of(i);
        if (j >= nsub) break;
        const bool more = i + 1 < SM_SPW && sm_sub_of(i + 1) < nsub;
        if (more) sm_fetch<false>(S, sm_sub_of(i + 1), Rn);
        float x[SM_EPT], y[SM_EPT];
        sm_finish<false>(S, j, Rc, x, y);
        sm_rec* rec = reinterpret_cast<sm_rec*>(a.s_rec) + (size_t)r * ZS_NSUM * a.max_subs + j;
#pragma unroll
        for (int u = 0; u < NK; u++) {
            if (!((jobs >> kinds[u]) & 1u)) continue;
            const sm_terms& f = F[u];
            double lo, mid, hi;
            sm_range(a, r, j, kinds[u], f, sm_pre_of(a, r, j), lo, mid, hi);
            const int eg = sm_predict(j, lo, hi);
            if (eg) {
                const seq_pair t = sm_total(f, x, y, eg);
                if (zs_lane() == 0) rec[(size_t)kinds[u] * a.max_subs] = sm_rec{eg, SM_SAFE, t.e, t.o};
            } else {
                // the stitch walks this sub-chunk from its exact terms,
                // unless its crossing record holds (exact terms also kept in
                // LDS for it)
                uint32_t kt = 0u;
                bool alt = false;
                const int xeg = sm_cross_grid(j, lo, mid, hi, &kt, &alt);
                float* xb = sm_xbuf[zs_wid()];
                float* da = sm_darea(a, r, kinds[u]) + (size_t)j * ZS_SUB;
                // (a rolled loop over the quarters: sixteen inlined exact
                // exponentials would hold too many registers)
#pragma unroll 1
                for (int qi = 0; qi < 4; qi++) {
                    float xv[4], yv[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        xv[e] = qi == 0 ? x[e] : (qi == 1 ? x[4 + e] : (qi == 2 ? x[8 + e] : x[12 + e]));
                        yv[e] = qi == 0 ? y[e] : (qi == 1 ? y[4 + e] : (qi == 2 ? y[8 + e] : y[12 + e]));
                    }
                    const uint32_t p = sm_pos<false>((uint32_t)zs_lane(), qi);
                    float dv[4];
#pragma unroll
                    for (int e = 0; e < 4; e++) dv[e] = sm_exact(f, sm_arg(f, xv[e], yv[e]));
                    if (j * ZS_SUB + p + 4 <= S.n) {
                        *reinterpret_cast<sm_f4*>(da + p) = sm_f4{dv[0], dv[1], dv[2], dv[3]};
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; e++)
                            if (j * ZS_SUB + p + e < S.n) da[p + e] = dv[e];
                    }
                    if (xeg || j == 0) {
                        // (terms past the row: none, as in the walk)
                        float dz[4];
#pragma unroll
                        for (int e = 0; e < 4; e++) dz[e] = j * ZS_SUB + p + e < S.n ? dv[e] : 0.0f;
                        *reinterpret_cast<sm_f4*>(xb + p) = sm_f4{dz[0], dz[1], dz[2], dz[3]};
                    }
                }
                sm_rec cr = {0, 0u, 0u, 0u};
                if (j == 0) {
                    // sub-chunk 0 from the sum's start value, term by term
                    __builtin_amdgcn_s_waitcnt(0);
                    __builtin_amdgcn_wave_barrier();
                    uint32_t sp;
                    const float s0 = sm_serial(xb, ZS_SUB, kinds[u] == ZS_SUM_OBS_H ? 0.0f : -0.0f, NAN, &sp);
                    cr = sm_rec{0, SM_EXACT, __float_as_uint(s0), 0xffffffffu};
                } else if (xeg) {
                    sm_xstate X = {kt, 0xffffffffu, {0u, 0u}, {0u, 0u}, {0u, 0u}, 0.0f};
#pragma unroll
                    for (int qi = 0; qi < 4; qi++) {
                        const sm_f4 q4 = *reinterpret_cast<const sm_f4*>(xb + sm_pos<false>((uint32_t)zs_lane(), qi));
                        const float dv[4] = {q4.x, q4.y, q4.z, q4.w};
                        sm_cross_quarter(X, dv, qi, xeg, alt);
                    }
                    const uint32_t fl = (X.xpos != 0xffffffffu ? SM_CROSS : 0u) | (alt ? SM_ALT : 0u);
                    if (fl) {
                        cr = sm_rec{xeg, fl, X.pre.e, X.pre.o};
                        if (zs_lane() == 0)
                            reinterpret_cast<sm_xrec*>(a.s_xrec)[((size_t)r * ZS_NSUM + kinds[u]) * a.max_subs + j] =
                                sm_xrec{X.xpos, X.vx, X.post.e, X.post.o, X.alt.e, X.alt.o};
                    }
                }
                if (zs_lane() == 0) rec[(size_t)kinds[u] * a.max_subs] = cr;
            }
        }
        if (more) Rc = Rn;
    }
}

// ---------------------------------------------------------------------------
// zs_k_sstitch<STAGE>: one 256-thread workgroup per (row, sum) (zs_walk.h):
// the sub-chunks the round kernel left unsafe are walked from the exact terms
// it stored for them, a safe one whose total did not apply from the source.
// ---------------------------------------------------------------------------
// A thread's 4 exact terms of sub-chunk j straight from the source (x~ / y
// with mask and patches): the rare safe sub-chunk whose total did not apply.
__device__ __forceinline__ void sm_terms_src(const sm_src& S, const sm_terms& f, uint32_t j, float (&d)[SW_TPT]) {
    const uint32_t id0 = j * ZS_SUB + SW_TPT * threadIdx.x;
    const uint32_t ia = min(id0, S.lim4);
    const sm_f4 vx = *reinterpret_cast<const sm_f4*>(S.px + ia);
    const sm_f4 vy = *reinterpret_cast<const sm_f4*>(S.py + ia);
    float x[4] = {vx.x, vx.y, vx.z, vx.w}, y[4] = {vy.x, vy.y, vy.z, vy.w};
    const uint32_t w = S.allow ? S.allow[min(id0, S.n - 1u) >> 5] >> (id0 & 31u) : 0xffffffffu;
#pragma unroll
    for (int e = 0; e < 4; e++) {
        if (!((w >> e) & 1u) || id0 + e >= S.n) { x[e] = -INFINITY; y[e] = -INFINITY; }
    }
    if (S.pid) {
        for (uint32_t p = S.psub[j]; p < S.psub[j + 1]; p++) {
            const uint32_t id = S.pid[p];
            if (id < id0 || id >= id0 + 4) continue;
            const uint32_t fl = S.pfl[p];
#pragma unroll
            for (int e = 0; e < 4; e++) {
                if (id != id0 + e) continue;
                if (fl & ZS_PF_BAN) { x[e] = -INFINITY; y[e] = -INFINITY; }
                if (fl & ZS_PF_Y) y[e] = S.pyv[p];
            }
        }
    }
#pragma unroll
    for (int e = 0; e < 4; e++) d[e] = sm_exact(f, sm_arg(f, x[e], y[e]));
}

// Terms of a row sum for sm_stitch.
struct sm_row_tp {
    const sm_src& S;
    const sm_terms& f;
    const float* darea;
    __device__ __forceinline__ void fetch(uint32_t j, sm_f4& raw) const {
        raw = *reinterpret_cast<const sm_f4*>(darea + min(j * ZS_SUB + SW_TPT * threadIdx.x, (S.n - 1u) & ~3u));
    }
    __device__ __forceinline__ void take(uint32_t j, const sm_f4& raw, float (&v)[SW_TPT]) const {
        const uint32_t id0 = j * ZS_SUB + SW_TPT * threadIdx.x;
        v[0] = raw.x; v[1] = raw.y; v[2] = raw.z; v[3] = raw.w;
#pragma unroll
        for (int e = 0; e < SW_TPT; e++)
            if (id0 + e >= S.n) v[e] = 0.0f;
    }
    __device__ __forceinline__ void direct(uint32_t j, float (&v)[SW_TPT]) const { sm_terms_src(S, f, j, v); }
};

template <int STAGE>
__global__ __launch_bounds__(SW_NT) void zs_k_sstitch(zs_sargs a) {
    const uint32_t r = blockIdx.x;
    zs_row_state* stp = a.rst + r;
    const int kind = sm_stage_kind<STAGE>();
    if (!((stp->rounds >> kind) & 1u)) return;
    [[maybe_unused]] const unsigned long long k0 = SW_CLK();
    sm_tab_fill();
    const zs_row_state& st = *stp;
    const zs_row_params P = a.b.d_params[r];
    const sm_src S = sm_src_of(a, r, st, P);
    const sm_terms f = sm_terms_of(kind, st, P);
    const uint32_t nsub = (S.n + ZS_SUB - 1) / ZS_SUB;
    const sm_rec* rec = reinterpret_cast<const sm_rec*>(a.s_rec) + ((size_t)r * ZS_NSUM + kind) * a.max_subs;
    const sm_xrec* xrec = reinterpret_cast<const sm_xrec*>(a.s_xrec) + ((size_t)r * ZS_NSUM + kind) * a.max_subs;
    for (uint32_t i = threadIdx.x; i < nsub; i += SW_NT) {
        const sm_rec e = rec[i];
        sm_sh.rec[i] = e;
        if (e.flags & (SM_CROSS | SM_ALT)) sm_sh.xrec[i] = xrec[i];
    }
    __syncthreads();
    [[maybe_unused]] const unsigned long long k1 = SW_CLK();
    sm_row_tp tp{S, f, sm_darea(a, r, kind)};
    uint32_t stop;
    const float s = sm_stitch<sm_row_tp, sm_f4>(tp, nsub, kind == ZS_SUM_OBS_H ? 0.0f : -0.0f, NAN, &stop);
    SW_K(STAGE - 1, SW_CLK() - k0, k1 - k0);
    if (threadIdx.x == 0) {
        if (kind == ZS_SUM_OBS_S) stp->obs_S = s;
        else if (kind == ZS_SUM_SAMP_S) stp->samp_S = s;
        else stp->obs_H = s;
    }
}

#ifdef ZS_WALK_DEBUG
extern "C" int zs_dbg_walk_hist(unsigned long long* out) {
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(sw_hist), 64 * sizeof(unsigned long long)) != hipSuccess) return -1;
    static unsigned long long zero[64];
    return hipMemcpyToSymbol(HIP_SYMBOL(sw_hist), zero, sizeof(zero)) == hipSuccess ? 0 : -1;
}
extern "C" int zs_dbg_walk_stats(unsigned long long* out) {
    if (hipMemcpyFromSymbol(out, HIP_SYMBOL(sw_dbg), 32 * sizeof(unsigned long long)) != hipSuccess) return -1;
    static unsigned long long zero[32];
    return hipMemcpyToSymbol(HIP_SYMBOL(sw_dbg), zero, sizeof(zero)) == hipSuccess ? 0 : -1;
}
#endif

// Launches one kernel of the row sums: 0 zs_k_sapx<1>, 1 zs_k_sround<1>,
// 2 zs_k_sstitch<1> (the sampler's S); 3 zs_k_sapx<2>, 4 zs_k_sround<2>,
// 5 zs_k_sstitch<2> (S_obs), 6 zs_k_sround<3>, 7 zs_k_sstitch<3> (entropy).
extern "C" int zs_sums_launch(const zs_sargs& a, uint32_t which, hipStream_t stream) {
    const uint32_t nsub = (a.b.V + ZS_SUB - 1) / ZS_SUB;
    const dim3 grid((nsub + SM_SPB - 1) / SM_SPB, a.b.B);
    switch (which) {
        case 0: hipLaunchKernelGGL(zs_k_sapx<1>, grid, dim3(SM_NT), 0, stream, a); break;
        case 1: hipLaunchKernelGGL(zs_k_sround<1>, grid, dim3(SM_NT), 0, stream, a); break;
        case 2: hipLaunchKernelGGL(zs_k_sstitch<1>, dim3(a.b.B), dim3(SW_NT), 0, stream, a); break;
        case 3: hipLaunchKernelGGL(zs_k_sapx<2>, grid, dim3(SM_NT), 0, stream, a); break;
        case 4: hipLaunchKernelGGL(zs_k_sround<2>, grid, dim3(SM_NT), 0, stream, a); break;
        case 5: hipLaunchKernelGGL(zs_k_sstitch<2>, dim3(a.b.B), dim3(SW_NT), 0, stream, a); break;
        case 6: hipLaunchKernelGGL(zs_k_sround<3>, grid, dim3(SM_NT), 0, stream, a); break;
        case 7: hipLaunchKernelGGL(zs_k_sstitch<3>, dim3(a.b.B), dim3(SW_NT), 0, stream, a); break;
        default: return -1;
    }
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
