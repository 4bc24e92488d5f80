// zs_sample.hip -- the per-step sampler over a batch of fp32 logit rows.
//
// Reference semantics (per row, in the order of rest.rs:2594-2624):
//   x~ = apply_mask(x)                    logit_fsm.rs:247-270 (bans, allow bits)
//   y  = adjust_logits(x~)                decode_ctrl.rs:107-126
//   token = sample_with_rng(y, cfg, r)    sampler.rs:31-128
//   logprobs / token_uncertainty on x~    logprobs.rs:34-54, hallucination.rs:129-154
//
// Kernels (one launch each, in stream order):
//   zs_k_prep     one workgroup per row: merge ban / bias / count-map lists into a
//                 per-row list of patched token ids (y values computed exactly).
//   zs_k_pass1    one workgroup per 8192-logit chunk: the only full HBM read.
//                 Observer statistics, sampler max / greedy argmax / flags, and
//                 exact top-K candidate lists (LDS radix select on total-order keys).
//   zs_k_combine  one workgroup per row: merges chunk results; finishes greedy,
//                 non-finite and small-survivor rows exactly on chip.
//   zs_k_big      one 1024-thread workgroup per remaining row: exact emulation of
//                 the reference's sequential f32 sums (S, min-p, top-p, draw).
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

// ===========================================================================
// zs_k_prep: per-row patch list.
// Entries are (id << 32) | (kind << 28) | order with kind 0 = ban, 1 = bias,
// 2 = count; sorting groups them by id with bans first and biases in list
// order, which reproduces the reference's per-token operation sequence.
// ===========================================================================
#define ZS_PREP_NT 256
__global__ __launch_bounds__(ZS_PREP_NT) void zs_k_prep(zs_sargs a) {
    const uint32_t r = blockIdx.x;
    const zs_batch& b = a.b;
    __shared__ unsigned long long ent[ZS_MAX_PATCHES];
    __shared__ uint32_t scan_sh[ZS_PREP_NT / 64];
    __shared__ uint32_t n_sh;
    const zs_row_params P = b.d_params[r];
    const uint32_t V = b.V;
    uint32_t ban0 = b.d_ban_off ? b.d_ban_off[r] : 0, ban1 = b.d_ban_off ? b.d_ban_off[r + 1] : 0;
    uint32_t bi0 = b.d_bias_off ? b.d_bias_off[r] : 0, bi1 = b.d_bias_off ? b.d_bias_off[r + 1] : 0;
    uint32_t c0 = b.d_cnt_off ? b.d_cnt_off[r] : 0, c1 = b.d_cnt_off ? b.d_cnt_off[r + 1] : 0;
    const bool pen = zs_penalty_active(P);
    if (!pen) { c1 = c0; }  // counts only matter when penalties are active
    uint32_t nb = ban1 - ban0, nbi = bi1 - bi0, nc = c1 - c0;
    uint32_t total = nb + nbi + nc;
    if (threadIdx.x == 0) n_sh = 0;
    __syncthreads();
    if (total > ZS_MAX_PATCHES) {
        if (threadIdx.x == 0) {
            a.p_cnt[r] = 0;
            a.rst[r].status = ZS_ST_LIMIT;
        }
        const uint32_t nsub = (V + ZS_SUB - 1) / ZS_SUB;
        for (uint32_t j = threadIdx.x; j <= nsub; j += ZS_PREP_NT) a.p_sub[(size_t)r * (a.max_subs + 1) + j] = 0;
        return;
    }
    // gather entries with id < V
    for (uint32_t i = threadIdx.x; i < total; i += ZS_PREP_NT) {
        uint32_t id, kind, ord;
        if (i < nb) { id = b.d_ban_ids[ban0 + i]; kind = 0; ord = i; }
        else if (i < nb + nbi) { ord = i - nb; id = b.d_bias_ids[bi0 + ord]; kind = 1; }
        else { ord = i - nb - nbi; id = b.d_cnt_ids[c0 + ord]; kind = 2; }
        if (id < V) {
            uint32_t pos = atomicAdd(&n_sh, 1u);
            ent[pos] = ((unsigned long long)id << 32) | ((unsigned long long)kind << 28) | ord;
        }
    }
    __syncthreads();
    uint32_t n = n_sh;
    uint32_t np2 = 1;
    while (np2 < n) np2 <<= 1;
    for (uint32_t i = n + threadIdx.x; i < np2; i += ZS_PREP_NT) ent[i] = ~0ull;
    __syncthreads();
    if (np2 > 1) block_sort_u64<ZS_PREP_NT>(ent, np2);
    // segment starts -> output slots
    uint32_t* out_id = a.p_id + (size_t)r * ZS_MAX_PATCHES;
    uint32_t* out_fl = a.p_flags + (size_t)r * ZS_MAX_PATCHES;
    float* out_y = a.p_y + (size_t)r * ZS_MAX_PATCHES;
    uint32_t base_out = 0;
    for (uint32_t s0 = 0; s0 < n; s0 += ZS_PREP_NT) {
        uint32_t i = s0 + threadIdx.x;
        uint32_t is_start = 0;
        if (i < n) {
            uint32_t id = (uint32_t)(ent[i] >> 32);
            is_start = (i == 0) || ((uint32_t)(ent[i - 1] >> 32) != id);
        }
        uint32_t tot;
        uint32_t ex = block_excl_scan_u<ZS_PREP_NT>(is_start, scan_sh, &tot);
        if (is_start) {
            uint32_t id = (uint32_t)(ent[i] >> 32);
            float x = b.d_logits[(size_t)r * b.ld + id];
            if ((P.flags & ZS_ROW_MASKED) && b.d_allow_bits && !zs_allowed_bit(b, r, id)) x = -INFINITY;
            uint32_t fl = 0;
            float y;
            uint32_t j = i;
            // bans (logit_fsm.rs:248-252)
            while (j < n && (uint32_t)(ent[j] >> 32) == id && ((ent[j] >> 28) & 3ull) == 0) {
                fl |= ZS_PF_BAN;
                j++;
            }
            if (fl & ZS_PF_BAN) x = -INFINITY;
            y = x;
            // logit_bias in list order (decode_ctrl.rs:108-112)
            while (j < n && (uint32_t)(ent[j] >> 32) == id && ((ent[j] >> 28) & 3ull) == 1) {
                uint32_t ord = (uint32_t)(ent[j] & 0x0fffffffull);
                y = y + b.d_bias_vals[bi0 + ord];
                fl |= ZS_PF_Y;
                j++;
            }
            // penalty (decode_ctrl.rs:113-125)
            if (j < n && (uint32_t)(ent[j] >> 32) == id && ((ent[j] >> 28) & 3ull) == 2) {
                uint32_t ord = (uint32_t)(ent[j] & 0x0fffffffull);
                uint32_t cnt = b.d_cnt_vals[c0 + ord];
                if (P.repeat != 1.0f) {
                    if (y > 0.0f) y = y / P.repeat;
                    else y = y * P.repeat;
                }
                float pen_v = __fmul_rn(P.frequency, (float)cnt);
                pen_v = __fadd_rn(pen_v, P.presence);
                y = __fsub_rn(y, pen_v);
                fl |= ZS_PF_Y;
            }
            out_id[base_out + ex] = id;
            out_fl[base_out + ex] = fl;
            out_y[base_out + ex] = y;
        }
        base_out += tot;
    }
    if (threadIdx.x == 0) {
        a.p_cnt[r] = base_out;
        a.rst[r].status = 0;
    }
    // first patch of every sub-chunk (patch ids are sorted and unique)
    __threadfence_block();
    __syncthreads();
    const uint32_t nsub = (V + ZS_SUB - 1) / ZS_SUB;
    uint32_t* psub = a.p_sub + (size_t)r * (a.max_subs + 1);
    for (uint32_t j = threadIdx.x; j <= nsub; j += ZS_PREP_NT) {
        uint32_t lo = 0, hi = base_out, key = j * ZS_SUB;
        while (lo < hi) { uint32_t mid = (lo + hi) >> 1; if (out_id[mid] < key) lo = mid + 1; else hi = mid; }
        psub[j] = lo;
    }
}

// ===========================================================================
// zs_k_pass1
// ===========================================================================
#define P1_EPT (ZS_P1_CH / ZS_P1_NT)

#define P1_SUP 1024
#define P1_SORT 256
struct p1_red {
    float omax, zmax;
    uint32_t fl, zfin, zabove, xabove;
    int last_nan;
};
struct p1_shared {
    p1_red red[ZS_P1_NT / 64];
    uint32_t hist[256];
    uint32_t u[8];
    int i[8];
    float f[8];
    double d[8];
    uint32_t cnt;
    uint32_t prefix, need, found;
    uint32_t pcur0, pcur1;
    uint32_t tmax[ZS_P1_NT];
    uint32_t skey[P1_SUP];
    uint32_t sidx[P1_SUP];
    uint32_t sel[4];
    unsigned long long s64[P1_SORT];
};

// Exact top-K (key desc, index asc) of the chunk's valid keys; writes the
// candidates (unordered) to out_key/out_idx. Element e = j*4+q of thread t has
// index base + (j*256 + t)*4 + q.
__device__ __forceinline__ void p1_topk(const uint32_t (&kv)[P1_EPT], uint32_t vmask, uint32_t nvalid, uint32_t K,
                        uint32_t base, uint32_t* out_key, uint32_t* out_idx, uint32_t* n_out, uint32_t* kth,
                        uint32_t* full, p1_shared& sh) {
    const int t = threadIdx.x;
    if (t == 0) sh.cnt = 0;
    __syncthreads();
    if (nvalid <= K) {
        for (int e = 0; e < P1_EPT; e++) {
            if ((vmask >> e) & 1u) {
                uint32_t pos = atomicAdd(&sh.cnt, 1u);
                if (pos < K) {
                    out_key[pos] = kv[e];
                    out_idx[pos] = base + ((e >> 2) * ZS_P1_NT + t) * 4 + (e & 3);
                }
            }
        }
        __syncthreads();
        *n_out = min(sh.cnt, K);
        *kth = 0;
        *full = 0;
        return;
    }
    uint32_t prefix = 0, mask = 0, need = K;
    for (int shift = 24; shift >= 0; shift -= 8) {
        if (t < 256) sh.hist[t] = 0;
        __syncthreads();
        for (int e = 0; e < P1_EPT; e++)
            if (((vmask >> e) & 1u) && (kv[e] & mask) == prefix)
                atomicAdd(&sh.hist[(kv[e] >> shift) & 255u], 1u);
        __syncthreads();
        if (t < 64) {
            // lane l owns bins 255-4l .. 252-4l (descending)
            uint32_t c[4], loc = 0;
            for (int q = 0; q < 4; q++) { c[q] = sh.hist[255 - 4 * t - q]; loc += c[q]; }
            uint32_t inc = wave_incl_scan_u(loc);
            uint32_t before = inc - loc;
            for (int q = 0; q < 4; q++) {
                if (before < need && need <= before + c[q]) {
                    sh.found = 255 - 4 * t - q;
                    sh.need = need - before;
                }
                before += c[q];
            }
        }
        __syncthreads();
        prefix |= sh.found << shift;
        mask |= 0xffu << shift;
        need = sh.need;
        __syncthreads();
    }
    const uint32_t kk = prefix;
    uint32_t my_eq = 0;
    for (int e = 0; e < P1_EPT; e++) {
        if (!((vmask >> e) & 1u)) continue;
        if (kv[e] > kk) {
            uint32_t pos = atomicAdd(&sh.cnt, 1u);
            if (pos < K) {
                out_key[pos] = kv[e];
                out_idx[pos] = base + ((e >> 2) * ZS_P1_NT + t) * 4 + (e & 3);
            }
        } else if (kv[e] == kk) {
            my_eq++;
        }
    }
    uint32_t n_eq = block_sum_u<ZS_P1_NT>(my_eq, sh.u);
    if (n_eq == need) {
        for (int e = 0; e < P1_EPT; e++) {
            if (((vmask >> e) & 1u) && kv[e] == kk) {
                uint32_t pos = atomicAdd(&sh.cnt, 1u);
                if (pos < K) {
                    out_key[pos] = kv[e];
                    out_idx[pos] = base + ((e >> 2) * ZS_P1_NT + t) * 4 + (e & 3);
                }
            }
        }
    } else {
        // lowest-index `need` elements among the equal ones, in index order
        uint32_t carry = 0;
        for (int j = 0; j < P1_EPT / 4; j++) {
            uint32_t c = 0;
            for (int q = 0; q < 4; q++) {
                int e = j * 4 + q;
                c += (((vmask >> e) & 1u) && kv[e] == kk) ? 1u : 0u;
            }
            uint32_t tot;
            uint32_t ex = block_excl_scan_u<ZS_P1_NT>(c, sh.u, &tot);
            uint32_t rank = carry + ex;
            for (int q = 0; q < 4; q++) {
                int e = j * 4 + q;
                if (((vmask >> e) & 1u) && kv[e] == kk) {
                    if (rank < need) {
                        uint32_t pos = atomicAdd(&sh.cnt, 1u);
                        if (pos < K) {
                            out_key[pos] = kv[e];
                            out_idx[pos] = base + (j * ZS_P1_NT + t) * 4 + q;
                        }
                    }
                    rank++;
                }
            }
            carry += tot;
        }
    }
    __syncthreads();
    *n_out = min(sh.cnt, K);
    *kth = kk;
    *full = (n_eq > need) ? 2u : 1u;  // 2: equal keys were left out
    __syncthreads();
}


// Fast exact top-K. Every wave sorts its 64 per-thread maxima; the c-th largest
// of them, c = ceil(K / 4), has at least c elements of its wave at or above
// it, so theta = the smallest of the four waves' values has at least K
// elements of the chunk at or above it: theta bounds the chunk's K-th largest
// key from below. The elements >= theta (a small superset of the top-K, with
// every element equal to the K-th key) are sorted by (key desc, index asc) --
// one wave for up to 64 of them, the workgroup for up to P1_SORT -- and the
// first K are the answer. Degenerate chunks (larger supersets) use the LDS
// radix select.
// nvalid: valid elements of the chunk; nfin: valid elements whose key is above
// that of -inf.
__device__ __forceinline__ void p1_topk_fast(const uint32_t (&kv)[P1_EPT], uint32_t vmask, uint32_t nvalid,
                             uint32_t nfin, uint32_t K, uint32_t base,
                             uint32_t* out_key, uint32_t* out_idx, uint32_t* n_out, uint32_t* kth,
                             uint32_t* full, p1_shared& sh) {
    const int t = threadIdx.x;
    uint32_t tm = 0;
#pragma unroll
    for (int e = 0; e < P1_EPT; e++)
        if ((vmask >> e) & 1u) tm = max(tm, kv[e]);
    const uint32_t c = (K + (ZS_P1_NT / 64) - 1) / (ZS_P1_NT / 64);
    if (nvalid <= K || c > 64) {
        p1_topk(kv, vmask, nvalid, K, base, out_key, out_idx, n_out, kth, full, sh);
        return;
    }
    // Fewer than K values above -inf (a masked chunk): all of them plus the
    // lowest-index -inf elements make the top-K.
    const uint32_t kninf = zs_total_key(-INFINITY);
    if (nfin < K) {
        if (t == 0) sh.cnt = 0;
        __syncthreads();
#pragma unroll
        for (int e = 0; e < P1_EPT; e++) {
            if (((vmask >> e) & 1u) && kv[e] > kninf) {
                const uint32_t p = atomicAdd(&sh.cnt, 1u);
                out_key[p] = kv[e];
                out_idx[p] = base + ((e >> 2) * ZS_P1_NT + t) * 4 + (e & 3);
            }
        }
        // -inf elements in index order: ids base + (j * NT + t) * 4 + q
        const uint32_t need = K - nfin;
        uint32_t carry = 0, ninf = 0;
        const uint32_t ninf_all = nvalid - nfin;
#pragma unroll
        for (int j = 0; j < P1_EPT / 4; j++) {
            if (carry >= need) break;  // uniform: the lowest ids are taken
            uint32_t cj = 0;
#pragma unroll
            for (int q = 0; q < 4; q++) cj += (((vmask >> (4 * j + q)) & 1u) && kv[4 * j + q] == kninf) ? 1u : 0u;
            uint32_t tot;
            uint32_t rank = carry + block_excl_scan_u<ZS_P1_NT>(cj, sh.u, &tot);
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int e = 4 * j + q;
                if (((vmask >> e) & 1u) && kv[e] == kninf) {
                    if (rank < need) {
                        out_key[nfin + rank] = kninf;
                        out_idx[nfin + rank] = base + (j * ZS_P1_NT + t) * 4 + q;
                    }
                    rank++;
                }
            }
            carry += tot;
            ninf += tot;
        }
        __syncthreads();
        (void)ninf;
        *n_out = min(K, nfin + ninf_all);
        *kth = kninf;
        *full = ninf_all > need ? 2u : 1u;
        __syncthreads();
        return;
    }
    // theta: a lower bound of the K-th largest key. Thread maxima belong to
    // distinct elements, so the K-th largest of the workgroup's 256 thread
    // maxima has at least K elements at or above it. Each wave sorts its 64;
    // for K <= 64 wave 0 merges the four sorted lists (elementwise max of an
    // ascending and a descending list keeps the larger half as a bitonic
    // sequence, which six exchange steps sort). For K > 64: the c-th largest
    // thread maximum of every wave, c = ceil(K / 4), and their minimum.
    // Threads without elements hold key 0, below every element.
    const int lane = zs_lane();
    const uint32_t srt = wave_sort_u32(tm);
    uint32_t theta;
    if (K <= 64) {
        sh.tmax[zs_wid() * 64 + lane] = srt;
        __syncthreads();
        if (t < 64) {
            uint32_t m = srt;
#pragma unroll
            for (int w = 1; w < ZS_P1_NT / 64; w++) {
                m = max(m, sh.tmax[w * 64 + 63 - lane]);
#pragma unroll
                for (int j = 32; j > 0; j >>= 1) {
                    const uint32_t o = __shfl_xor(m, j, 64);
                    m = (lane & j) ? max(m, o) : min(m, o);
                }
            }
            if (lane == 64 - (int)K) sh.sel[0] = m;
        }
        __syncthreads();
        theta = sh.sel[0];
    } else {
        const uint32_t thw = __shfl(srt, 64 - (int)c, 64);
        if (lane == 0) sh.sel[zs_wid()] = thw;
        __syncthreads();
        theta = sh.sel[0];
#pragma unroll
        for (int w = 1; w < ZS_P1_NT / 64; w++) theta = min(theta, sh.sel[w]);
    }
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < P1_EPT; e++) cnt += (((vmask >> e) & 1u) && kv[e] >= theta) ? 1u : 0u;
    uint32_t nsup;
    uint32_t pos = block_excl_scan_u<ZS_P1_NT>(cnt, sh.u, &nsup);
    if (nsup > P1_SORT) {
        p1_topk(kv, vmask, nvalid, K, base, out_key, out_idx, n_out, kth, full, sh);
        return;
    }
    // composite ((~key) << 32 | index): ascending order = key desc, index asc
#pragma unroll
    for (int e = 0; e < P1_EPT; e++) {
        if (((vmask >> e) & 1u) && kv[e] >= theta) {
            const uint32_t idx = base + ((e >> 2) * ZS_P1_NT + t) * 4 + (e & 3);
            sh.s64[pos++] = ((unsigned long long)(~kv[e]) << 32) | idx;
        }
    }
    __syncthreads();
    if (nsup <= 64) {
        if (t < 64) {
            unsigned long long v = (uint32_t)t < nsup ? sh.s64[t] : ~0ull;
            v = wave_sort_u64(v);
            const unsigned long long vk = __shfl(v, (int)K - 1, 64);
            const unsigned long long vn = __shfl(v, min((int)K, 63), 64);
            if ((uint32_t)t < K) { out_key[t] = ~(uint32_t)(v >> 32); out_idx[t] = (uint32_t)v; }
            if (t == 0) {
                sh.sel[0] = ~(uint32_t)(vk >> 32);
                sh.sel[1] = (K < nsup && (uint32_t)(vn >> 32) == (uint32_t)(vk >> 32)) ? 2u : 1u;
            }
        }
    } else {
        for (uint32_t i = nsup + t; i < P1_SORT; i += ZS_P1_NT) sh.s64[i] = ~0ull;
        __syncthreads();
        block_sort_reg_u64<ZS_P1_NT, P1_SORT / ZS_P1_NT>(sh.s64, P1_SORT);
        for (uint32_t i = t; i < K; i += ZS_P1_NT) {
            const unsigned long long v = sh.s64[i];
            out_key[i] = ~(uint32_t)(v >> 32);
            out_idx[i] = (uint32_t)v;
        }
        if (t == 0) {
            const uint32_t hk = (uint32_t)(sh.s64[K - 1] >> 32);
            sh.sel[0] = ~hk;
            sh.sel[1] = (K < nsup && (uint32_t)(sh.s64[K] >> 32) == hk) ? 2u : 1u;
        }
    }
    __syncthreads();
    *n_out = K;
    *kth = sh.sel[0];
    *full = sh.sel[1];
    __syncthreads();
}

// Observer candidates without the exact cut: every element whose key is at
// least theta, the K-th largest thread maximum (K <= 64), when at most `cap`
// of them exist. The list then holds the chunk's top K (and possibly more), in
// any order -- what the combine kernel's merge needs. Returns false (nothing
// written) when more than `cap` elements reach theta.
__device__ __forceinline__ bool p1_superset(const uint32_t (&kv)[P1_EPT], uint32_t vmask, uint32_t K, uint32_t cap,
                                            uint32_t base, uint32_t* out_key, uint32_t* out_idx, uint32_t* n_out,
                                            p1_shared& sh) {
    const int t = threadIdx.x, lane = zs_lane();
    uint32_t tm = 0;
#pragma unroll
    for (int e = 0; e < P1_EPT; e++)
        if ((vmask >> e) & 1u) tm = max(tm, kv[e]);
    const uint32_t srt = wave_sort_u32(tm);
    sh.tmax[zs_wid() * 64 + lane] = srt;
    if (t == 0) sh.cnt = 0;
    __syncthreads();
    if (t < 64) {
        uint32_t m = srt;
#pragma unroll
        for (int w = 1; w < ZS_P1_NT / 64; w++) {
            m = max(m, sh.tmax[w * 64 + 63 - lane]);
#pragma unroll
            for (int j = 32; j > 0; j >>= 1) {
                const uint32_t o = __shfl_xor(m, j, 64);
                m = (lane & j) ? max(m, o) : min(m, o);
            }
        }
        if (lane == 64 - (int)K) sh.sel[2] = m;
    }
    __syncthreads();
    const uint32_t theta = max(sh.sel[2], 1u);
    uint32_t cnt = 0;
#pragma unroll
    for (int e = 0; e < P1_EPT; e++) cnt += (((vmask >> e) & 1u) && kv[e] >= theta) ? 1u : 0u;
    const uint32_t nsup = block_sum_u<ZS_P1_NT>(cnt, sh.u);
    if (nsup > cap) return false;
#pragma unroll
    for (int e = 0; e < P1_EPT; e++) {
        if (((vmask >> e) & 1u) && kv[e] >= theta) {
            const uint32_t p = atomicAdd(&sh.cnt, 1u);
            out_key[p] = kv[e];
            out_idx[p] = base + ((e >> 2) * ZS_P1_NT + t) * 4 + (e & 3);
        }
    }
    *n_out = nsup;
    return true;
}

// Compaction of the chunk's finite sampler values (the list when the chunk has
// at most K of them: then it holds every element a top-k or a small-survivor
// path can keep).
__device__ __forceinline__ void p1_finite(const uint32_t (&zv)[P1_EPT], uint32_t vmask,
                          uint32_t base, uint32_t* out_key, uint32_t* out_idx, p1_shared& sh) {
    const int t = threadIdx.x;
    uint32_t cnt = 0;
    const uint32_t kninf = zs_total_key(-INFINITY), kpinf = zs_total_key(INFINITY);
    // z > -inf: keys above that of -inf, NaN (above +inf) excluded
#pragma unroll
    for (int e = 0; e < P1_EPT; e++) cnt += (((vmask >> e) & 1u) && zv[e] > kninf && zv[e] <= kpinf) ? 1u : 0u;
    uint32_t tot;
    uint32_t pos = block_excl_scan_u<ZS_P1_NT>(cnt, sh.u, &tot);
#pragma unroll
    for (int e = 0; e < P1_EPT; e++) {
        if (((vmask >> e) & 1u) && zv[e] > kninf && zv[e] <= kpinf) {
            out_key[pos] = zv[e];
            out_idx[pos] = base + ((e >> 2) * ZS_P1_NT + t) * 4 + (e & 3);
            pos++;
        }
    }
}

// element e of the calling thread in a [P1_EPT][ZS_P1_NT] LDS array
struct p1_lds_arr {
    uint32_t* p;
    __device__ __forceinline__ uint32_t& operator[](int e) const { return p[e * ZS_P1_NT]; }
};

__global__ __launch_bounds__(ZS_P1_NT) __attribute__((amdgpu_waves_per_eu(3))) void zs_k_pass1(zs_sargs a) {
    const uint32_t c = blockIdx.x, r = blockIdx.y;
    const zs_batch& b = a.b;
    const uint32_t V = b.V;
    const uint32_t base = c * ZS_P1_CH;
    if (base >= V) return;
    __shared__ p1_shared sh;
    const int t = threadIdx.x;
    const zs_row_params P = b.d_params[r];
    const float T = P.temperature;
    const bool masked = (P.flags & ZS_ROW_MASKED) && b.d_allow_bits;
    const float* row = b.d_logits + (size_t)r * b.ld;

    // patch range of this chunk (patch ids are sorted; zs_k_prep stored the
    // first patch of every 1024-id sub-chunk)
    const uint32_t* pid = a.p_id + (size_t)r * ZS_MAX_PATCHES;
    const uint32_t* psub = a.p_sub + (size_t)r * (a.max_subs + 1);
    const uint32_t nsub_row = (V + ZS_SUB - 1) / ZS_SUB;
    const uint32_t pc0 = psub[c * ZS_SUBS_PER_CHUNK];
    const uint32_t pc1 = psub[min((c + 1) * ZS_SUBS_PER_CHUNK, nsub_row)];

    // x~ lives in LDS as total-order keys (thread t's element e at xsh[e][t])
    // until the observer list, z in registers (keys after the temperature):
    // both arrays in registers would halve occupancy. Every later use compares
    // keys; the float is recovered where arithmetic needs it.
    __shared__ uint32_t xsh[P1_EPT][ZS_P1_NT];
    const p1_lds_arr xo{&xsh[0][t]};
    const uint32_t kninf = zs_total_key(-INFINITY), kpinf = zs_total_key(INFINITY);
    float zv[P1_EPT];
    uint32_t vmask = 0;
#pragma unroll
    for (int j = 0; j < P1_EPT / 4; j++) {
        uint32_t idx = base + (j * ZS_P1_NT + t) * 4;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        uint32_t w = 0xffffffffu;
        if (idx < V) {
            v = *reinterpret_cast<const float4*>(row + idx);
            if (masked) w = b.d_allow_bits[(size_t)r * b.allow_words + (idx >> 5)] >> (idx & 31);
        }
        float vv[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            int e = j * 4 + q;
            bool valid = idx + q < V;
            float x = vv[q];
            if (masked && !((w >> q) & 1u)) x = -INFINITY;
            if (!valid) x = -INFINITY;  // neutral in every statistic
            xo[e] = zs_total_key(x);
            zv[e] = x;
            if (valid) vmask |= 1u << e;
        }
    }
    __syncthreads();
    // patches: bans change x~, bias/penalty set y. Staged through LDS a
    // batch at a time (one load per thread), then each thread applies those
    // that fall on its elements.
    {
        const uint32_t* pfl = a.p_flags + (size_t)r * ZS_MAX_PATCHES;
        const float* py = a.p_y + (size_t)r * ZS_MAX_PATCHES;
        for (uint32_t pb = pc0; pb < pc1; pb += ZS_P1_NT) {
            const uint32_t n = min((uint32_t)ZS_P1_NT, pc1 - pb);
            if ((uint32_t)t < n) {
                sh.skey[t] = pid[pb + t] - base;
                sh.sidx[t] = pfl[pb + t];
                sh.tmax[t] = zs_f2u(py[pb + t]);
            }
            __syncthreads();
            for (uint32_t i = 0; i < n; i++) {
                const uint32_t off = sh.skey[i];
                const uint32_t q = off & 3, tt = (off >> 2) % ZS_P1_NT, j = (off >> 2) / ZS_P1_NT;
                if ((int)tt != t) continue;
                const uint32_t fl = sh.sidx[i];
                const float y = zs_u2f(sh.tmax[i]);
#pragma unroll
                for (int jj = 0; jj < P1_EPT / 4; jj++)
#pragma unroll
                    for (int qq = 0; qq < 4; qq++)
                        if (jj == (int)j && qq == (int)q) {
                            if (fl & ZS_PF_BAN) { xo[jj * 4 + qq] = kninf; zv[jj * 4 + qq] = -INFINITY; }
                            if (fl & ZS_PF_Y) zv[jj * 4 + qq] = y;
                        }
            }
            __syncthreads();
        }
    }
    // z = y / T, kept as keys
    uint32_t kz[P1_EPT];
#pragma unroll
    for (int e = 0; e < P1_EPT; e++) kz[e] = zs_total_key(zs_temper(zv[e], T));

    // ---- chunk statistics of x~ (observers) and z (sampler), one workgroup
    // reduction: maxima, NaN / +inf flags, the last NaN of z, and counts of
    // finite z and of elements whose key is above that of -inf for the lists
    // branch-free on keys: NaN keys lie above +inf's (positive) or below
    // -inf's (negative); the maxima skip them (fmaxf semantics); the rare
    // waves with a NaN z redo their elements for the last NaN and the finite
    // count (+inf counts as finite there: the test is z > -inf)
    uint32_t okm = kninf, zkm = kninf;
    uint32_t fl = 0, zfin, zabove = 0, xabove = 0;
    bool xnan = false, znan = false;
    int last_nan = -1;
#pragma unroll
    for (int e = 0; e < P1_EPT; e++) {
        const uint32_t kx = xo[e], k = kz[e];
        xnan |= (kx > kpinf) | (kx < kninf);
        znan |= (k > kpinf) | (k < kninf);
        okm = max(okm, kx <= kpinf ? kx : kninf);
        zkm = max(zkm, k <= kpinf ? k : kninf);
        xabove += kx > kninf ? 1u : 0u;
        zabove += k > kninf ? 1u : 0u;
    }
    zfin = zabove;
    if (__ballot(znan)) {
        zfin = 0;
#pragma unroll
        for (int e = 0; e < P1_EPT; e++) {
            if (!((vmask >> e) & 1u)) continue;
            const uint32_t k = kz[e];
            const uint32_t idx = base + ((e >> 2) * ZS_P1_NT + t) * 4 + (e & 3);
            if (k > kpinf || k < kninf) last_nan = max(last_nan, (int)idx);
            zfin += (k > kninf && k <= kpinf) ? 1u : 0u;
        }
    }
    if (xnan) fl |= ZS_CF_OBS_NAN;
    if (znan) fl |= ZS_CF_Z_NAN;
    if (zkm == kpinf) fl |= ZS_CF_Z_PINF;
    float omax = zs_key_to_float(okm), zmax = zs_key_to_float(zkm);
    for (int d = 32; d > 0; d >>= 1) {
        omax = fmaxf(omax, __shfl_xor(omax, d, 64));
        zmax = fmaxf(zmax, __shfl_xor(zmax, d, 64));
        fl |= __shfl_xor(fl, d, 64);
        zfin += __shfl_xor(zfin, d, 64);
        zabove += __shfl_xor(zabove, d, 64);
        xabove += __shfl_xor(xabove, d, 64);
        last_nan = max(last_nan, __shfl_xor(last_nan, d, 64));
    }
    if (zs_lane() == 0) {
        p1_red& R = sh.red[zs_wid()];
        R.omax = omax; R.zmax = zmax; R.fl = fl; R.zfin = zfin;
        R.zabove = zabove; R.xabove = xabove; R.last_nan = last_nan;
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < ZS_P1_NT / 64; w++) {
        const p1_red& R = sh.red[w];
        omax = fmaxf(omax, R.omax); zmax = fmaxf(zmax, R.zmax); fl |= R.fl;
        last_nan = max(last_nan, R.last_nan);
    }
    zfin = zabove = xabove = 0;
#pragma unroll
    for (int w = 0; w < ZS_P1_NT / 64; w++) {
        zfin += sh.red[w].zfin; zabove += sh.red[w].zabove; xabove += sh.red[w].xabove;
    }
    const uint32_t nvalid = min((uint32_t)ZS_P1_CH, V - base);
    // greedy: argmax-last (ties -> larger index) over all, and over the tail
    // after the chunk's last NaN (the whole chunk when it has no NaN). A pair
    // (value key, index + 1) compares by key, then by index; 0 = none.
    unsigned long long best_all = 0, best_tail = 0;
    int tail_n = 0;
    if (T <= 0.0f) {  // greedy rows only (uniform per workgroup)
        uint32_t bk = 0, bi = 0, tk = 0, ti = 0;
        uint32_t tn = 0;
#pragma unroll
        for (int e = 0; e < P1_EPT; e++) {
            const float z = zs_key_to_float(kz[e]);
            if (!((vmask >> e) & 1u) || z != z) continue;
            const uint32_t idx = base + ((e >> 2) * ZS_P1_NT + t) * 4 + (e & 3);
            // -0.0 and +0.0 compare equal in the reference (partial_cmp): map both to +0
            const uint32_t k = zs_total_key(z == 0.0f ? 0.0f : z);
            if (k >= bk) { bk = k; bi = idx + 1; }  // ids ascend with e: ties -> later
            if ((int)idx > last_nan) {
                tn++;
                if (k >= tk) { tk = k; ti = idx + 1; }
            }
        }
        best_all = ((unsigned long long)bk << 32) | bi;
        best_tail = ((unsigned long long)tk << 32) | ti;
        __shared__ unsigned long long u64sh[2][ZS_P1_NT / 64];
        for (int d = 32; d > 0; d >>= 1) {
            unsigned long long o1 = __shfl_xor(best_all, d, 64);
            unsigned long long o2 = __shfl_xor(best_tail, d, 64);
            best_all = o1 > best_all ? o1 : best_all;
            best_tail = o2 > best_tail ? o2 : best_tail;
        }
        if (zs_lane() == 0) { u64sh[0][zs_wid()] = best_all; u64sh[1][zs_wid()] = best_tail; }
        __syncthreads();
        for (int i = 0; i < ZS_P1_NT / 64; i++) {
            best_all = u64sh[0][i] > best_all ? u64sh[0][i] : best_all;
            best_tail = u64sh[1][i] > best_tail ? u64sh[1][i] : best_tail;
        }
        __syncthreads();
        tail_n = (int)block_sum_u<ZS_P1_NT>(tn, sh.u);
    }

    // ---- approximate moments per 1024-logit sub-chunk (predictions for the
    // exact-sum rounds). Float4 j of thread t holds ids base + (j*NT + t)*4..+3,
    // so it lies in sub-chunk j*P1_SPF + t*4/1024 of the chunk: a wave's float4
    // row lies inside one sub-chunk, and four waves make up a sub-chunk row.
    {
        constexpr int P1_SPF = ZS_P1_NT * 4 / ZS_SUB;  // sub-chunks per float4 row
        constexpr int P1_J = P1_EPT / 4;
        static_assert(P1_SPF * P1_J == ZS_SUBS_PER_CHUNK, "float4 rows tile the sub-chunks");
        const int wid = zs_wid(), wh = (wid * 256) / ZS_SUB;
        const bool om = (P.flags & (ZS_ROW_LOGPROBS | ZS_ROW_UNCERTAINTY)) && omax > -INFINITY && omax < INFINITY;
        const bool zm = T > 0.0f && zmax > -INFINITY && zmax < INFINITY;
        __shared__ float msh[ZS_P1_NT / 64][P1_J][3];
        // bit 2s: sub-chunk s holds the chunk's observer max, bit 2s+1: its sampler max
        uint32_t hasmax = 0;
        static_assert(P1_J == 8, "the reduce-scatter below splits 8 rows over 3 lane bits");
        float mv[3][P1_J];
#pragma unroll
        for (int j = 0; j < P1_J; j++) {
            float m1 = 0.0f, md = 0.0f, mz = 0.0f;
            const int sj = j * P1_SPF + wh;
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int e = j * 4 + q;
                if (!((vmask >> e) & 1u)) continue;
                const float xe = zs_key_to_float(xo[e]), ze = zs_key_to_float(kz[e]);
                if (xe == omax) hasmax |= 1u << (2 * sj);
                if (ze == zmax) hasmax |= 2u << (2 * sj);
                if (om) {
                    float d = xe - omax;
                    if (d > -INFINITY) { float ex = __expf(d); m1 += ex; md += d * ex; }
                }
                if (zm) {
                    float d = ze - zmax;
                    if (d > -INFINITY) mz += __expf(d);
                }
            }
            mv[0][j] = m1; mv[1][j] = md; mv[2][j] = mz;
        }
        // reduce-scatter over the wave: each exchange halves the rows a lane
        // keeps (lane bits 5, 4, 3 pick them), then 8-lane sums; lane 8j ends
        // with row j's totals
        {
            const uint32_t lane = (uint32_t)zs_lane();
#pragma unroll
            for (int u = 0; u < 3; u++) {
                float v4[4], v2[2];
                const bool h5 = (lane & 32u) != 0, h4 = (lane & 16u) != 0, h3 = (lane & 8u) != 0;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    const float send = h5 ? mv[u][k] : mv[u][k + 4];
                    v4[k] = (h5 ? mv[u][k + 4] : mv[u][k]) + __shfl_xor(send, 32, 64);
                }
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const float send = h4 ? v4[k] : v4[k + 2];
                    v2[k] = (h4 ? v4[k + 2] : v4[k]) + __shfl_xor(send, 16, 64);
                }
                float v1 = (h3 ? v2[1] : v2[0]) + __shfl_xor(h3 ? v2[0] : v2[1], 8, 64);
                v1 += __shfl_xor(v1, 4, 64);
                v1 += __shfl_xor(v1, 2, 64);
                v1 += __shfl_xor(v1, 1, 64);
                if ((lane & 7u) == 0) msh[wid][lane >> 3][u] = v1;
            }
        }
        for (int d = 32; d > 0; d >>= 1) hasmax |= __shfl_xor(hasmax, d, 64);
        __shared__ uint32_t hsh[ZS_P1_NT / 64];
        if (zs_lane() == 0) hsh[wid] = hasmax;
        __syncthreads();
        if (t < ZS_SUBS_PER_CHUNK) {
            const int j = t / P1_SPF, h = t % P1_SPF;
            zs_sub_mom mm;
            mm.e1 = mm.ed = mm.ez = 0.0f;
            uint32_t hm = 0;
            for (int w = 0; w < ZS_P1_NT / 64; w++) {
                hm |= hsh[w];
                if ((w * 256) / ZS_SUB != h) continue;
                mm.e1 += msh[w][j][0]; mm.ed += msh[w][j][1]; mm.ez += msh[w][j][2];
            }
            mm.pad = zs_u2f((hm >> (2 * t)) & 3u);
            const uint32_t sub = c * ZS_SUBS_PER_CHUNK + t;
            if (sub * ZS_SUB < V) a.sub_mom[(size_t)r * a.max_subs + sub] = mm;
        }
        __syncthreads();
    }

    // ---- candidate lists (keys recomputed from the values where needed)
    const size_t lofs = ((size_t)r * a.nch + c);
    // sampler list size: top_k when the row has a top-k cut within range
    const bool has_topk = P.top_k > 0 && P.top_k < V;
    const uint32_t Ks = (has_topk && P.top_k <= ZS_KS) ? P.top_k : ZS_KS;
    uint32_t ns, s_kth, s_full;
    ns = s_kth = s_full = 0;
    // The list is read by a top-k cut within ZS_KS and by the small-survivor
    // path, which needs every chunk to have at most ZS_KS finite values.
    if (T > 0.0f) {
        if (zfin <= Ks) {
            p1_finite(kz, vmask, base, a.cs_key + lofs * ZS_KS, a.cs_idx + lofs * ZS_KS, sh);
            ns = zfin;
        } else if (has_topk && P.top_k <= ZS_KS) {
            p1_topk_fast(kz, vmask, nvalid, zabove, Ks, base, a.cs_key + lofs * ZS_KS, a.cs_idx + lofs * ZS_KS, &ns, &s_kth,
                         &s_full, sh);
        }
    }
    uint32_t ntl = P.top_logprobs > 20 ? 20 : P.top_logprobs;
    uint32_t Ko = ntl + 8;
    if (Ko > ZS_KO) Ko = ZS_KO;
    uint32_t no, o_kth, o_full;
    no = o_kth = o_full = 0;
    uint32_t xr[P1_EPT];  // z is dead here: x~ keys back in registers for the list
#pragma unroll
    for (int e = 0; e < P1_EPT; e++) xr[e] = xo[e];
    if ((P.flags & (ZS_ROW_LOGPROBS | ZS_ROW_UNCERTAINTY)) &&
        !(nvalid > Ko && p1_superset(xr, vmask, Ko, ZS_KO, base, a.co_key + lofs * ZS_KO, a.co_idx + lofs * ZS_KO,
                                     &no, sh)))
        p1_topk_fast(xr, vmask, nvalid, xabove, Ko, base, a.co_key + lofs * ZS_KO, a.co_idx + lofs * ZS_KO, &no, &o_kth,
                     &o_full, sh);

    if (t == 0) {
        zs_chunk_stat cs;
        cs.obs_max = omax;
        cs.z_max = zmax;
        cs.flags = fl;
        cs.z_finite = zfin;
        cs.g_last_nan = last_nan;
        cs.g_arg_all = best_all ? (uint32_t)(best_all & 0xffffffffull) - 1u : 0xffffffffu;
        cs.g_val_all = best_all ? zs_key_to_float((uint32_t)(best_all >> 32)) : -INFINITY;
        cs.g_arg_tail = best_tail ? (uint32_t)(best_tail & 0xffffffffull) - 1u : 0xffffffffu;
        cs.g_val_tail = best_tail ? zs_key_to_float((uint32_t)(best_tail >> 32)) : -INFINITY;
        cs.g_tail_n = tail_n;
        cs.ns = ns;
        cs.no = no;
        cs.s_kth = s_kth;
        cs.o_kth = o_kth;
        cs.s_full = s_full;
        cs.o_full = o_full;
        a.cst[lofs] = cs;
    }
}

// ===========================================================================
// zs_k_combine
// ===========================================================================

// Predicted grid of a sequential sum at each sub-chunk start from approximate
// sub-chunk sums A_j (one wave, 4 sub-chunks per lane). A sub-chunk is fragile
// -- processed exactly by the stitch -- when the running sum may leave its
// binade inside it or sits too close to a binade edge for the prediction to be
// trusted (the f32 sum differs from the exact prefix by far less than 2^-8).
// ONE(j) tells whether sub-chunk j holds the term exp(0) = 1 exactly: an f32
// running sum of non-negative terms never decreases, so once that term is in,
// the sum is >= 1 and the lower edge of [1, 2) cannot be crossed -- without
// this, the common peaked rows (sum just above 1) would be fragile throughout.
// A misprediction only costs an exact pass: the stitch checks every grid.
template <class F, class G>
__device__ void zs_predict_subs(zs_sub_sum* out, uint32_t nsub, const F& A, const G& ONE, bool all_fragile) {
    const int lane = zs_lane();
    double v[4], loc = 0.0;
    int j1 = ZS_BIGI;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        uint32_t j = 4 * lane + q;
        v[q] = j < nsub ? A(j) : 0.0;
        loc += v[q];
        if (j < nsub && j1 == ZS_BIGI && ONE(j)) j1 = (int)j;
    }
    j1 = wave_min_i(j1);
    double inc = loc;
    for (int d = 1; d < 64; d <<= 1) {
        double y = __shfl_up(inc, d, 64);
        if (lane >= d) inc += y;
    }
    double run = inc - loc;
    const double delta = 1.0 / 256.0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        uint32_t j = 4 * lane + q;
        double lo = run, hi = run + v[q];
        run = hi;
        if (j >= nsub) continue;
        zs_sub_sum e;
        double lm = lo * (1.0 - delta), hm = hi * (1.0 + delta);
        if ((int)j > j1) {
            lm = fmax(lm, 1.0);
            lo = fmax(lo, 1.0);
        }
        // every sum below 2^-125 lies on the finest grid (2^-149), so tiny
        // prefixes share one binade
        const int blo = lm < 0x1p-125 ? -125 : ilogb(lm);
        const int bhi = hm < 0x1p-125 ? -125 : ilogb(hm);
        bool fragile = all_fragile || !(lm >= 0.0) || blo != bhi || !(hm < 3.0e38);
        e.eg = fragile ? 0 : zs_grid_exp((float)lo);
        e.flags = fragile ? ZS_SF_FRAGILE : 0u;
        e.total = 0;
        e.pad = 0;
        out[j] = e;
    }
}

#define CB_NT 256
__global__ __launch_bounds__(CB_NT) void zs_k_combine(zs_sargs a) {
    const uint32_t r = blockIdx.x;
    const zs_batch& b = a.b;
    const uint32_t V = b.V;
    const int t = threadIdx.x;
    const uint32_t nch = (V + ZS_P1_CH - 1) / ZS_P1_CH;
    __shared__ unsigned long long sbuf[ZS_MAX_CHUNKS * ZS_KS];
    __shared__ float sval[ZS_SMALL_CAP];
    __shared__ uint32_t sidx[ZS_SMALL_CAP];
    __shared__ seq_sh<CB_NT> sq;
    __shared__ uint32_t n_sh;
    __shared__ uint32_t cid_sh[ZS_OBS_CAND];
    __shared__ float cx_sh[ZS_OBS_CAND];
    const zs_row_params P = b.d_params[r];
    // the row state is written field by field by thread 0 (a private copy of
    // the whole struct per thread would live in scratch memory)
    zs_row_state& st = a.rst[r];
    if (st.status & ZS_ST_LIMIT) {
        if (t == 0) {
            st.mode = ZS_MODE_DONE;
            st.token = 0xffffffffu;
            st.obs_need = 0;
            st.rounds = 0;
            st.n_cand = 0;
            st.klist = 0;
            st.kpend = 0;
        }
        return;
    }
    // the row's chunk statistics in LDS (one parallel load; the loops over
    // chunks below would otherwise wait on one global load per chunk)
    __shared__ zs_chunk_stat cs_sh[ZS_MAX_CHUNKS];
    {
        static_assert(sizeof(zs_chunk_stat) % 4 == 0, "word copy");
        constexpr uint32_t W = sizeof(zs_chunk_stat) / 4;
        const uint32_t* src = reinterpret_cast<const uint32_t*>(a.cst + (size_t)r * a.nch);
        uint32_t* dst = reinterpret_cast<uint32_t*>(cs_sh);
        for (uint32_t i = t; i < nch * W; i += CB_NT) dst[i] = src[i];
    }
    __syncthreads();
    const zs_chunk_stat* cs = cs_sh;

    // ---------------- observers: max, special rows, top candidates ----------------
    float M = -INFINITY;
    uint32_t fl = 0;
    for (uint32_t c = 0; c < nch; c++) { M = fmaxf(M, cs[c].obs_max); fl |= cs[c].flags; }
    // lse = max + ln(sum) is NaN for a NaN, a +inf or an all -inf row
    const bool special = (fl & ZS_CF_OBS_NAN) || M == INFINITY || M == -INFINITY;
    const bool want_lp = (P.flags & ZS_ROW_LOGPROBS) != 0;
    const bool want_unc = (P.flags & ZS_ROW_UNCERTAINTY) != 0;
    uint32_t status = 0;
    uint32_t obs_need = 0;
    if (!special && (want_lp || want_unc)) obs_need |= ZS_OBS_S;
    if (!special && want_unc) obs_need |= ZS_OBS_H;
    uint32_t n_cand = 0;
    if (want_lp || want_unc) {
        if (t == 0) n_sh = 0;
        __syncthreads();
        {
            // all chunks' lists at once (their order in sbuf does not matter: sorted next)
            const uint32_t* kk = a.co_key + (size_t)r * a.nch * ZS_KO;
            const uint32_t* ii = a.co_idx + (size_t)r * a.nch * ZS_KO;
            for (uint32_t i = t; i < nch * ZS_KO; i += CB_NT) {
                if (i % ZS_KO >= cs[i / ZS_KO].no) continue;
                uint32_t pos = atomicAdd(&n_sh, 1u);
                sbuf[pos] = ((unsigned long long)(~kk[i]) << 32) | ii[i];
            }
        }
        __syncthreads();
        uint32_t nco = n_sh;
        uint32_t np2 = 1;
        while (np2 < nco) np2 <<= 1;
        for (uint32_t i = nco + t; i < np2; i += CB_NT) sbuf[i] = ~0ull;
        __syncthreads();
        if (np2 > 1) block_sort_u64<CB_NT>(sbuf, np2);
        n_cand = nco < ZS_OBS_CAND ? nco : ZS_OBS_CAND;
        if (t < (int)n_cand) {
            cid_sh[t] = (uint32_t)(sbuf[t] & 0xffffffffull);
            cx_sh[t] = zs_key_to_float(~(uint32_t)(sbuf[t] >> 32));
        }
        __syncthreads();
    }
    // the sampler sees x~ itself when T == 1 and no bias / penalty applies
    uint32_t has_y = 0;
    {
        const uint32_t np = a.p_cnt[r];
        const uint32_t* pfl = a.p_flags + (size_t)r * ZS_MAX_PATCHES;
        for (uint32_t i = t; i < np; i += CB_NT) has_y |= (pfl[i] & ZS_PF_Y) ? 1u : 0u;
        has_y = block_or_u<CB_NT>(has_y, sq.a);
    }
    const uint32_t z_is_x = (P.temperature == 1.0f && !has_y) ? 1u : 0u;

    // ---------------- sampler ----------------
    const float T = P.temperature;
    uint32_t token = 0;
    uint32_t mode = ZS_MODE_DONE;
    uint32_t has_thr = 0, thr_key = 0;
    float zmax = -INFINITY;
    for (uint32_t c = 0; c < nch; c++) zmax = fmaxf(zmax, cs[c].z_max);
    if (T <= 0.0f) {
        // sampler.rs:35-42, max_by over partial_cmp: the last maximal element,
        // and a NaN restarts the fold (partial_cmp -> Equal keeps the later one).
        status |= ZS_ST_GREEDY;
        int L = -1;
        for (uint32_t c = 0; c < nch; c++) L = max(L, cs[c].g_last_nan);
        float bv = 0.f;
        uint32_t bi = 0xffffffffu;
        bool any = false;
        uint32_t cstart = 0;
        if (L >= 0) {
            uint32_t cl = (uint32_t)L / ZS_P1_CH;
            if (cs[cl].g_tail_n > 0) { bv = cs[cl].g_val_tail; bi = cs[cl].g_arg_tail; any = true; }
            cstart = cl + 1;
        }
        for (uint32_t c = cstart; c < nch; c++) {
            if (cs[c].g_arg_all == 0xffffffffu) continue;
            float v = cs[c].g_val_all;
            if (!any || !(bv > v)) { bv = v; bi = cs[c].g_arg_all; any = true; }
        }
        token = any ? bi : (uint32_t)L;
        if (!any && L < 0) token = 0;
    } else if ((fl & (ZS_CF_Z_NAN | ZS_CF_Z_PINF)) || zmax == -INFINITY) {
        // exp_sum is NaN: every comparison in the draw fails -> V-1 (sampler.rs:127)
        status |= ZS_ST_NONFINITE;
        token = V - 1;
    } else {
        const bool has_topk = P.top_k > 0 && P.top_k < V;
        // gather sampler candidates
        if (t == 0) n_sh = 0;
        __syncthreads();
        {
            const uint32_t* kk = a.cs_key + (size_t)r * a.nch * ZS_KS;
            const uint32_t* ii = a.cs_idx + (size_t)r * a.nch * ZS_KS;
#pragma unroll 4
            for (uint32_t i = t; i < nch * ZS_KS; i += CB_NT) {
                if (i % ZS_KS >= cs[i / ZS_KS].ns) continue;
                uint32_t pos = atomicAdd(&n_sh, 1u);
                sbuf[pos] = ((unsigned long long)(~kk[i]) << 32) | ii[i];
            }
        }
        __syncthreads();
        uint32_t ncs = n_sh;
        uint32_t np2 = 1;
        while (np2 < ncs) np2 <<= 1;
        for (uint32_t i = ncs + t; i < np2; i += CB_NT) sbuf[i] = ~0ull;
        __syncthreads();
        if (np2 > 1) block_sort_u64<CB_NT>(sbuf, np2);
        bool small = false;
        float thr = -INFINITY;
        if (has_topk && P.top_k <= ZS_KS) {
            // fewer listed values than k: every finite value is listed and the
            // k-th largest of the row is -inf
            thr_key = P.top_k <= ncs ? ~(uint32_t)(sbuf[P.top_k - 1] >> 32) : zs_total_key(-INFINITY);
            has_thr = 1;
            thr = zs_key_to_float(thr_key);
            bool complete = true;
            for (uint32_t c = 0; c < nch; c++) {
                if (!cs[c].s_full) continue;
                if (cs[c].s_kth == thr_key && cs[c].s_full == 2) complete = false;
                if (thr == 0.0f) complete = false;  // the other zero also survives
            }
            small = complete;
        } else if (has_topk) {
            has_thr = 2;
        } else {
            uint32_t fin = 0;
            bool ok = true;
            for (uint32_t c = 0; c < nch; c++) {
                fin += cs[c].z_finite;
                if (cs[c].z_finite > ZS_KS) ok = false;
            }
            small = ok && fin <= ZS_SMALL_CAP;
        }
        if (small) {
            // survivors: !(z < thr) (sampler.rs:59-63) and finite, gathered by index
            if (t == 0) n_sh = 0;
            __syncthreads();
            for (uint32_t i = t; i < ncs; i += CB_NT) {
                float z = zs_key_to_float(~(uint32_t)(sbuf[i] >> 32));
                bool surv = !(z < thr) && z > -INFINITY;
                if (surv) {
                    uint32_t pos = atomicAdd(&n_sh, 1u);
                    if (pos < ZS_SMALL_CAP) { sval[pos] = z; sidx[pos] = (uint32_t)(sbuf[i] & 0xffffffffull); }
                }
            }
            __syncthreads();
            uint32_t n = n_sh;
            __syncthreads();
            if (n > ZS_SMALL_CAP) {
                small = false;
            } else {
                if (t < 64) {
                    const uint32_t tk = n <= 64 ? small_path_wave<1>(b.d_seed[r], b.d_counter[r], V, P, n, zmax, sval, sidx)
                                                : small_path_wave<ZS_SMALL_CAP / 64>(b.d_seed[r], b.d_counter[r], V, P, n, zmax, sval, sidx);
                    if (t == 0) n_sh = tk;
                }
                __syncthreads();
                token = n_sh;
                status |= ZS_ST_SMALL;
            }
        }
        if (!small) mode = ZS_MODE_BIG;
    }
    // ---- predictions for the parallel exact-sum rounds
    uint32_t rounds = 0;
    {
        const uint32_t nsub = (V + ZS_SUB - 1) / ZS_SUB;
        const zs_sub_mom* mom = a.sub_mom + (size_t)r * a.max_subs;
        if (obs_need & ZS_OBS_S) {
            rounds |= 1u << ZS_SUM_OBS_S;
            if (t < 64)
                zs_predict_subs(a.sub_sum + ((size_t)r * ZS_NSUM + ZS_SUM_OBS_S) * a.max_subs, nsub,
                                [&](uint32_t j) {
                                    float mc = cs[j / ZS_SUBS_PER_CHUNK].obs_max;
                                    return (double)mom[j].e1 * exp((double)mc - (double)M);
                                },
                                [&](uint32_t j) {
                                    return (zs_f2u(mom[j].pad) & 1u) && cs[j / ZS_SUBS_PER_CHUNK].obs_max == M;
                                },
                                false);
        }
        const bool reuse = z_is_x && !has_thr && (obs_need & ZS_OBS_S);
        if (mode == ZS_MODE_BIG && !reuse && has_thr != 2) {  // has_thr 2: threshold found later
            rounds |= 1u << ZS_SUM_SAMP_S;
            if (t < 64)
                zs_predict_subs(a.sub_sum + ((size_t)r * ZS_NSUM + ZS_SUM_SAMP_S) * a.max_subs, nsub,
                                [&](uint32_t j) {
                                    float mc = cs[j / ZS_SUBS_PER_CHUNK].z_max;
                                    return mc > -INFINITY ? (double)mom[j].ez * exp((double)mc - (double)zmax) : 0.0;
                                },
                                [&](uint32_t j) {
                                    return (zs_f2u(mom[j].pad) & 2u) && cs[j / ZS_SUBS_PER_CHUNK].z_max == zmax;
                                },
                                has_thr != 0);
        }
        if (obs_need & ZS_OBS_H) rounds |= 1u << ZS_SUM_OBS_H;
    }
    if (t == 0) {
        st.rounds = rounds;
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
        for (uint32_t j = 0; j < n_cand; j++) { st.cand_id[j] = cid_sh[j]; st.cand_x[j] = cx_sh[j]; }
        st.z_is_x = z_is_x;
        st.klist = 0;
        st.kpend = 0;
    }
    if (mode == ZS_MODE_BIG) {
        // bucket counts and masses of the top-p walk, accumulated by zs_k_pv
        zs_tp_bucket* bk = a.tp_bk + (size_t)r * ZS_TP_NB;
        for (uint32_t i = t; i < ZS_TP_NB; i += CB_NT) { bk[i].cnt = 0u; bk[i].mass = 0.0f; }
    }
}


// ===========================================================================
// Parallel exact-sum rounds. A round kernel gives every 1024-logit sub-chunk
// its total increment on the predicted grid (one wave per sub-chunk, all CUs);
// a stitch kernel walks a row's sub-chunks in order with the exact running sum,
// accepting a total when the prediction holds and recomputing the sub-chunk
// with the exact wave-level scan otherwise. Observer sums (tolerance outputs)
// take increments from the fast exp; the sampler sum uses certified ones.
// ===========================================================================
struct sub_row {
    const float* row;
    const uint32_t* allow;
    const uint32_t* pid;
    const uint32_t* pfl;
    const float* py;
    const uint32_t* psub;
    uint32_t V;
    float T;
    bool masked;
};

__device__ __forceinline__ sub_row make_sub_row(const zs_sargs& a, uint32_t r, const zs_row_params& P) {
    const zs_batch& b = a.b;
    sub_row R;
    R.row = b.d_logits + (size_t)r * b.ld;
    R.masked = (P.flags & ZS_ROW_MASKED) && b.d_allow_bits;
    R.allow = R.masked ? b.d_allow_bits + (size_t)r * b.allow_words : nullptr;
    R.pid = a.p_id + (size_t)r * ZS_MAX_PATCHES;
    R.pfl = a.p_flags + (size_t)r * ZS_MAX_PATCHES;
    R.py = a.p_y + (size_t)r * ZS_MAX_PATCHES;
    R.psub = a.p_sub + (size_t)r * (a.max_subs + 1);
    R.V = b.V;
    R.T = P.temperature;
    return R;
}

// thread t holds elements j*1024 + EPT*t .. +EPT-1 of sub-chunk j
// (EPT * threads = 1024)
template <int EPT>
__device__ __forceinline__ void sub_load_t(const sub_row& R, uint32_t j, uint32_t t, float (&x)[EPT], float (&z)[EPT]) {
    const uint32_t base = j * ZS_SUB + (uint32_t)EPT * t;
    uint32_t w = 0xffffffffu;
    if (R.masked && base < R.V) w = R.allow[base >> 5] >> (base & 31);
    if constexpr (EPT >= 4) {
#pragma unroll
        for (int k = 0; k < EPT / 4; k++) {
            float4 v = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
            if (base + 4 * k < R.V) v = *reinterpret_cast<const float4*>(R.row + base + 4 * k);
            x[4 * k] = v.x; x[4 * k + 1] = v.y; x[4 * k + 2] = v.z; x[4 * k + 3] = v.w;
        }
    } else if constexpr (EPT == 2) {
        float2 v = make_float2(-INFINITY, -INFINITY);
        if (base < R.V) v = *reinterpret_cast<const float2*>(R.row + base);  // V is a multiple of 4 or row padded
        x[0] = v.x; x[1] = v.y;
    } else {
        x[0] = base < R.V ? R.row[base] : -INFINITY;
    }
#pragma unroll
    for (int q = 0; q < EPT; q++) {
        if (base + q >= R.V || (R.masked && !((w >> q) & 1u))) x[q] = -INFINITY;
        z[q] = x[q];
    }
    const uint32_t p0 = R.psub[j], p1 = R.psub[j + 1];
    for (uint32_t p = p0; p < p1; p++) {
        uint32_t off = R.pid[p] - base;
        if (off < (uint32_t)EPT) {
            uint32_t fl = R.pfl[p];
            float py = R.py[p];
#pragma unroll
            for (int q = 0; q < EPT; q++) {
                if ((uint32_t)q != off) continue;
                if (fl & ZS_PF_BAN) { x[q] = -INFINITY; z[q] = -INFINITY; }
                if (fl & ZS_PF_Y) z[q] = py;
            }
        }
    }
#pragma unroll
    for (int q = 0; q < EPT; q++) z[q] = zs_temper(z[q], R.T);
}

// lane l of the wave holds elements j*1024 + 16l .. +15 of sub-chunk j
__device__ __forceinline__ void sub_load(const sub_row& R, uint32_t j, float (&x)[16], float (&z)[16]) {
    sub_load_t<16>(R, j, (uint32_t)zs_lane(), x, z);
}

__device__ __forceinline__ uint32_t wave_sum_sat(uint32_t v) {
    for (int d = 32; d > 0; d >>= 1) v = zs_sat_add(v, __shfl_xor(v, d, 64));
    return v;
}

// approximate exp for the observer sums
__device__ __forceinline__ float zs_exp_obs(float d) {
    if (d >= ZS_EXP_FAST_MIN) return zs_exp_fast(d);
    return d < ZS_EXP_ZERO ? 0.0f : zs_expf(d);
}

// observer terms with approximate values (tolerance outputs): the exact
// machinery is still applied to these values, so only terms whose fast-exp
// rounding differs move the sum, by a grid unit each
template <int EPT>
struct obs_exp_terms {
    float a[EPT];
    __device__ __forceinline__ void inc(int j, int eg, uint32_t* ie, uint32_t* io) const {
        seq_pair p = seq_pair_of(zs_pick(a, j), eg);
        *ie = p.e;
        *io = p.o;
    }
    __device__ __forceinline__ float val(int j) const { return zs_pick(a, j); }
};

__global__ __launch_bounds__(256) void zs_k_roundA(zs_sargs a) {
    const uint32_t r = blockIdx.y;
    const uint32_t j = blockIdx.x * 4 + zs_wid();
    const zs_row_state* st = a.rst + r;
    const uint32_t rounds = st->rounds;
    if (!(rounds & ((1u << ZS_SUM_OBS_S) | (1u << ZS_SUM_SAMP_S)))) return;
    const uint32_t V = a.b.V;
    const uint32_t nsub = (V + ZS_SUB - 1) / ZS_SUB;
    if (j >= nsub) return;
    const zs_row_params P = a.b.d_params[r];
    sub_row R = make_sub_row(a, r, P);
    zs_sub_sum* ss = a.sub_sum + (size_t)r * ZS_NSUM * a.max_subs;
    const bool do_obs = (rounds >> ZS_SUM_OBS_S) & 1u;
    const bool do_samp = (rounds >> ZS_SUM_SAMP_S) & 1u;
    zs_sub_sum eo = ss[ZS_SUM_OBS_S * a.max_subs + j];
    zs_sub_sum es = ss[ZS_SUM_SAMP_S * a.max_subs + j];
    const bool need_o = do_obs && !(eo.flags & ZS_SF_FRAGILE);
    const bool need_s = do_samp && !(es.flags & ZS_SF_FRAGILE);
    if (!need_o && !need_s) return;
    float x[16], z[16];
    sub_load(R, j, x, z);
    if (need_o) {
        const float M = st->obs_max;
        uint32_t tot = 0;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            uint32_t tie;
            tot = zs_sat_add(tot, zs_seq_inc(zs_exp_obs(x[q] - M), eo.eg, &tie));
        }
        tot = wave_sum_sat(tot);
        if (zs_lane() == 0) {
            zs_sub_sum& o = ss[ZS_SUM_OBS_S * a.max_subs + j];
            o.total = tot;
            o.flags = eo.flags | ZS_SF_DONE;
        }
    }
    if (need_s) {
        const float m = st->z_max;
        const bool use_thr = st->has_thr != 0;
        const float thr = zs_key_to_float(st->thr_key);
        exp_terms<16> f;
#pragma unroll
        for (int q = 0; q < 16; q++) f.set(q, (use_thr && z[q] < thr) ? -INFINITY : z[q] - m);
        uint32_t tot = 0, tie = 0;
#pragma unroll
        for (int q = 0; q < 16; q++) {
            uint32_t ie, io;
            f.inc(q, es.eg, &ie, &io);
            if (ie != io) tie = 1;
            tot = zs_sat_add(tot, ie);
        }
        tot = wave_sum_sat(tot);
        tie = wave_or_u(tie);
        if (zs_lane() == 0) {
            zs_sub_sum& o = ss[ZS_SUM_SAMP_S * a.max_subs + j];
            o.total = tot;
            o.flags = es.flags | ZS_SF_DONE | (tie ? ZS_SF_TIE : 0u);
        }
    }
}

// H = -sum p (d - ln S) terms with the fast exp (tolerance output)
__device__ __forceinline__ float zs_ent_obs(float d, float inv, float lns) {
    float p = zs_exp_obs(d) * inv;
    if (!(p > 0.0f)) return 0.0f;
    return -(p * (d - lns));
}

template <int EPT>
struct obs_ent_terms {
    float a[EPT];
    __device__ __forceinline__ void inc(int j, int eg, uint32_t* ie, uint32_t* io) const {
        seq_pair p = seq_pair_of(zs_pick(a, j), eg);
        *ie = p.e;
        *io = p.o;
    }
    __device__ __forceinline__ float val(int j) const { return zs_pick(a, j); }
};

__global__ __launch_bounds__(256) void zs_k_roundB(zs_sargs a) {
    const uint32_t r = blockIdx.y;
    const uint32_t j = blockIdx.x * 4 + zs_wid();
    const zs_row_state* st = a.rst + r;
    if (!((st->rounds >> ZS_SUM_OBS_H) & 1u)) return;
    const uint32_t V = a.b.V;
    const uint32_t nsub = (V + ZS_SUB - 1) / ZS_SUB;
    if (j >= nsub) return;
    zs_sub_sum* ss = a.sub_sum + ((size_t)r * ZS_NSUM + ZS_SUM_OBS_H) * a.max_subs;
    zs_sub_sum e = ss[j];
    if (e.flags & ZS_SF_FRAGILE) return;
    const zs_row_params P = a.b.d_params[r];
    sub_row R = make_sub_row(a, r, P);
    float x[16], z[16];
    sub_load(R, j, x, z);
    const float M = st->obs_max, S = st->obs_S;
    const float inv = 1.0f / S, lns = (float)log((double)S);
    uint32_t tot = 0;
#pragma unroll
    for (int q = 0; q < 16; q++) {
        uint32_t tie;
        tot = zs_sat_add(tot, zs_seq_inc(zs_ent_obs(x[q] - M, inv, lns), e.eg, &tie));
    }
    tot = wave_sum_sat(tot);
    if (zs_lane() == 0) {
        ss[j].total = tot;
        ss[j].flags = e.flags | ZS_SF_DONE;
    }
}

#define ST_NT 512
#define ST_EPT (ZS_SUB / ST_NT)

struct st_sh {
    seq_sh<ST_NT> seq;
    float head[64];
    zs_sub_sum rec[ZS_MAX_SUBS];
};

// Exact processing of one sub-chunk by the workgroup: the first 64 terms of a
// sum that starts at zero are added serially by thread 0 (the running sum
// crosses many binades there), the rest with the increment scan.
template <class F>
__device__ __forceinline__ void stitch_sub(const F& f, float& s, bool first, st_sh& sh) {
    int start = 0;
    if (first) {
        const int t = threadIdx.x;
        if (t < 64 / ST_EPT) {
#pragma unroll
            for (int q = 0; q < ST_EPT; q++) sh.head[ST_EPT * t + q] = f.val(q);
        }
        __syncthreads();
        if (t == 0) {
            float acc = s;
            for (int i = 0; i < 64; i++) acc = acc + sh.head[i];
            sh.seq.s = acc;
        }
        __syncthreads();
        s = sh.seq.s;
        __syncthreads();
        start = 64;
    }
    seq_group_f<ST_NT, ST_EPT>(f, start, s, NAN, sh.seq);
}

// One workgroup per (row, sum): the exact running sum over the row's
// sub-chunks, taking the rounds' totals where the predicted grid holds.
template <int KIND>
__device__ __forceinline__ void stitch_body(const zs_sargs& a) {
    const uint32_t r = blockIdx.x;
    zs_row_state* st = a.rst + r;
    const uint32_t rounds = st->rounds;
    if (!((rounds >> KIND) & 1u)) return;
    __shared__ st_sh sh;
    const uint32_t t = threadIdx.x;
    const uint32_t V = a.b.V;
    const uint32_t nsub = (V + ZS_SUB - 1) / ZS_SUB;
    const zs_row_params P = a.b.d_params[r];
    sub_row R = make_sub_row(a, r, P);
    const zs_sub_sum* ss = a.sub_sum + ((size_t)r * ZS_NSUM + KIND) * a.max_subs;
    for (uint32_t j = t; j < nsub; j += ST_NT) sh.rec[j] = ss[j];
    __syncthreads();
    const float M = st->obs_max, m = st->z_max;
    const bool use_thr = st->has_thr != 0;
    const float thr = zs_key_to_float(st->thr_key);
    float inv = 0.0f, lns = 0.0f;
    if (KIND == ZS_SUM_OBS_H) {
        inv = 1.0f / st->obs_S;
        lns = (float)log((double)st->obs_S);
    }
    float s = KIND == ZS_SUM_OBS_H ? 0.0f : -0.0f;
    for (uint32_t j = 0; j < nsub; j++) {
        const zs_sub_sum e = sh.rec[j];
        const int eg = zs_grid_exp(s);
        const uint32_t k0 = zs_grid_k(s);
        if ((e.flags & ZS_SF_DONE) && !(e.flags & (ZS_SF_FRAGILE | ZS_SF_TIE)) && e.eg == eg &&
            k0 + e.total < ZS_BINADE) {
            s = zs_grid_value(k0 + e.total, eg);
            continue;
        }
        const bool first = (j == 0);
        float x[ST_EPT], z[ST_EPT];
        sub_load_t<ST_EPT>(R, j, t, x, z);
        if (KIND == ZS_SUM_OBS_S) {
            obs_exp_terms<ST_EPT> f;
#pragma unroll
            for (int q = 0; q < ST_EPT; q++) f.a[q] = zs_exp_obs(x[q] - M);
            stitch_sub(f, s, first, sh);
        } else if (KIND == ZS_SUM_SAMP_S) {
            exp_terms<ST_EPT> f;
#pragma unroll
            for (int q = 0; q < ST_EPT; q++) f.set(q, (use_thr && z[q] < thr) ? -INFINITY : z[q] - m);
            stitch_sub(f, s, first, sh);
        } else {
            obs_ent_terms<ST_EPT> f;
#pragma unroll
            for (int q = 0; q < ST_EPT; q++) f.a[q] = zs_ent_obs(x[q] - M, inv, lns);
            stitch_sub(f, s, first, sh);
        }
    }
    if (KIND == ZS_SUM_OBS_S) {
        if (t == 0) st->obs_S = s;
        if (((rounds >> ZS_SUM_OBS_H) & 1u) && t < 64) {
            // predictions for the entropy sum: p = e * inv, term = p (ln S - d)
            const float iv = 1.0f / s;
            const double ls = log((double)s);
            const zs_sub_mom* mom = a.sub_mom + (size_t)r * a.max_subs;
            const zs_chunk_stat* cs = a.cst + (size_t)r * a.nch;
            zs_predict_subs(a.sub_sum + ((size_t)r * ZS_NSUM + ZS_SUM_OBS_H) * a.max_subs, nsub,
                            [&](uint32_t jj) {
                                double mc = (double)cs[jj / ZS_SUBS_PER_CHUNK].obs_max;
                                double sc = exp(mc - (double)M);
                                double e1 = (double)mom[jj].e1 * sc;
                                double ed = ((double)mom[jj].ed + (mc - (double)M) * (double)mom[jj].e1) * sc;
                                double v = (double)iv * (ls * e1 - ed);
                                return v > 0.0 ? v : 0.0;
                            },
                            [](uint32_t) { return false; },
                            false);
        }
    } else if (KIND == ZS_SUM_SAMP_S) {
        if (t == 0) st->samp_S = s;
    } else {
        if (t == 0) st->obs_H = s;
    }
}

// the observers' S (blockIdx.y 0) and the sampler's S (1) side by side
__global__ __launch_bounds__(ST_NT) void zs_k_stitchA(zs_sargs a) {
    if (blockIdx.y == 0) stitch_body<ZS_SUM_OBS_S>(a);
    else stitch_body<ZS_SUM_SAMP_S>(a);
}
__global__ __launch_bounds__(ST_NT) void zs_k_stitchB(zs_sargs a) { stitch_body<ZS_SUM_OBS_H>(a); }

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
    uint32_t sortbuf[ZS_SORT_CAP];
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
__device__ __forceinline__ big_raw big_fetch(const big_row& R, uint32_t g) {
    const uint32_t idx0 = g * ZS_BIG_G + 4 * threadIdx.x;
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
// ZS_BIG_G / ZS_SUB sub-chunks (per-sub-chunk patch offsets from zs_k_prep).
__device__ __forceinline__ void big_finish(const big_row& R, uint32_t g, const big_raw& raw, float (&x)[4],
                                           float (&z)[4]) {
    const uint32_t idx0 = g * ZS_BIG_G + 4 * threadIdx.x;
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
#pragma unroll
    for (int q = 0; q < 4; q++) z[q] = zs_temper(z[q], R.T);
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
// the rounds summed it (or the observers' S is the same sum: z == x~, no cut).
__device__ __forceinline__ bool big_s_from_rounds(const zs_row_state& st) {
    const bool reuse = st.z_is_x && !st.has_thr && (st.obs_need & ZS_OBS_S);
    return reuse || ((st.rounds >> ZS_SUM_SAMP_S) & 1u);
}
__device__ __forceinline__ float big_s_value(const zs_row_state& st) {
    const bool reuse = st.z_is_x && !st.has_thr && (st.obs_need & ZS_OBS_S);
    return reuse ? st.obs_S : st.samp_S;
}

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
__global__ __launch_bounds__(ZS_BIG_NT) void zs_k_pv(zs_sargs a) {
    const uint32_t g = blockIdx.x, r = blockIdx.y;
    const zs_row_state& st = a.rst[r];
    if (st.mode != ZS_MODE_BIG || !big_s_from_rounds(st)) return;
    const zs_batch& b = a.b;
    const uint32_t V = b.V;
    const uint32_t idx0 = g * ZS_BIG_G + 4 * threadIdx.x;
    const zs_row_params P = b.d_params[r];
    const bool hist = tp_fast_row(st, P);
    __shared__ uint32_t hc[ZS_TP_NB];
    __shared__ float hm[ZS_TP_NB];
    if (hist) {
        for (uint32_t i = threadIdx.x; i < ZS_TP_NB; i += ZS_BIG_NT) { hc[i] = 0u; hm[i] = 0.0f; }
        __syncthreads();
    }
    if (idx0 < V) {
        big_row R;
        R.row = b.d_logits + (size_t)r * b.ld;
        R.masked = (P.flags & ZS_ROW_MASKED) && b.d_allow_bits;
        R.allow = R.masked ? b.d_allow_bits + (size_t)r * b.allow_words : nullptr;
        R.pid = a.p_id + (size_t)r * ZS_MAX_PATCHES;
        R.pfl = a.p_flags + (size_t)r * ZS_MAX_PATCHES;
        R.py = a.p_y + (size_t)r * ZS_MAX_PATCHES;
        R.psub = a.p_sub + (size_t)r * (a.max_subs + 1);
        R.nsub = (V + ZS_SUB - 1) / ZS_SUB;
        R.V = V;
        R.T = P.temperature;
        const bool use_thr = st.has_thr != 0;
        const float thr = zs_key_to_float(st.thr_key), m = st.z_max, S = big_s_value(st);
        float x[4], z[4];
        big_finish(R, g, big_fetch(R, g), x, z);
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
        for (uint32_t i = threadIdx.x; i < ZS_TP_NB; i += ZS_BIG_NT) {
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
                if (j < ZS_TP_CAND) cl[2 + j] = i;
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

__global__ __launch_bounds__(TP_SORT_NT) void zs_k_tp_sort(zs_sargs a) {
    const uint32_t c = blockIdx.x, r = blockIdx.y;
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
__device__ __forceinline__ int tp_walk(const zs_sargs& a, uint32_t r, float top_p, walk_out* wo) {
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
    uint32_t b0 = 0;
    while (b0 < ZS_TP_NB) {
        const uint32_t bb = b0 + lane;
        uint32_t cnt = 0u, meta = 0u;
        unsigned long long tot = 0ull;
        if (bb < ZS_TP_NB) { cnt = bk[bb].cnt; meta = bk[bb].meta; tot = bk[bb].tot; }
        const bool special = cnt && ((int)(meta & TP_M_EG) != eg || (meta & TP_M_TIE0));
        const unsigned long long inc = (cnt && !special) ? tot : 0ull;
        unsigned long long incl = inc;
        for (int d = 1; d < 64; d <<= 1) {
            const unsigned long long y = __shfl_up(incl, d, 64);
            if (lane >= (uint32_t)d) incl += y;
        }
        const unsigned long long lim = min((unsigned long long)ZS_BINADE, (unsigned long long)kthr);
        const unsigned long long hm = __ballot(cnt && (special || k + incl >= lim));
        if (!hm) {
            k += __shfl(incl, 63, 64);
            b0 += 64;
            continue;
        }
        const uint32_t f = (uint32_t)__ffsll((long long)hm) - 1u;
        k += __shfl(incl - inc, (int)f, 64);
        const uint32_t b = b0 + f;
        b0 = b + 1;
        const uint32_t n = __shfl(cnt, (int)f, 64), bm = __shfl(meta, (int)f, 64);
        if (!(bm & TP_M_SORTED)) {
            return 0;
        }
        const uint32_t st0 = bk[b].start;
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
            // one addition at a time (sampler.rs:103)
            float ss = zs_grid_value((uint32_t)k, eg);
            for (uint32_t i = pos; i < n && !stop; i += 64) {
                const float v = i + lane < n ? zs_u2f(gv[st0 + i + lane]) : 0.0f;
                const uint32_t m = min(64u, n - i);
                for (uint32_t j = 0; j < m; j++) {
                    ss = ss + zs_readlane_f(v, j);
                    if (ss >= top_p) { stop = true; at = i + j; break; }
                }
            }
            if (!stop) set_sum(ss);
        }
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
    __shared__ big_shared sh;
    const int t = threadIdx.x;
    const zs_batch& b = a.b;
    const zs_row_params P = b.d_params[r];
    big_row R;
    R.row = b.d_logits + (size_t)r * b.ld;
    R.masked = (P.flags & ZS_ROW_MASKED) && b.d_allow_bits;
    R.allow = R.masked ? b.d_allow_bits + (size_t)r * b.allow_words : nullptr;
    R.pid = a.p_id + (size_t)r * ZS_MAX_PATCHES;
    R.pfl = a.p_flags + (size_t)r * ZS_MAX_PATCHES;
    R.py = a.p_y + (size_t)r * ZS_MAX_PATCHES;
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
    const bool use_thr = has_thr != 0;
    const float thr = zs_key_to_float(thr_key);

    // ---- softmax denominator: from the parallel rounds (sampler S, or the
    // observers' S when z == x~ and no top-k cut applies), else summed here
    const bool reuse = stt.z_is_x && !use_thr && (stt.obs_need & ZS_OBS_S);
    float S = reuse ? stt.obs_S : stt.samp_S;
    if (!reuse && !((stt.rounds >> ZS_SUM_SAMP_S) & 1u)) {
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

    // ---- top-p (sampler.rs:91-115)
    const bool topp = P.top_p < 1.0f && P.top_p > 0.0f;
    uint32_t vstar = 0, istar = 0xffffffffu;  // kept: p1 > v* or (p1 == v* and idx <= i*)
    float sum2 = 0.0f;
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
                const int res = tp_walk(a, r, P.top_p, &w);
                if (t == 0) { sh.u[0] = (uint32_t)res; sh.u[1] = w.v; sh.u[2] = w.rank; }
            }
            __syncthreads();
            fw = (int)sh.u[0];
            wo = {fw == 1, sh.u[1], sh.u[2]};
            __syncthreads();
        }
        if (fw == 0) {
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
            }
            return;
        } else {
            // every positive p kept: sum over the whole row
            vstar = 0;
            istar = 0xffffffffu;
            sum2 = -0.0f;
            stream_p1([&](uint32_t, const float (&p)[4]) {
                seq_group<ZS_BIG_NT, 4>(p, 0, sum2, NAN, sh.q);
                return false;
            });
        }
    }
    // ---- draw (sampler.rs:118-127)
    const float rr = zs_philox_uniform(b.d_seed[r], b.d_counter[r], 0u);
    uint32_t token = V - 1;
    if (rr <= 0.0f) {
        token = 0;
    } else {
        float cum = 0.0f;
        const bool renorm = topp && sum2 > 0.0f;
        stream_p1([&](uint32_t g, const float (&p)[4]) {
            float tv[4];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                float pp = p[q];
                if (renorm) {
                    const uint32_t pb = zs_f2u(pp), idx = g * ZS_BIG_G + 4 * t + q;
                    const bool keep = pb > vstar || (pb == vstar && idx <= istar);
                    pp = keep ? pp / sum2 : 0.0f;
                }
                tv[q] = pp;
            }
            int stp = seq_group<ZS_BIG_NT, 4>(tv, 0, cum, rr, sh.q);
            if (stp >= 0) { token = g * ZS_BIG_G + stp; return true; }
            return false;
        });
    }
    if (t == 0) {
        a.rst[r].token = token;
        a.rst[r].mode = ZS_MODE_DONE;
    }
}

// ===========================================================================
// Compaction of the kept set {p1 >= v*} in index order (rows with a top-p
// stop), over all CUs: zs_k_kcount counts per 4096-id group the values above
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

__global__ __launch_bounds__(ZS_BIG_NT) void zs_k_kcount(zs_sargs a) {
    const uint32_t g = blockIdx.x, r = blockIdx.y;
    const zs_row_state& st = a.rst[r];
    if (!st.kpend) return;
    const uint32_t t = threadIdx.x, V = a.b.V;
    const uint32_t idx0 = g * ZS_BIG_G + 4 * t;
    const uint4 v = idx0 < V ? *reinterpret_cast<const uint4*>(a.pv + (size_t)r * a.max_vocab + idx0) : make_uint4(0u, 0u, 0u, 0u);
    const uint32_t pb[4] = {v.x, v.y, v.z, v.w};
    const uint32_t vs = st.vstar;
    uint32_t c = 0;  // (above << 16) | equal
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float p = kc_p1(st, pb[q]);
        const uint32_t b = zs_f2u(p);
        if (p > 0.0f && b >= vs) c += b > vs ? 0x10000u : 1u;
    }
    __shared__ uint32_t sh[ZS_BIG_NT / 64];
    c = wave_sum_u(c);
    if (zs_lane() == 0) sh[zs_wid()] = c;
    __syncthreads();
    if (t == 0) {
        uint32_t tot = 0;
        for (int i = 0; i < ZS_BIG_NT / 64; i++) tot += sh[i];
        a.kcnt[(size_t)r * a.nch * 2 + g] = tot;
    }
    // the kept-list sub-chunk sums are added by zs_k_kwrite
    if (t < ZS_BIG_G / ZS_SUB) a.k_ap[(size_t)r * a.max_subs + g * (ZS_BIG_G / ZS_SUB) + t] = 0.0;
}

__global__ __launch_bounds__(ZS_BIG_NT) void zs_k_kwrite(zs_sargs a) {
    const uint32_t g = blockIdx.x, r = blockIdx.y;
    zs_row_state& st = a.rst[r];
    if (!st.kpend) return;
    const uint32_t t = threadIdx.x, V = a.b.V;
    const uint32_t ng = (V + ZS_BIG_G - 1) / ZS_BIG_G;
    __shared__ uint32_t sh[ZS_BIG_NT / 64];
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
    __syncthreads();
    const uint32_t base = base_sh[0], eq0 = base_sh[1];
    const uint32_t idx0 = g * ZS_BIG_G + 4 * t;
    const uint4 v = idx0 < V ? *reinterpret_cast<const uint4*>(a.pv + (size_t)r * a.max_vocab + idx0) : make_uint4(0u, 0u, 0u, 0u);
    const uint32_t pb[4] = {v.x, v.y, v.z, v.w};
    const uint32_t vs = st.vstar, rank = st.krank;
    uint32_t kb[4];
    uint32_t c = 0;  // (kept << 16) | equal
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float p = kc_p1(st, pb[q]);
        kb[q] = zs_f2u(p);
        if (p > 0.0f && kb[q] >= vs) c += 0x10000u + (kb[q] == vs ? 1u : 0u);
    }
    uint32_t tot;
    uint32_t ex = block_excl_scan_u<ZS_BIG_NT>(c, sh, &tot);
    uint32_t pos = base + (ex >> 16), eq = eq0 + (ex & 0xffffu);
    uint32_t* kp = a.pairs + (size_t)r * a.max_vocab * 2;
    uint32_t* ki = kp + a.max_vocab;
    const uint32_t sub0 = base / ZS_SUB;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        if (!(zs_u2f(kb[q]) > 0.0f && kb[q] >= vs)) continue;
        const uint32_t idx = idx0 + q;
        kp[pos] = kb[q];
        ki[pos] = idx;
        bool in = true;
        if (kb[q] == vs) {
            if (eq == rank) st.istar = idx;
            in = eq <= rank;
            eq++;
        }
        if (in) atomicAdd(&lap[pos / ZS_SUB - sub0], (double)zs_u2f(kb[q]));
        pos++;
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
    const uint32_t* ki;
    uint32_t nk, vstar, istar;
    float inv;  // 0: the kept p themselves (sum2), else p / sum2 (draw)
    float sum2;
};
__device__ __forceinline__ klist_row make_klist(const zs_sargs& a, uint32_t r, const zs_row_state& st, int kind) {
    klist_row L;
    L.kp = a.pairs + (size_t)r * a.max_vocab * 2;
    L.ki = L.kp + a.max_vocab;
    L.nk = st.nk;
    L.vstar = st.vstar;
    L.istar = st.istar;
    L.sum2 = kind ? st.sum2 : 1.0f;
    L.inv = kind ? 1.0f : 0.0f;
    return L;
}
// term i of the list: the kept p (0 for the equal values after i*), divided by
// sum2 for the draw
__device__ __forceinline__ float klist_term(const klist_row& L, uint32_t i) {
    if (i >= L.nk) return 0.0f;
    const uint32_t pb = L.kp[i];
    if (!(pb > L.vstar || L.ki[i] <= L.istar)) return 0.0f;
    const float p = zs_u2f(pb);
    return L.inv != 0.0f ? p / L.sum2 : p;
}

// one wave per (sub-chunk, row)
template <int KIND>
__global__ __launch_bounds__(256) void zs_k_roundK(zs_sargs a) {
    const uint32_t r = blockIdx.y;
    const uint32_t j = blockIdx.x * 4 + zs_wid();
    const zs_row_state& st = a.rst[r];
    if (!st.klist) return;
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
    const int blo = lm < 0x1p-125 ? -125 : ilogb(lm);
    const int bhi = hm < 0x1p-125 ? -125 : ilogb(hm);
    zs_sub_sum e;
    e.pad = 0;
    if (j == 0 || blo != bhi || !(hm < 3.0e38)) {
        e.eg = 0;
        e.flags = ZS_SF_FRAGILE;
        e.total = 0;
    } else {
        e.eg = zs_grid_exp((float)lo);
        uint32_t tot = 0, tie = 0;
#pragma unroll
        for (int q = 0; q < ZS_SUB / 64; q++) {
            uint32_t tq;
            tot = zs_sat_add(tot, zs_seq_inc(klist_term(L, j * ZS_SUB + q * 64 + zs_lane()), e.eg, &tq));
            tie |= tq;
        }
        tot = wave_sum_sat(tot);
        tie = wave_or_u(tie);
        e.total = tot;
        e.flags = ZS_SF_DONE | (tie ? ZS_SF_TIE : 0u);
    }
    if (zs_lane() == 0) a.k_sum[((size_t)r * 2 + KIND) * a.max_subs + j] = e;
}

// one workgroup per row: sum2 (KIND 0), or the draw (KIND 1) -- the first
// entry after which the running sum reaches the uniform
#define SK_NT 512
#define SK_EPT (ZS_SUB / SK_NT)
template <int KIND>
__global__ __launch_bounds__(SK_NT) void zs_k_stitchK(zs_sargs a) {
    const uint32_t r = blockIdx.x;
    zs_row_state* stp = a.rst + r;
    if (!stp->klist) return;
    const zs_row_state st = *stp;
    __shared__ seq_sh<SK_NT> sh;
    __shared__ zs_sub_sum rec[ZS_MAX_SUBS];
    const int t = threadIdx.x;
    const klist_row L = make_klist(a, r, st, KIND);
    const uint32_t nks = (L.nk + ZS_SUB - 1) / ZS_SUB;
    const zs_sub_sum* ks = a.k_sum + ((size_t)r * 2 + KIND) * a.max_subs;
    for (uint32_t j = t; j < nks; j += SK_NT) rec[j] = ks[j];
    __syncthreads();
    float thresh = NAN;
    uint32_t token = a.b.V - 1;
    bool done = false;
    if (KIND == 1) {
        const float rr = zs_philox_uniform(a.b.d_seed[r], a.b.d_counter[r], 0u);
        if (rr <= 0.0f) { token = 0; done = true; }  // cumsum >= r at the first id
        thresh = rr;
    }
    float s = KIND ? 0.0f : -0.0f;
    for (uint32_t j = 0; j < nks && !done; j++) {
        const zs_sub_sum e = rec[j];
        const int eg = zs_grid_exp(s);
        const uint32_t k0 = zs_grid_k(s);
        if ((e.flags & ZS_SF_DONE) && !(e.flags & (ZS_SF_FRAGILE | ZS_SF_TIE)) && e.eg == eg &&
            k0 + e.total < ZS_BINADE) {
            const uint32_t kthr = KIND ? zs_grid_thresh(thresh, eg) : 0xffffffffu;
            if (kthr == 0xffffffffu || k0 + e.total < kthr) {
                s = zs_grid_value(k0 + e.total, eg);
                continue;
            }
        }
        float tv[SK_EPT];
#pragma unroll
        for (int q = 0; q < SK_EPT; q++) tv[q] = klist_term(L, j * ZS_SUB + SK_EPT * t + q);
        const int stop = seq_group<SK_NT, SK_EPT>(tv, 0, s, thresh, sh);
        if (KIND == 1 && stop >= 0) {
            token = L.ki[j * ZS_SUB + (uint32_t)stop];
            done = true;
        }
    }
    if (t == 0) {
        if (KIND == 0) {
            stp->sum2 = s;
        } else {
            stp->token = token;
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
        const uint32_t* pid = a.p_id + (size_t)r * ZS_MAX_PATCHES;
        const uint32_t* psub = a.p_sub + (size_t)r * (a.max_subs + 1);
        const uint32_t nsub = (b.V + ZS_SUB - 1) / ZS_SUB;
        const uint32_t p0 = psub[tok / ZS_SUB], p1 = psub[min(tok / ZS_SUB + 1, nsub)];
        bool ban = false;
        for (uint32_t p = p0 + lane; p < p1; p += 64)
            if (pid[p] == tok && (a.p_flags[(size_t)r * ZS_MAX_PATCHES + p] & ZS_PF_BAN)) ban = true;
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
            if (mine && rank < n) { tid[rank] = id; tlp[rank] = lp; }
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
    a.cst = ctx->cst;
    a.cs_key = ctx->cs_key;
    a.cs_idx = ctx->cs_idx;
    a.co_key = ctx->co_key;
    a.co_idx = ctx->co_idx;
    a.rst = ctx->rst;
    a.pairs = ctx->pairs;
    a.nch = ctx->max_chunks;
    a.max_vocab = ctx->max_vocab;
    a.pv = ctx->pv;
    a.sub_mom = ctx->sub_mom;
    a.sub_sum = ctx->sub_sum;
    a.p_sub = ctx->p_sub;
    a.max_subs = ctx->max_subs;
    a.k_ap = ctx->k_ap;
    a.k_sum = ctx->k_sum;
    a.tp_bk = ctx->tp_bk;
    a.tp_cl = ctx->tp_cl;
    a.tp_pre = ctx->tp_pre;
    a.kcnt = ctx->kcnt;
    const uint32_t B = bt->B;
    const uint32_t nch = (bt->V + ZS_P1_CH - 1) / ZS_P1_CH;
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
    hipLaunchKernelGGL(zs_k_pv, dim3((bt->V + ZS_BIG_G - 1) / ZS_BIG_G, B), dim3(ZS_BIG_NT), 0, stream, a);
    mark("zs_k_pv");
    hipLaunchKernelGGL(zs_k_tp_plan, dim3(B), dim3(ZS_BIG_NT), 0, stream, a);
    mark("zs_k_tp_plan");
    hipLaunchKernelGGL(zs_k_tp_inc, dim3((bt->V + ZS_BIG_G - 1) / ZS_BIG_G, B), dim3(ZS_BIG_NT), 0, stream, a);
    mark("zs_k_tp_inc");
    hipLaunchKernelGGL(zs_k_tp_sort, dim3(ZS_TP_CAND, B), dim3(TP_SORT_NT), 0, stream, a);
    mark("zs_k_tp_sort");
    hipLaunchKernelGGL(zs_k_big, dim3(B), dim3(ZS_BIG_NT), 0, stream, a);
    mark("zs_k_big");
    hipLaunchKernelGGL(zs_k_kcount, dim3((bt->V + ZS_BIG_G - 1) / ZS_BIG_G, B), dim3(ZS_BIG_NT), 0, stream, a);
    hipLaunchKernelGGL(zs_k_kwrite, dim3((bt->V + ZS_BIG_G - 1) / ZS_BIG_G, B), dim3(ZS_BIG_NT), 0, stream, a);
    mark("zs_k_kcompact");
    const uint32_t nsubk = (bt->V + ZS_SUB - 1) / ZS_SUB;
    hipLaunchKernelGGL(zs_k_roundK<0>, dim3((nsubk + 3) / 4, B), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(zs_k_stitchK<0>, dim3(B), dim3(SK_NT), 0, stream, a);
    hipLaunchKernelGGL(zs_k_roundK<1>, dim3((nsubk + 3) / 4, B), dim3(256), 0, stream, a);
    hipLaunchKernelGGL(zs_k_stitchK<1>, dim3(B), dim3(SK_NT), 0, stream, a);
    mark("zs_k_kept");
    hipLaunchKernelGGL(zs_k_final, dim3(B), dim3(64), 0, stream, a);
    mark("zs_k_final");
    if (prof) ctx->n_timed = ev - 1;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return zs_set_error(ctx, ZS_EHIP, "zs_sample launch: %s", hipGetErrorString(e));
    return ZS_OK;
}
