#include <atomic>
#include <stddef.h>
// zs_api.cpp -- host side of libzs: contexts, token tables, DFAs (liveness on
// the host), argument validation, and the C entry points of include/zs.h.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <algorithm>
#include <map>
#include <vector>
#include "zs_internal.h"

// launchers (zs_sample.hip, zs_dfa.hip)
extern "C" int zs_sample_launch(zs_ctx* ctx, const zs_batch* bt, hipStream_t stream);
extern "C" int zs_spec_launch(const zs_spec_args& a, const zs_prof& prof, hipStream_t stream);
extern "C" int zs_lane_argmax_launch(const float* logits, uint32_t B, uint32_t V, uint64_t ld, const float* temp,
                                     const uint32_t* seed, const uint32_t* ih, unsigned long long* keys,
                                     uint32_t* out, hipStream_t stream);
extern "C" int zs_lane_hash_fill(uint32_t* ih, uint32_t n, hipStream_t stream);
extern "C" int zs_lane_topk_launch(const float* logits, uint32_t B, uint32_t V, uint64_t ld, uint32_t K,
                                   float* vals, uint32_t* idxs, unsigned long long* ck, uint32_t* cn,
                                   hipStream_t stream);
extern "C" int zs_lane_sample_topk_launch(const float* vals, const uint32_t* idxs, uint32_t B, uint32_t K,
                                          const float* temp, const uint32_t* top_k, const float* top_p,
                                          const uint32_t* seed, uint32_t* out, hipStream_t stream);
extern "C" int zs_lane_topk_draw_launch(const float* logits, uint32_t B, uint32_t V, uint64_t ld, uint32_t K,
                                        float* vals, uint32_t* idxs, unsigned long long* ck, uint32_t* cn,
                                        const float* temp, const uint32_t* top_k, const float* top_p,
                                        const uint32_t* seed, uint32_t* out, hipStream_t stream);
extern "C" int zs_dfa_mask_launch(const dm_args& a, bool lds, uint32_t ncu, uint32_t* any_scratch, hipStream_t stream);

int zs_set_error(zs_ctx* ctx, int code, const char* fmt, ...) {
    if (ctx) {
        va_list ap;
        va_start(ap, fmt);
        vsnprintf(ctx->err, sizeof(ctx->err), fmt, ap);
        va_end(ap);
    }
    return code;
}

#define ZS_HIP(ctx, call)                                                                   \
    do {                                                                                    \
        hipError_t e_ = (call);                                                             \
        if (e_ != hipSuccess)                                                               \
            return zs_set_error((ctx), ZS_EHIP, "%s: %s", #call, hipGetErrorString(e_));   \
    } while (0)

template <typename T>
static int zs_alloc(zs_ctx* ctx, T** p, size_t n) {
    *p = nullptr;
    if (n == 0) n = 1;
    hipError_t e = hipMalloc((void**)p, n * sizeof(T));
    if (e != hipSuccess) {
        *p = nullptr;
        return zs_set_error(ctx, ZS_ENOMEM, "hipMalloc(%zu bytes): %s", n * sizeof(T), hipGetErrorString(e));
    }
    return ZS_OK;
}

extern "C" int zs_abi_version(void) { return ZS_ABI_VERSION; }

// Field offsets of the ABI structs, in declaration order.
#define ZS_OFF(T, f) offsetof(T, f)
extern "C" int zs_struct_layout(int which, size_t* size, size_t* offsets, size_t cap) {
    static const size_t batch[] = {
        ZS_OFF(zs_batch, B), ZS_OFF(zs_batch, V), ZS_OFF(zs_batch, ld), ZS_OFF(zs_batch, d_logits),
        ZS_OFF(zs_batch, d_params), ZS_OFF(zs_batch, d_cnt_off), ZS_OFF(zs_batch, d_cnt_ids),
        ZS_OFF(zs_batch, d_cnt_vals), ZS_OFF(zs_batch, d_bias_off), ZS_OFF(zs_batch, d_bias_ids),
        ZS_OFF(zs_batch, d_bias_vals), ZS_OFF(zs_batch, d_ban_off), ZS_OFF(zs_batch, d_ban_ids),
        ZS_OFF(zs_batch, d_allow_bits), ZS_OFF(zs_batch, allow_words), ZS_OFF(zs_batch, top_stride),
        ZS_OFF(zs_batch, d_seed), ZS_OFF(zs_batch, d_counter), ZS_OFF(zs_batch, d_token),
        ZS_OFF(zs_batch, d_logprob), ZS_OFF(zs_batch, d_top_ids), ZS_OFF(zs_batch, d_top_lps),
        ZS_OFF(zs_batch, d_top_n), ZS_OFF(zs_batch, d_entropy), ZS_OFF(zs_batch, d_max_prob),
        ZS_OFF(zs_batch, d_margin), ZS_OFF(zs_batch, d_chosen_lp), ZS_OFF(zs_batch, d_status),
        ZS_OFF(zs_batch, pass_event)};
    static const size_t params[] = {
        ZS_OFF(zs_row_params, temperature), ZS_OFF(zs_row_params, top_k), ZS_OFF(zs_row_params, top_p),
        ZS_OFF(zs_row_params, min_p), ZS_OFF(zs_row_params, repeat), ZS_OFF(zs_row_params, presence),
        ZS_OFF(zs_row_params, frequency), ZS_OFF(zs_row_params, top_logprobs), ZS_OFF(zs_row_params, flags),
        ZS_OFF(zs_row_params, pad)};
    static const size_t spec[] = {
        ZS_OFF(zs_spec_batch, B), ZS_OFF(zs_spec_batch, V), ZS_OFF(zs_spec_batch, k), ZS_OFF(zs_spec_batch, ld),
        ZS_OFF(zs_spec_batch, d_target), ZS_OFF(zs_spec_batch, d_draft), ZS_OFF(zs_spec_batch, d_draft_ids),
        ZS_OFF(zs_spec_batch, d_temperature), ZS_OFF(zs_spec_batch, d_seed), ZS_OFF(zs_spec_batch, d_counter),
        ZS_OFF(zs_spec_batch, d_accepted), ZS_OFF(zs_spec_batch, d_next), ZS_OFF(zs_spec_batch, flags)};
    static const size_t lane[] = {
        ZS_OFF(zs_lane_stream, temp), ZS_OFF(zs_lane_stream, top_k), ZS_OFF(zs_lane_stream, top_p),
        ZS_OFF(zs_lane_stream, base_seed), ZS_OFF(zs_lane_stream, gen_index)};
    static const size_t rep[] = {
        ZS_OFF(zs_halluc_report, risk_score), ZS_OFF(zs_halluc_report, mean_entropy),
        ZS_OFF(zs_halluc_report, normalized_entropy), ZS_OFF(zs_halluc_report, risky_fraction),
        ZS_OFF(zs_halluc_report, peak_token), ZS_OFF(zs_halluc_report, n_tokens)};
    const size_t* f;
    size_t n, sz;
    switch (which) {
        case ZS_LAYOUT_BATCH: f = batch; n = sizeof(batch) / sizeof(size_t); sz = sizeof(zs_batch); break;
        case ZS_LAYOUT_ROW_PARAMS: f = params; n = sizeof(params) / sizeof(size_t); sz = sizeof(zs_row_params); break;
        case ZS_LAYOUT_SPEC_BATCH: f = spec; n = sizeof(spec) / sizeof(size_t); sz = sizeof(zs_spec_batch); break;
        case ZS_LAYOUT_LANE_STREAM: f = lane; n = sizeof(lane) / sizeof(size_t); sz = sizeof(zs_lane_stream); break;
        case ZS_LAYOUT_HALLUC_REPORT: f = rep; n = sizeof(rep) / sizeof(size_t); sz = sizeof(zs_halluc_report); break;
        default: return ZS_EINVAL;
    }
    if (size) *size = sz;
    for (size_t i = 0; offsets && i < n && i < cap; i++) offsets[i] = f[i];
    return (int)n;
}

extern "C" const char* zs_last_error(const zs_ctx* ctx) { return ctx ? ctx->err : "null context"; }

extern "C" void zs_ctx_destroy(zs_ctx* ctx) {
    if (!ctx) return;
    int dev = 0;
    (void)hipGetDevice(&dev);
    (void)hipSetDevice(ctx->device);
    for (int i = 0; i < 24; i++)
        if (ctx->events[i]) (void)hipEventDestroy((hipEvent_t)ctx->events[i]);
    if (ctx->fork_event) (void)hipEventDestroy((hipEvent_t)ctx->fork_event);
    if (ctx->join_event) (void)hipEventDestroy((hipEvent_t)ctx->join_event);
    if (ctx->side_stream) (void)hipStreamDestroy((hipStream_t)ctx->side_stream);
    for (int i = 0; i < 2; i++)
        if (ctx->lane_event[i]) {
            (void)hipEventSynchronize((hipEvent_t)ctx->lane_event[i]);
            (void)hipEventDestroy((hipEvent_t)ctx->lane_event[i]);
        }
    if (ctx->lane_host) (void)hipHostFree(ctx->lane_host);
    void* ptrs[] = {ctx->p_cnt, ctx->p_id, ctx->p_flags, ctx->p_y, ctx->rst, ctx->pairs, ctx->pv, ctx->mask_scratch, ctx->spec_chunks,
                    ctx->spec_rows, ctx->p_sub, ctx->k_ap, ctx->k_sum, ctx->s_rec, ctx->s_apx, ctx->gath, ctx->s_hterm, ctx->tp_bk, ctx->tp_cl, ctx->tp_pre, ctx->kcnt, ctx->tp_task, ctx->rw_part, ctx->rw_ctr,
                    ctx->lane_temp, ctx->lane_vals, ctx->lane_ih, ctx->lane_keys,
                    ctx->lane_idxs, ctx->lane_ck, ctx->lane_cn};
    for (void* p : ptrs)
        if (p) (void)hipFree(p);
    (void)hipSetDevice(dev);
    free(ctx);
}

extern "C" int zs_ctx_create(int device, uint32_t max_rows, uint32_t max_vocab, zs_ctx** out) {
    if (!out) return ZS_EINVAL;
    *out = nullptr;
    zs_ctx* ctx = (zs_ctx*)calloc(1, sizeof(zs_ctx));
    if (!ctx) return ZS_ENOMEM;
    if (max_rows == 0 || max_vocab == 0 || max_vocab > ZS_MAX_VOCAB) {
        free(ctx);
        return ZS_EINVAL;
    }
    ctx->device = device;
    ctx->max_rows = max_rows;
    ctx->max_vocab = max_vocab;
    ctx->max_chunks = (max_vocab + ZS_P1_CH - 1) / ZS_P1_CH;
    ctx->max_subs = ctx->max_chunks * ZS_SUBS_PER_CHUNK;
    int ndev = 0;
    if (hipGetDeviceCount(&ndev) != hipSuccess || device < 0 || device >= ndev) {
        free(ctx);
        return ZS_EHIP;
    }
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(device);
    int rc = ZS_OK;
    int ncu = 0;
    if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, device) != hipSuccess || ncu <= 0) ncu = 256;
    ctx->num_cus = (uint32_t)ncu;
    const size_t R = max_rows, C = ctx->max_chunks;
    if (!rc) rc = zs_alloc(ctx, &ctx->p_cnt, R);
    // the merged patch list: at most one entry per id of a row
    if (!rc) rc = zs_alloc(ctx, &ctx->p_id, R * (size_t)max_vocab);
    if (!rc) rc = zs_alloc(ctx, &ctx->p_flags, R * (size_t)max_vocab);
    if (!rc) rc = zs_alloc(ctx, &ctx->p_y, R * (size_t)max_vocab);
    if (!rc) rc = zs_alloc(ctx, &ctx->rst, R);
    if (!rc) rc = zs_alloc(ctx, &ctx->pairs, R * (size_t)max_vocab * 2 + 8);  // 16-byte loads at the tail
    if (!rc) rc = zs_alloc(ctx, &ctx->pv, R * (size_t)max_vocab + 4);  // 16-byte loads at the tail
    if (!rc) rc = zs_alloc(ctx, (uint32_t**)&ctx->mask_scratch, R);
    // epochs start at 1 over zeroed flags (set-up only, outside any stream
    // work a caller could capture)
    if (!rc && (hipMemset(ctx->mask_scratch, 0, R * sizeof(uint32_t)) != hipSuccess ||
                hipDeviceSynchronize() != hipSuccess))
        rc = ZS_EHIP;
    if (!rc) rc = zs_alloc(ctx, &ctx->spec_chunks, R * (2 * ZS_SPEC_KMAX + 1) * C);
    if (!rc) rc = zs_alloc(ctx, &ctx->p_sub, R * (ctx->max_subs + 1));
    if (!rc) rc = zs_alloc(ctx, &ctx->k_ap, R * ctx->max_subs);
    if (!rc) rc = zs_alloc(ctx, &ctx->k_sum, 3 * R * 2 * ctx->max_subs);   // records, then crossing records (24 bytes each)
    if (!rc) rc = zs_alloc(ctx, &ctx->s_rec, 3 * R * ZS_NSUM * ctx->max_subs);   // records, then crossing records (24 bytes each)
    if (!rc) rc = zs_alloc(ctx, &ctx->s_apx, R * 8 * ctx->max_subs);
    if (!rc) rc = zs_alloc(ctx, &ctx->gath, R * (2 * (size_t)max_vocab + 16));
    if (!rc) rc = zs_alloc(ctx, &ctx->s_hterm, R * ((size_t)max_vocab + 8));
    if (!rc) rc = zs_alloc(ctx, &ctx->tp_bk, R * ZS_TP_NB);
    if (!rc) rc = zs_alloc(ctx, &ctx->tp_cl, R * ZS_TP_CL);
    if (!rc) rc = zs_alloc(ctx, &ctx->tp_pre, R * (size_t)max_vocab * 2 + 8);  // 16-byte loads at the tail
    if (!rc) rc = zs_alloc(ctx, &ctx->kcnt, R * C * 2);
    if (!rc) rc = zs_alloc(ctx, &ctx->tp_task, 1 + R * ZS_TP_CAND);
    if (!rc) rc = zs_alloc(ctx, &ctx->rw_part, R * 2 * ZS_ROW_PART);
    if (!rc) rc = zs_alloc(ctx, &ctx->rw_ctr, R);
    // (set-up only, outside any stream work a caller could capture)
    if (!rc && (hipMemset(ctx->rw_ctr, 0, R * sizeof(uint32_t)) != hipSuccess || hipDeviceSynchronize() != hipSuccess))
        rc = ZS_EHIP;
    if (!rc) rc = zs_alloc(ctx, &ctx->spec_rows, R);
    // the lane knobs in one block laid out as the staging areas (temp, top_k,
    // top_p, seed; R each): one copy per call
    if (!rc) rc = zs_alloc(ctx, &ctx->lane_temp, 4 * (size_t)R);
    if (!rc) {
        ctx->lane_topk = reinterpret_cast<uint32_t*>(ctx->lane_temp + R);
        ctx->lane_topp = ctx->lane_temp + 2 * (size_t)R;
        ctx->lane_seed = reinterpret_cast<uint32_t*>(ctx->lane_temp + 3 * (size_t)R);
    }
    if (!rc) rc = zs_alloc(ctx, &ctx->lane_vals, R * ZS_LANE_K);
    if (!rc) rc = zs_alloc(ctx, &ctx->lane_idxs, R * ZS_LANE_K);
    if (!rc) rc = zs_alloc(ctx, &ctx->lane_ck, R * C * ZS_LANE_K);
    if (!rc) rc = zs_alloc(ctx, &ctx->lane_cn, R * C);
    if (!rc) rc = zs_alloc(ctx, &ctx->lane_ih, (size_t)ctx->max_vocab + 4);
    if (!rc) rc = zs_alloc(ctx, &ctx->lane_keys, R);
    if (!rc && hipMemset(ctx->lane_keys, 0, R * sizeof(unsigned long long)) != hipSuccess) rc = ZS_EHIP;
    if (!rc && (zs_lane_hash_fill(ctx->lane_ih, ctx->max_vocab + 4, nullptr) || hipDeviceSynchronize() != hipSuccess))
        rc = ZS_EHIP;
    if (!rc) {
        void* h = nullptr;
        hipEvent_t e0 = nullptr, e1 = nullptr;
        if (hipHostMalloc(&h, 8 * R * sizeof(uint32_t), hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&e0, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&e1, hipEventDisableTiming) != hipSuccess)
            rc = ZS_ENOMEM;
        ctx->lane_host = (uint32_t*)h;
        ctx->lane_event[0] = e0;
        ctx->lane_event[1] = e1;
        ctx->lane_slot = 0;
    }
    if (!rc) {
        hipStream_t s2 = nullptr;
        hipEvent_t e1 = nullptr, e2 = nullptr;
        if (hipStreamCreateWithFlags(&s2, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&e1, hipEventDisableTiming) != hipSuccess ||
            hipEventCreateWithFlags(&e2, hipEventDisableTiming) != hipSuccess)
            rc = ZS_EHIP;
        ctx->side_stream = s2;
        ctx->fork_event = e1;
        ctx->join_event = e2;
    }
    (void)hipSetDevice(prev);
    if (rc) {
        zs_ctx_destroy(ctx);
        return rc;
    }
    *out = ctx;
    return ZS_OK;
}

// ---------------------------------------------------------------------------
// token byte table
// ---------------------------------------------------------------------------
struct zs_vocab_dev {
    uint32_t* tok16;
    uint8_t* tlen;
};

extern "C" void zs_vocab_destroy(zs_vocab* v) {
    if (!v) return;
    (void)hipFree(v->d_offsets);
    (void)hipFree(v->d_bytes);
    (void)hipFree(v->d_valid);
    (void)hipFree(v->d_packed);
    (void)hipFree(v->d_wbytes);
    (void)hipFree(v->d_wmeta);
    free(v->h_offsets);
    free(v->h_bytes);
    free(v->h_valid);
    free(v);
}

extern "C" int zs_vocab_create(zs_ctx* ctx, const uint32_t* h_offsets, const uint8_t* h_bytes,
                               const uint8_t* h_valid, uint32_t ntab, uint32_t eos, zs_vocab** out) {
    if (!ctx || !out || !h_offsets || !h_valid || (!h_bytes && h_offsets[ntab] > 0))
        return zs_set_error(ctx, ZS_EINVAL, "zs_vocab_create: null argument");
    *out = nullptr;
    for (uint32_t t = 0; t < ntab; t++) {
        if (h_offsets[t + 1] < h_offsets[t])
            return zs_set_error(ctx, ZS_EINVAL, "zs_vocab_create: offsets decrease at %u", t);
        if (h_offsets[t + 1] - h_offsets[t] > 255)
            return zs_set_error(ctx, ZS_ELIMIT, "zs_vocab_create: token %u longer than 255 bytes", t);
    }
    zs_vocab* v = (zs_vocab*)calloc(1, sizeof(zs_vocab));
    v->ctx = ctx;
    v->ntab = ntab;
    v->eos = eos;
    // serials are unique in the process (a DFA's memo may meet vocabularies
    // of several contexts): 0 is never handed out
    static std::atomic<uint32_t> next_serial{0};
    v->serial = next_serial.fetch_add(1u, std::memory_order_relaxed) + 1u;
    v->nbytes = h_offsets[ntab] - h_offsets[0];
    v->h_offsets = (uint32_t*)malloc(sizeof(uint32_t) * (ntab + 1));
    v->h_bytes = (uint8_t*)malloc(v->nbytes + 1);
    v->h_valid = (uint8_t*)malloc(ntab + 1);
    for (uint32_t t = 0; t <= ntab; t++) v->h_offsets[t] = h_offsets[t] - h_offsets[0];
    if (v->nbytes) memcpy(v->h_bytes, h_bytes + h_offsets[0], v->nbytes);
    memcpy(v->h_valid, h_valid, ntab);
    // dense 16-byte prefix + length per token
    std::vector<uint32_t> tok16((size_t)ntab * 4 + 4, 0);
    std::vector<uint8_t> tlen(ntab + 1, 0);
    uint32_t maxlen = 0;
    for (uint32_t t = 0; t < ntab; t++) {
        uint32_t o = v->h_offsets[t], n = v->h_offsets[t + 1] - o;
        if (n > maxlen) maxlen = n;
        tlen[t] = (uint8_t)(n > 255 ? 255 : n);
        for (uint32_t i = 0; i < n && i < 16; i++) tok16[(size_t)t * 4 + i / 4] |= (uint32_t)v->h_bytes[o + i] << (8 * (i % 4));
    }
    v->maxlen = maxlen;
    // walk order by length inside each tile (tokens never allowed: length 0)
    v->nwtile = (ntab + ZS_WALK_TILE - 1) / ZS_WALK_TILE;
    std::vector<uint32_t> wbytes((size_t)v->nwtile * ZS_WALK_TILE * 4, 0), wmeta((size_t)v->nwtile * ZS_WALK_TILE, 0xffffffffu);
    for (uint32_t tl = 0; tl < v->nwtile; tl++) {
        std::vector<uint32_t> ids;
        for (uint32_t t = tl * ZS_WALK_TILE; t < ntab && t < (tl + 1) * ZS_WALK_TILE; t++) ids.push_back(t);
        // walk length: 0 = never allowed (not valid), 0x3fff = valid with no bytes
        auto wlen = [&](uint32_t t) { return h_valid[t] ? (tlen[t] ? (uint32_t)tlen[t] : 0x3fffu) : 0u; };
        std::stable_sort(ids.begin(), ids.end(), [&](uint32_t x, uint32_t y) { return wlen(x) < wlen(y); });
        for (size_t k = 0; k < ids.size(); k++) {
            const size_t slot = (size_t)tl * ZS_WALK_TILE + k;
            wmeta[slot] = ids[k] | (wlen(ids[k]) << 18);
            for (int q = 0; q < 4; q++) wbytes[slot * 4 + q] = tok16[(size_t)ids[k] * 4 + q];
        }
    }
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(ctx->device);
    int rc = ZS_OK;
    // d_packed holds tok16 followed by tlen (bytes)
    size_t tok_words = (size_t)ntab * 4 + 4;
    size_t len_words = (ntab + 4) / 4 + 1;
    if (!rc) rc = zs_alloc(ctx, &v->d_offsets, ntab + 1);
    if (!rc) rc = zs_alloc(ctx, &v->d_bytes, v->nbytes + 1);
    if (!rc) rc = zs_alloc(ctx, &v->d_valid, ntab + 1);
    if (!rc) rc = zs_alloc(ctx, &v->d_packed, tok_words + len_words);
    if (!rc) rc = zs_alloc(ctx, &v->d_wbytes, wbytes.size());
    if (!rc) rc = zs_alloc(ctx, &v->d_wmeta, wmeta.size());
    if (!rc) {
        hipError_t e = hipMemcpy(v->d_wbytes, wbytes.data(), wbytes.size() * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(v->d_wmeta, wmeta.data(), wmeta.size() * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy(v->d_offsets, v->h_offsets, sizeof(uint32_t) * (ntab + 1), hipMemcpyHostToDevice);
        if (e == hipSuccess && v->nbytes) e = hipMemcpy(v->d_bytes, v->h_bytes, v->nbytes, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(v->d_valid, v->h_valid, ntab, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(v->d_packed, tok16.data(), tok_words * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy((uint8_t*)(v->d_packed + tok_words), tlen.data(), ntab + 1, hipMemcpyHostToDevice);
        if (e != hipSuccess) rc = zs_set_error(ctx, ZS_EHIP, "zs_vocab_create: %s", hipGetErrorString(e));
    }
    (void)hipSetDevice(prev);
    if (rc) {
        zs_vocab_destroy(v);
        return rc;
    }
    *out = v;
    return ZS_OK;
}

// ---------------------------------------------------------------------------
// DFA
// ---------------------------------------------------------------------------
extern "C" void zs_dfa_destroy(zs_dfa* d) {
    if (!d) return;
    (void)hipFree(d->d_trans);
    (void)hipFree(d->d_cls);
    (void)hipFree(d->d_bad);
    (void)hipFree(d->d_accept);
    (void)hipFree(d->d_packed);
    (void)hipFree(d->d_clsinfo);
    (void)hipFree(d->d_remap);
    (void)hipFree(d->d_memo);
    (void)hipFree(d->d_memo_key);
    (void)hipFree(d->d_viable);
    free(d->h_viable);
    free(d->h_remap);
    (void)hipFree(d->d_memo_any);
    free(d->h_trans);
    free(d->h_dead);
    free(d->h_accept);
    free(d->h_live);
    free(d);
}

// is_live for every state (logit_fsm.rs:121-161): live(u) iff an accepting
// state is reachable from u through non-dead transitions, u included. The
// reference explores forward and iterates a fixpoint; the same set is the
// reverse-reachability closure of the accepting states.
static void zs_compute_live(const uint32_t* trans, const uint8_t* dead, const uint8_t* accept, uint32_t S,
                            uint8_t* live) {
    std::vector<uint32_t> roff(S + 1, 0), radj;
    for (uint32_t u = 0; u < S; u++)
        for (uint32_t b = 0; b < 256; b++) {
            uint32_t v = trans[(size_t)u * 256 + b];
            if (!dead[v]) roff[v + 1]++;
        }
    for (uint32_t i = 0; i < S; i++) roff[i + 1] += roff[i];
    radj.resize(roff[S]);
    std::vector<uint32_t> fill(roff.begin(), roff.end() - 1);
    for (uint32_t u = 0; u < S; u++)
        for (uint32_t b = 0; b < 256; b++) {
            uint32_t v = trans[(size_t)u * 256 + b];
            if (!dead[v]) radj[fill[v]++] = u;
        }
    std::vector<uint32_t> q;
    for (uint32_t u = 0; u < S; u++) {
        live[u] = accept[u] ? 1 : 0;
        if (live[u]) q.push_back(u);
    }
    for (size_t h = 0; h < q.size(); h++) {
        uint32_t v = q[h];
        for (uint32_t k = roff[v]; k < roff[v + 1]; k++) {
            uint32_t u = radj[k];
            if (!live[u]) { live[u] = 1; q.push_back(u); }
        }
    }
}

extern "C" int zs_dfa_create(zs_ctx* ctx, const uint32_t* h_trans, uint32_t nstates, const uint8_t* h_dead,
                             const uint8_t* h_accept, zs_dfa** out) {
    if (!ctx || !out || !h_trans || !h_dead || !h_accept || nstates == 0)
        return zs_set_error(ctx, ZS_EINVAL, "zs_dfa_create: null argument");
    *out = nullptr;
    if (nstates >= 0xffffu) return zs_set_error(ctx, ZS_ELIMIT, "zs_dfa_create: %u states (max 65534)", nstates);
    for (size_t i = 0; i < (size_t)nstates * 256; i++)
        if (h_trans[i] >= nstates) return zs_set_error(ctx, ZS_EINVAL, "zs_dfa_create: transition %zu out of range", i);
    zs_dfa* d = (zs_dfa*)calloc(1, sizeof(zs_dfa));
    d->ctx = ctx;
    d->nstates = nstates;
    d->h_trans = (uint32_t*)malloc(sizeof(uint32_t) * nstates * 256);
    d->h_dead = (uint8_t*)malloc(nstates);
    d->h_accept = (uint8_t*)malloc(nstates);
    d->h_live = (uint8_t*)malloc(nstates);
    memcpy(d->h_trans, h_trans, sizeof(uint32_t) * nstates * 256);
    for (uint32_t s = 0; s < nstates; s++) {
        d->h_dead[s] = h_dead[s] ? 1 : 0;
        d->h_accept[s] = h_accept[s] ? 1 : 0;
    }
    zs_compute_live(d->h_trans, d->h_dead, d->h_accept, nstates, d->h_live);
    // fold dead / quit / non-live targets into the sentinel, then byte classes
    std::vector<uint8_t> bad(nstates);
    for (uint32_t s = 0; s < nstates; s++) bad[s] = (d->h_dead[s] || !d->h_live[s]) ? 1 : 0;
    std::vector<uint16_t> col(nstates);
    std::map<std::vector<uint16_t>, uint32_t> classes;
    uint8_t cls[256];
    std::vector<std::vector<uint16_t>> cols;
    for (uint32_t b = 0; b < 256; b++) {
        for (uint32_t s = 0; s < nstates; s++) {
            uint32_t v = d->h_trans[(size_t)s * 256 + b];
            col[s] = bad[v] ? 0xffffu : (uint16_t)v;
        }
        auto it = classes.find(col);
        if (it == classes.end()) {
            uint32_t id = (uint32_t)classes.size();
            classes.emplace(col, id);
            cols.push_back(col);
            cls[b] = (uint8_t)id;
        } else {
            cls[b] = (uint8_t)it->second;
        }
    }
    uint32_t ncls = (uint32_t)cols.size();
    std::vector<uint16_t> tab((size_t)nstates * ncls);
    for (uint32_t c = 0; c < ncls; c++)
        for (uint32_t s = 0; s < nstates; s++) tab[(size_t)s * ncls + c] = cols[c][s];
    d->ncls = ncls;
    // bit-packed copy over the good states only
    std::vector<uint16_t> remap(nstates, 0xffffu);
    uint32_t ngood = 0;
    for (uint32_t s = 0; s < nstates; s++)
        if (!bad[s]) remap[s] = (uint16_t)ngood++;
    d->h_remap = (uint16_t*)malloc(sizeof(uint16_t) * nstates);
    memcpy(d->h_remap, remap.data(), sizeof(uint16_t) * nstates);
    d->h_viable = (uint8_t*)calloc(ngood + 1, 1);
    // the fail value is ngood, a sink row whose entries all lead to itself, so a
    // walk needs no liveness test per step; entries of `bits` bits packed back
    // to back inside a row, each row padded to whole 32-bit words (row s, class
    // c at bit s * rw + c * bits, rw = 32 * ceil(ncls * bits / 32)), so that the
    // walk finds an entry's first word with one multiply-add
    uint32_t bits = 1;
    while ((1u << bits) - 1u < ngood) bits++;
    const uint32_t rw = (ncls * bits + 31u) & ~31u;  // bits per state row
    const uint64_t nbits = (uint64_t)(ngood + 1) * rw;
    // + slack for the two-word reads, rounded to whole 16-byte quads
    std::vector<uint32_t> packed(((size_t)((nbits + 31) / 32 + 1) + 3) & ~(size_t)3, 0u);
    const uint32_t fail = ngood;
    for (uint32_t s = 0; s <= nstates; s++) {
        if (s < nstates && bad[s]) continue;
        const uint32_t row = s < nstates ? remap[s] : ngood;
        for (uint32_t c = 0; c < ncls; c++) {
            const uint16_t tgt = s < nstates ? cols[c][s] : 0xffffu;
            const uint64_t v = tgt == 0xffffu ? fail : remap[tgt];
            const uint64_t off = (uint64_t)row * rw + (uint64_t)c * bits;
            packed[off >> 5] |= (uint32_t)(v << (off & 31));
            if ((off & 31) + bits > 32) packed[(off >> 5) + 1] |= (uint32_t)(v >> (32 - (off & 31)));
        }
    }
    uint16_t clsinfo[256];
    for (uint32_t b = 0; b < 256; b++) clsinfo[b] = (uint16_t)(cls[b] * bits);
    d->ngood = ngood;
    d->bits = bits;
    {
        uint64_t goodt = 0;
        for (uint32_t s = 0; s < nstates; s++)
            if (!bad[s])
                for (uint32_t b = 0; b < 256; b++) goodt += bad[d->h_trans[(size_t)s * 256 + b]] ? 0 : 1;
        d->dense = goodt * 10 > (uint64_t)ngood * 256 * 3 ? 1 : 0;
    }
    d->rw = rw;
    d->packed_lds = packed.size() * 4 <= ZS_DFA_LDS_BYTES && rw < 65536 ? 1 : 0;
    uint32_t staged_words = 0;   // LDS-staged words of a form followed by its base map
    if (!d->packed_lds) {
        // Displaced rows (the double-array layout of a trie): good state g
        // gets a distinct base b_g, and its transition on class c is entry
        // b_g + c = b_g << 16 | b_target; an entry whose upper half is not the
        // reading state's base (another state's entry, or an empty one,
        // 0xffffffff) is a fail. A walk step is one 32-bit LDS read and a
        // compare. Bases are placed first-fit, states with the most
        // transitions first; the fail value F is a base no state owns.
        std::vector<uint32_t> order(ngood), nt(ngood, 0), gs(ngood);
        for (uint32_t s = 0; s < nstates; s++) {
            if (bad[s]) continue;
            const uint32_t g = remap[s];
            gs[g] = s;
            for (uint32_t c = 0; c < ncls; c++) nt[g] += cols[c][s] != 0xffffu;
        }
        for (uint32_t g = 0; g < ngood; g++) order[g] = g;
        std::stable_sort(order.begin(), order.end(), [&](uint32_t x, uint32_t y) { return nt[x] > nt[y]; });
        std::vector<uint8_t> occ, isbase;
        std::vector<uint32_t> base(ngood, 0);
        auto grow = [&](size_t n) {
            if (occ.size() < n) occ.resize(n, 0), isbase.resize(n, 0);
        };
        uint32_t first_free = 0, nent = 0;
        std::vector<uint32_t> cs;
        for (uint32_t g : order) {
            const uint32_t s = gs[g];
            cs.clear();
            for (uint32_t c = 0; c < ncls; c++)
                if (cols[c][s] != 0xffffu) cs.push_back(c);
            uint32_t b = cs.empty() ? 0 : (first_free > cs[0] ? first_free - cs[0] : 0);
            for (;; b++) {
                grow((size_t)b + ncls + 1);
                if (isbase[b]) continue;
                bool ok = true;
                for (uint32_t c : cs)
                    if (occ[b + c]) { ok = false; break; }
                if (ok) break;
            }
            base[g] = b;
            isbase[b] = 1;
            for (uint32_t c : cs) occ[b + c] = 1;
            while (first_free < occ.size() && occ[first_free]) first_free++;
            nent = std::max(nent, b + ncls);
        }
        uint32_t F = 0;
        while (F < isbase.size() && isbase[F]) F++;
        nent = std::max(nent, F + ncls);
        const size_t words = ((size_t)nent + 3) & ~(size_t)3;
        if (F < 0xffffu && nent <= 0xffffu && (words + ZS_DFA_RD_ROWS / 2) * 4 <= ZS_DFA_LDS_BYTES) {
            std::vector<uint32_t> rd(words, 0xffffffffu);
            for (uint32_t g = 0; g < ngood; g++) {
                const uint32_t s = gs[g];
                for (uint32_t c = 0; c < ncls; c++) {
                    const uint16_t tgt = cols[c][s];
                    if (tgt != 0xffffu) rd[base[g] + c] = base[g] << 16 | base[remap[tgt]];
                }
            }
            // then (not staged) the base of every state by its original id
            staged_words = (uint32_t)rd.size();
            rd.resize(rd.size() + (nstates + 1) / 2, 0u);
            uint16_t* map = reinterpret_cast<uint16_t*>(rd.data() + staged_words);
            for (uint32_t s = 0; s < nstates; s++) map[s] = bad[s] ? (uint16_t)F : (uint16_t)base[remap[s]];
            packed.swap(rd);
            for (uint32_t b = 0; b < 256; b++) clsinfo[b] = cls[b];
            d->sparse = 2;
            d->rd_fail = F;
            d->packed_lds = 1;
        }
    }
    if (!d->packed_lds && ncls <= 64) {
        // Sparse rows for tables past the LDS budget (large grammars are
        // mostly fail entries): per good state {class mask lo, hi, first
        // target, 0}, the sink last with an empty mask, then the u16 targets
        // of the set classes in class order.
        std::vector<uint32_t> rec((size_t)(ngood + 1) * 4, 0u);
        std::vector<uint16_t> tgts;
        for (uint32_t s = 0; s < nstates; s++) {
            if (bad[s]) continue;
            const uint32_t row = remap[s];
            uint64_t mask = 0;
            rec[(size_t)row * 4 + 2] = (uint32_t)tgts.size();
            for (uint32_t c = 0; c < ncls; c++) {
                const uint16_t tgt = cols[c][s];
                if (tgt == 0xffffu) continue;
                mask |= 1ull << c;
                tgts.push_back(remap[tgt]);
            }
            rec[(size_t)row * 4] = (uint32_t)mask;
            rec[(size_t)row * 4 + 1] = (uint32_t)(mask >> 32);
        }
        std::vector<uint32_t> sp(rec);
        sp.resize(rec.size() + (tgts.size() + 1) / 2, 0u);
        if (!tgts.empty()) memcpy(sp.data() + rec.size(), tgts.data(), tgts.size() * 2);
        sp.resize((sp.size() + 3) & ~(size_t)3, 0u);
        if (sp.size() * 4 <= ZS_DFA_LDS_BYTES) {
            packed.swap(sp);
            for (uint32_t b = 0; b < 256; b++) clsinfo[b] = cls[b];
            d->sparse = 1;
            d->packed_lds = 1;
        }
    }
    int prev = 0;
    (void)hipGetDevice(&prev);
    (void)hipSetDevice(ctx->device);
    int rc = ZS_OK;
    if (!rc) rc = zs_alloc(ctx, &d->d_trans, tab.size());
    if (!rc) rc = zs_alloc(ctx, &d->d_cls, 256);
    if (!rc) rc = zs_alloc(ctx, &d->d_bad, nstates);
    if (!rc) rc = zs_alloc(ctx, &d->d_accept, nstates);
    if (!rc) rc = zs_alloc(ctx, &d->d_packed, packed.size());
    if (!rc) rc = zs_alloc(ctx, &d->d_clsinfo, 256);
    if (!rc) rc = zs_alloc(ctx, &d->d_remap, nstates);
    // the memo: one slot of ceil(max_vocab / 32) words per good state, up to
    // ZS_DFA_MEMO_BYTES (states past the cap are walked on every call)
    d->memo_words = (ctx->max_vocab + 31) / 32;
    d->memo_slots = (uint32_t)std::min<uint64_t>(std::min<uint64_t>(ngood, 0xfff0u),
                                                  ZS_DFA_MEMO_BYTES / ((uint64_t)d->memo_words * 4));
    d->memo_tag = 1;   // the keys start at 0: tag 0 is never used
    if (!rc && d->memo_slots) rc = zs_alloc(ctx, &d->d_memo, (size_t)d->memo_slots * d->memo_words);
    if (!rc && d->memo_slots) rc = zs_alloc(ctx, &d->d_memo_key, d->memo_slots);
    if (!rc) rc = zs_alloc(ctx, &d->d_viable, ngood + 1);
    if (!rc && d->memo_slots) rc = zs_alloc(ctx, &d->d_memo_any, d->memo_slots);
    if (!rc && d->memo_slots && hipMemset(d->d_memo_key, 0, (size_t)d->memo_slots * 8) != hipSuccess)
        rc = zs_set_error(ctx, ZS_EHIP, "zs_dfa_create: memo clear failed");
    if (!rc) {
        d->packed_words = staged_words ? staged_words : (uint32_t)packed.size();
        hipError_t e = hipMemcpy(d->d_packed, packed.data(), packed.size() * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(d->d_clsinfo, clsinfo, 256 * 2, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(d->d_remap, remap.data(), nstates * 2, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(d->d_trans, tab.data(), tab.size() * 2, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(d->d_cls, cls, 256, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(d->d_bad, bad.data(), nstates, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = hipMemcpy(d->d_accept, d->h_accept, nstates, hipMemcpyHostToDevice);
        if (e != hipSuccess) rc = zs_set_error(ctx, ZS_EHIP, "zs_dfa_create: %s", hipGetErrorString(e));
    }
    (void)hipSetDevice(prev);
    if (rc) {
        zs_dfa_destroy(d);
        return rc;
    }
    *out = d;
    return ZS_OK;
}

extern "C" int zs_dfa_table_form(const zs_dfa* d) {
    if (!d) return -1;
    return d->packed_lds ? (int)d->sparse : 3;
}

extern "C" int zs_dfa_is_live(const zs_dfa* d, uint32_t s) { return (d && s < d->nstates) ? d->h_live[s] : 0; }
extern "C" int zs_dfa_is_accept(const zs_dfa* d, uint32_t s) {
    return (d && s < d->nstates) ? d->h_accept[s] : 0;
}

extern "C" int zs_dfa_advance(const zs_dfa* d, const zs_vocab* v, uint32_t state, uint32_t token,
                              uint32_t* out_state, int* viable) {
    if (!d || !v || !out_state || state >= d->nstates) return ZS_EINVAL;
    *out_state = state;
    if (viable) *viable = 1;
    if (token == v->eos) return ZS_OK;                    // logit_fsm.rs:277-279
    if (token >= v->ntab || !v->h_valid[token]) return ZS_OK;
    uint32_t s = state;
    for (uint32_t i = v->h_offsets[token]; i < v->h_offsets[token + 1]; i++) {
        s = d->h_trans[(size_t)s * 256 + v->h_bytes[i]];
        if (d->h_dead[s]) {                               // logit_fsm.rs:283-287
            if (viable) *viable = 0;
            return ZS_OK;
        }
    }
    *out_state = s;
    return ZS_OK;
}

// Is the viability of every good state (some token of the vocabulary is
// allowed, logit_fsm.rs:258-262) known without walking the vocabulary? A
// state is viable when the vocabulary has a valid empty token (allowed from
// every live state) or a single-byte token b with trans(s, b) neither dead
// nor non-live (logit_fsm.rs:170-178); it is not viable when no byte leads to
// such a state and there is no empty token (every walk of one byte or more
// fails at its first byte). Otherwise it stays open and the mask kernel's
// walk decides. Fills d->h_viable per good state; returns 1 when no state is
// open. Host, once per (DFA, vocabulary): nstates * 256 steps.
static uint32_t zs_dfa_all_quick(const zs_dfa* d, const zs_vocab* v) {
    bool has1[256] = {false}, empty = false;
    for (uint32_t t = 0; t < v->ntab; t++) {
        if (!v->h_valid[t]) continue;
        const uint32_t n = v->h_offsets[t + 1] - v->h_offsets[t];
        if (n == 0) empty = true;
        if (n == 1) has1[v->h_bytes[v->h_offsets[t]]] = true;
    }
    uint32_t all = 1;
    for (uint32_t s = 0; s < d->nstates; s++) {
        if (d->h_dead[s] || !d->h_live[s]) continue;
        bool one = false, any_good = false;
        for (uint32_t b = 0; b < 256 && !one; b++) {
            const uint32_t u = d->h_trans[(size_t)s * 256 + b];
            const bool good = !d->h_dead[u] && d->h_live[u];
            any_good |= good;
            one = good && has1[b];
        }
        const uint32_t g = d->h_remap[s];
        d->h_viable[g] = (empty || one) ? 1 : 0;
        if (!empty && !one && any_good) all = 0;
    }
    return all;
}

extern "C" void zs_dfa_memo_clear(zs_dfa* dfa) {
    if (!dfa) return;
    // a slot is valid only while its word equals the tag; the words are
    // zeroed at creation, so tag 0 is skipped (after 2^32 - 1 clears a slot
    // could hold a stale tag: the memo is then dropped for this DFA)
    if (++dfa->memo_tag == 0) {
        dfa->memo_tag = 1;
        dfa->memo_slots = 0;
    }
}

extern "C" int zs_dfa_mask(zs_ctx* ctx, const zs_dfa* dfa, const zs_vocab* vocab, const int32_t* d_states,
                           uint32_t B, uint32_t V, uint32_t* d_out_bits, uint32_t* d_any, void* stream) {
    if (!ctx || !dfa || !vocab || !d_states || !d_out_bits)
        return zs_set_error(ctx, ZS_EINVAL, "zs_dfa_mask: null argument");
    if (B == 0) return ZS_OK;
    if (B > ctx->max_rows) return zs_set_error(ctx, ZS_ELIMIT, "zs_dfa_mask: B=%u > max_rows=%u", B, ctx->max_rows);
    dm_args a{};
    a.trans = dfa->d_trans;
    a.cls = dfa->d_cls;
    a.bad_start = dfa->d_bad;
    a.accept = dfa->d_accept;
    size_t tok_words = (size_t)vocab->ntab * 4 + 4;
    a.tok16 = vocab->d_packed;
    a.tlen = (const uint8_t*)(vocab->d_packed + tok_words);
    a.offsets = vocab->d_offsets;
    a.bytes = vocab->d_bytes;
    a.valid = vocab->d_valid;
    a.ntab = vocab->ntab;
    a.eos = vocab->eos;
    a.nstates = dfa->nstates;
    a.ncls = dfa->ncls;
    a.packed = dfa->d_packed;
    a.packed_words = dfa->packed_words;
    a.wbytes = vocab->d_wbytes;
    a.wmeta = vocab->d_wmeta;
    a.nwtile = vocab->nwtile;
    a.clsinfo = dfa->d_clsinfo;
    a.remap = dfa->d_remap;
    a.ngood = dfa->ngood;
    a.sparse = dfa->sparse;
    a.rd_fail = dfa->rd_fail;
    a.rdmap = dfa->sparse == 2 ? reinterpret_cast<const uint16_t*>(dfa->d_packed + dfa->packed_words) : nullptr;
    a.dense = dfa->dense;
    a.bits = dfa->bits;
    a.rw = dfa->rw;
    a.states = d_states;
    a.B = B;
    a.V = V;
    a.words = (V + 31) / 32;
    a.out = d_out_bits;
    const bool packed = dfa->packed_lds != 0 && B <= ZS_DFA_MAXROWS;
    // the memo holds masks of one (vocabulary, V): another pair invalidates it
    if (dfa->memo_serial != vocab->serial || dfa->memo_V != V) {
        if (dfa->memo_serial != vocab->serial) {
            dfa->all_quick = zs_dfa_all_quick(dfa, vocab);
            if (dfa->all_quick &&
                hipMemcpyAsync(dfa->d_viable, dfa->h_viable, dfa->ngood ? dfa->ngood : 1, hipMemcpyHostToDevice,
                               (hipStream_t)stream) != hipSuccess)
                dfa->all_quick = 0;
        }
        dfa->memo_serial = vocab->serial;
        dfa->memo_V = V;
        zs_dfa_memo_clear(const_cast<zs_dfa*>(dfa));
    }
    a.eos_direct = dfa->all_quick;
    a.viable = dfa->d_viable;
    a.memo = dfa->d_memo;
    a.memo_key = dfa->d_memo_key;
    a.memo_any = dfa->d_memo_any;
    a.memo_seq = ++dfa->memo_seq;
    a.memo_slots = V <= ctx->max_vocab ? dfa->memo_slots : 0u;
    a.memo_words = dfa->memo_words;
    a.memo_tag = dfa->memo_tag;
    // Viability flags: the context's flags hold the epoch of the call that
    // found a viable token, on both kernel paths (no clearing pass, and a flag
    // left by an earlier call on the other path never reads as viable); the
    // caller's d_any then receives 0/1 from the EOS kernel. Only the
    // L2-table path with a caller-supplied d_any uses plain cleared flags.
    uint32_t* any = d_any;
    a.epoch = 0;
    if (packed || !d_any) {
        if (++ctx->mask_epoch == 0) ctx->mask_epoch = 1;  // 0 is what the flags start as
        a.epoch = ctx->mask_epoch;
        a.any_user = d_any;
        any = (uint32_t*)ctx->mask_scratch;
    }
    if (zs_dfa_mask_launch(a, packed, ctx->num_cus, any, (hipStream_t)stream))
        return zs_set_error(ctx, ZS_EHIP, "zs_dfa_mask: launch failed: %s", hipGetErrorString(hipGetLastError()));
    return ZS_OK;
}

extern "C" int zs_sample(zs_ctx* ctx, const zs_batch* b, void* stream) {
    if (!ctx || !b) return zs_set_error(ctx, ZS_EINVAL, "zs_sample: null argument");
    if (b->B == 0) return ZS_OK;
    if (b->B > ctx->max_rows) return zs_set_error(ctx, ZS_ELIMIT, "zs_sample: B=%u > max_rows=%u", b->B, ctx->max_rows);
    if (b->V == 0 || b->V > ctx->max_vocab)
        return zs_set_error(ctx, ZS_ELIMIT, "zs_sample: V=%u outside 1..max_vocab=%u", b->V, ctx->max_vocab);
    if (b->ld < b->V || (b->ld & 3u) || ((uintptr_t)b->d_logits & 15u))
        return zs_set_error(ctx, ZS_EINVAL, "zs_sample: ld must be >= V and a multiple of 4, logits 16-byte aligned");
    if (!b->d_logits || !b->d_params || !b->d_seed || !b->d_counter || !b->d_token || !b->d_logprob ||
        !b->d_top_ids || !b->d_top_lps || !b->d_top_n || !b->d_entropy || !b->d_max_prob || !b->d_margin ||
        !b->d_chosen_lp || !b->d_status)
        return zs_set_error(ctx, ZS_EINVAL, "zs_sample: null required pointer");
    if (b->top_stride == 0) return zs_set_error(ctx, ZS_EINVAL, "zs_sample: top_stride must be >= 1");
    if ((b->d_cnt_off && (!b->d_cnt_ids || !b->d_cnt_vals)) || (b->d_bias_off && (!b->d_bias_ids || !b->d_bias_vals)) ||
        (b->d_ban_off && !b->d_ban_ids))
        return zs_set_error(ctx, ZS_EINVAL, "zs_sample: CSR offsets without entries");
    if (b->d_allow_bits && b->allow_words < (b->V + 31) / 32)
        return zs_set_error(ctx, ZS_EINVAL, "zs_sample: allow_words < ceil(V/32)");
    int prev = 0;
    (void)hipGetDevice(&prev);
    if (prev != ctx->device) (void)hipSetDevice(ctx->device);
    int rc = zs_sample_launch(ctx, b, (hipStream_t)stream);
    if (prev != ctx->device) (void)hipSetDevice(prev);
    return rc;
}

extern "C" int zs_set_profiling(zs_ctx* ctx, int on) {
    if (!ctx) return ZS_EINVAL;
    if (on && !ctx->events[0]) {
        int prev = 0;
        (void)hipGetDevice(&prev);
        (void)hipSetDevice(ctx->device);
        for (int i = 0; i < 24; i++) {
            hipEvent_t e;
            ZS_HIP(ctx, hipEventCreate(&e));
            ctx->events[i] = e;
        }
        for (int i = 0; i < 8; i++) {
            hipEvent_t e;
            ZS_HIP(ctx, hipEventCreate(&e));
            ctx->spec_events[i] = e;
        }
        (void)hipSetDevice(prev);
    }
    ctx->profiling = on ? 1 : 0;
    ctx->n_timed = 0;
    ctx->n_spec_timed = 0;
    return ZS_OK;
}

extern "C" int zs_last_timings(zs_ctx* ctx, const char** names, float* ms, int cap) {
    if (!ctx) return ZS_EINVAL;
    int k = 0;
    const int n = ctx->n_timed, m = ctx->n_spec_timed;
    if (n > 0) {
        ZS_HIP(ctx, hipEventSynchronize((hipEvent_t)ctx->events[n]));
        for (int i = 0; i < n && k < cap; i++, k++) {
            float t = 0.f;
            ZS_HIP(ctx, hipEventElapsedTime(&t, (hipEvent_t)ctx->events[i], (hipEvent_t)ctx->events[i + 1]));
            if (names) names[k] = ctx->timed_names[i + 1];
            if (ms) ms[k] = t;
        }
    }
    if (m > 0) {
        ZS_HIP(ctx, hipEventSynchronize((hipEvent_t)ctx->spec_events[m]));
        for (int i = 0; i < m && k < cap; i++, k++) {
            float t = 0.f;
            ZS_HIP(ctx, hipEventElapsedTime(&t, (hipEvent_t)ctx->spec_events[i], (hipEvent_t)ctx->spec_events[i + 1]));
            if (names) names[k] = ctx->spec_names[i + 1];
            if (ms) ms[k] = t;
        }
    }
    return k;
}

static int zs_device_guard_begin(zs_ctx* ctx) {
    int prev = 0;
    (void)hipGetDevice(&prev);
    if (prev != ctx->device) (void)hipSetDevice(ctx->device);
    return prev;
}
static void zs_device_guard_end(zs_ctx* ctx, int prev) {
    if (prev != ctx->device) (void)hipSetDevice(prev);
}

extern "C" int zs_spec_verify(zs_ctx* ctx, const zs_spec_batch* b, void* stream) {
    if (!ctx || !b) return zs_set_error(ctx, ZS_EINVAL, "zs_spec_verify: null argument");
    if (b->B == 0) return ZS_OK;
    if (b->B > ctx->max_rows || b->V == 0 || b->V > ctx->max_vocab || b->k > ZS_SPEC_KMAX)
        return zs_set_error(ctx, ZS_ELIMIT, "zs_spec_verify: B=%u V=%u k=%u outside the context limits", b->B, b->V,
                            b->k);
    if (!b->d_target || (b->k && !b->d_draft_ids) || !b->d_temperature || !b->d_seed || !b->d_counter ||
        !b->d_accepted || !b->d_next)
        return zs_set_error(ctx, ZS_EINVAL, "zs_spec_verify: null required pointer");
    if (b->ld < b->V || (b->ld & 3u) || ((uintptr_t)b->d_target & 15u) || ((uintptr_t)b->d_draft & 15u))
        return zs_set_error(ctx, ZS_EINVAL, "zs_spec_verify: ld must be >= V and a multiple of 4, logits 16-byte aligned");
    zs_spec_args a{};
    a.B = b->B; a.V = b->V; a.k = b->k; a.ld = b->ld;
    a.target = b->d_target; a.draft = b->k ? b->d_draft : nullptr; a.draft_ids = b->d_draft_ids;
    a.temperature = b->d_temperature; a.seed = b->d_seed; a.counter = b->d_counter;
    a.accepted = b->d_accepted; a.next = b->d_next;
    a.cst = ctx->spec_chunks; a.rs = ctx->spec_rows;
    a.nch = ctx->max_chunks; a.npos_max = 2 * ZS_SPEC_KMAX + 1;
    if (b->flags & ~(uint32_t)ZS_SPEC_BACKGROUND)
        return zs_set_error(ctx, ZS_EINVAL, "zs_spec_verify: unknown flags %#x", b->flags);
    a.background = (b->flags & ZS_SPEC_BACKGROUND) ? 1u : 0u;
    int prev = zs_device_guard_begin(ctx);
    zs_prof prof{ctx->profiling, ctx->spec_events, ctx->spec_names, &ctx->n_spec_timed};
    int rc = zs_spec_launch(a, prof, (hipStream_t)stream);
    zs_device_guard_end(ctx, prev);
    if (rc) return zs_set_error(ctx, ZS_EHIP, "zs_spec_verify: launch failed: %s", hipGetErrorString(hipGetLastError()));
    return ZS_OK;
}

static int lane_check(zs_ctx* ctx, uint32_t B, uint32_t V, uint64_t ld, const void* logits, const char* who) {
    if (!ctx || !logits) return zs_set_error(ctx, ZS_EINVAL, "%s: null argument", who);
    if (ld < V || (ld & 3u) || ((uintptr_t)logits & 15u))
        return zs_set_error(ctx, ZS_EINVAL, "%s: ld must be >= V and a multiple of 4, logits 16-byte aligned", who);
    return ZS_OK;
}

extern "C" int zs_lane_argmax(zs_ctx* ctx, const float* d_logits, uint32_t B, uint32_t V, uint64_t ld,
                              uint32_t* d_out, void* stream) {
    int rc = lane_check(ctx, B, V, ld, d_logits, "zs_lane_argmax");
    if (rc) return rc;
    if (!d_out) return zs_set_error(ctx, ZS_EINVAL, "zs_lane_argmax: null output");
    if (B == 0) return ZS_OK;
    int prev = zs_device_guard_begin(ctx);
    rc = zs_lane_argmax_launch(d_logits, B, V, ld, nullptr, nullptr, nullptr, nullptr, d_out, (hipStream_t)stream);
    zs_device_guard_end(ctx, prev);
    return rc ? zs_set_error(ctx, ZS_EHIP, "zs_lane_argmax: launch failed") : ZS_OK;
}

extern "C" int zs_lane_sample(zs_ctx* ctx, const float* d_logits, uint32_t B, uint32_t V, uint64_t ld,
                              const float* d_temperature, const uint32_t* d_seed, uint32_t* d_out, void* stream) {
    int rc = lane_check(ctx, B, V, ld, d_logits, "zs_lane_sample");
    if (rc) return rc;
    if (!d_out || !d_temperature || !d_seed) return zs_set_error(ctx, ZS_EINVAL, "zs_lane_sample: null argument");
    if (B == 0) return ZS_OK;
    int prev = zs_device_guard_begin(ctx);
    rc = zs_lane_argmax_launch(d_logits, B, V, ld, d_temperature, d_seed, ctx->lane_ih, ctx->lane_keys, d_out, (hipStream_t)stream);
    zs_device_guard_end(ctx, prev);
    return rc ? zs_set_error(ctx, ZS_EHIP, "zs_lane_sample: launch failed") : ZS_OK;
}

extern "C" int zs_lane_topk(zs_ctx* ctx, const float* d_logits, uint32_t B, uint32_t V, uint64_t ld, uint32_t K,
                            float* d_vals, uint32_t* d_idxs, void* stream) {
    int rc = lane_check(ctx, B, V, ld, d_logits, "zs_lane_topk");
    if (rc) return rc;
    if (!d_vals || !d_idxs) return zs_set_error(ctx, ZS_EINVAL, "zs_lane_topk: null output");
    if (K == 0 || K > 1024) return zs_set_error(ctx, ZS_ELIMIT, "zs_lane_topk: K=%u outside 1..1024", K);
    if (B == 0) return ZS_OK;
    int prev = zs_device_guard_begin(ctx);
    const bool fits = B <= ctx->max_rows && V <= ctx->max_vocab;
    rc = zs_lane_topk_launch(d_logits, B, V, ld, K, d_vals, d_idxs, fits ? ctx->lane_ck : nullptr,
                             fits ? ctx->lane_cn : nullptr, (hipStream_t)stream);
    zs_device_guard_end(ctx, prev);
    return rc ? zs_set_error(ctx, ZS_EHIP, "zs_lane_topk: launch failed") : ZS_OK;
}

extern "C" int zs_lane_sample_topk(zs_ctx* ctx, const float* d_vals, const uint32_t* d_idxs, uint32_t B, uint32_t K,
                                   const float* d_temperature, const uint32_t* d_top_k, const float* d_top_p,
                                   const uint32_t* d_seed, uint32_t* d_out, void* stream) {
    if (!ctx || !d_vals || !d_idxs || !d_temperature || !d_top_k || !d_top_p || !d_seed || !d_out)
        return zs_set_error(ctx, ZS_EINVAL, "zs_lane_sample_topk: null argument");
    if (K == 0) return zs_set_error(ctx, ZS_EINVAL, "zs_lane_sample_topk: K == 0");
    if (B == 0) return ZS_OK;
    int prev = zs_device_guard_begin(ctx);
    int rc = zs_lane_sample_topk_launch(d_vals, d_idxs, B, K, d_temperature, d_top_k, d_top_p, d_seed, d_out,
                                        (hipStream_t)stream);
    zs_device_guard_end(ctx, prev);
    return rc ? zs_set_error(ctx, ZS_EHIP, "zs_lane_sample_topk: launch failed") : ZS_OK;
}

extern "C" uint32_t zs_step_seed(uint32_t base, uint32_t gen_idx) { return base + gen_idx * 0x9E3779B1u; }

// ContinuousBatcher::step's token selection (gpu/batch.rs:176-192) with the
// CPU nucleus over the read-back top-64 pool (gpu/mod.rs:2213-2229) moved to
// the device: one call, m ids out, nothing read back.
extern "C" int zs_lane_step(zs_ctx* ctx, const float* d_logits, uint32_t m, uint32_t V, uint64_t ld,
                            const zs_lane_stream* h_streams, uint32_t* d_out, int* path, void* stream) {
    int rc = lane_check(ctx, m, V, ld, d_logits, "zs_lane_step");
    if (rc) return rc;
    if (!d_out || (m && !h_streams)) return zs_set_error(ctx, ZS_EINVAL, "zs_lane_step: null argument");
    if (m > ctx->max_rows) return zs_set_error(ctx, ZS_ELIMIT, "zs_lane_step: m=%u > max_rows=%u", m, ctx->max_rows);
    if (V == 0) return zs_set_error(ctx, ZS_EINVAL, "zs_lane_step: V == 0");
    // the cheapest path that serves every stream: top-K > temperature > greedy
    int p = ZS_LANE_ARGMAX;
    for (uint32_t i = 0; i < m; i++) {
        const zs_lane_stream& s = h_streams[i];
        if (s.top_k > 0 || (s.top_p > 0.0f && s.top_p < 1.0f)) { p = ZS_LANE_TOPK; break; }  // needs_topk
        if (s.temp > 0.0f) p = ZS_LANE_SAMPLE;
    }
    if (path) *path = p;
    if (m == 0) return ZS_OK;
    const hipStream_t st = (hipStream_t)stream;
    const int prev = zs_device_guard_begin(ctx);
    if (p != ZS_LANE_ARGMAX) {
        // two staging areas, alternating: wait for the copy made from this
        // one two calls ago (the call before it keeps running meanwhile)
        const uint32_t slot = ctx->lane_slot;
        ctx->lane_slot ^= 1u;
        if (hipEventSynchronize((hipEvent_t)ctx->lane_event[slot]) != hipSuccess) rc = ZS_EHIP;
        const size_t R = ctx->max_rows;
        uint32_t* area = ctx->lane_host + (size_t)slot * 4 * R;
        float* ht = (float*)area;
        uint32_t* hk = area + R;
        float* hp = (float*)(area + 2 * R);
        uint32_t* hs = area + 3 * R;
        for (uint32_t i = 0; i < m; i++) {
            ht[i] = h_streams[i].temp;
            hk[i] = h_streams[i].top_k;
            hp[i] = h_streams[i].top_p;
            hs[i] = zs_step_seed(h_streams[i].base_seed, h_streams[i].gen_index);
        }
        // one copy of the whole area (the four knob arrays; entries past m unused)
        const size_t nb = (3 * R + m) * 4;
        if (!rc && (hipMemcpyAsync(ctx->lane_temp, area, nb, hipMemcpyHostToDevice, st) != hipSuccess ||
                    hipEventRecord((hipEvent_t)ctx->lane_event[slot], st) != hipSuccess))
            rc = ZS_EHIP;
    }
    if (!rc) {
        if (p == ZS_LANE_ARGMAX)
            rc = zs_lane_argmax_launch(d_logits, m, V, ld, nullptr, nullptr, nullptr, nullptr, d_out, st);
        else if (p == ZS_LANE_SAMPLE)
            rc = zs_lane_argmax_launch(d_logits, m, V, ld, ctx->lane_temp, ctx->lane_seed, ctx->lane_ih, ctx->lane_keys, d_out, st);
        else {
            rc = zs_lane_topk_draw_launch(d_logits, m, V, ld, ZS_LANE_K, ctx->lane_vals, ctx->lane_idxs,
                                          V <= ctx->max_vocab ? ctx->lane_ck : nullptr, ctx->lane_cn, ctx->lane_temp,
                                          ctx->lane_topk, ctx->lane_topp, ctx->lane_seed, d_out, st);
        }
        if (rc) rc = ZS_EHIP;
    }
    zs_device_guard_end(ctx, prev);
    return rc ? zs_set_error(ctx, rc, "zs_lane_step: %s", hipGetErrorString(hipGetLastError())) : ZS_OK;
}
