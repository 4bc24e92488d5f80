/*
 * zs_oracle.c -- CPU restatement of the reference (fankh/zllm) logits
 * post-processing and sampling path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the parity checker: tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it; the product
 * (zllm_amd/, libzs.so) never links, calls or routes through it.
 *
 * Every function restates one reference function and cites it (file:line
 * relative to the reference repo root). Arithmetic is IEEE f32 exactly as the
 * Rust source performs it: sequential sums in index order, glibc expf/logf
 * (Rust's f32::exp/ln lower to them on Linux), no FMA contraction (built with
 * -ffp-contract=off), IEEE division.
 *
 * Parity status of each function is recorded in the header comment of the
 * function; "pinned" means a reference known-answer test, a closed form or a
 * brute-force check in tests/ covers it.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ZO_API __attribute__((visibility("default")))

static inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

/* Rust f32::total_cmp key (core::f32::total_cmp): flip the magnitude bits of
 * negative numbers, then compare as i32. */
static inline int32_t total_key(float f) {
    int32_t b = (int32_t)f2u(f);
    b ^= (int32_t)(((uint32_t)(b >> 31)) >> 1);
    return b;
}

typedef struct { uint32_t idx; float val; } pair_t;

/* Descending by total_cmp, ties by ascending index == Rust's stable
 * `sort_by(|a, b| b.1.total_cmp(&a.1))` over (index, value) pairs that start in
 * index order. */
static int cmp_desc_total(const void* a, const void* b) {
    const pair_t* x = (const pair_t*)a;
    const pair_t* y = (const pair_t*)b;
    int32_t kx = total_key(x->val), ky = total_key(y->val);
    if (kx != ky) return kx > ky ? -1 : 1;
    return x->idx < y->idx ? -1 : (x->idx > y->idx);
}

/* Rust f32::max: if either operand is NaN the other is returned (libm fmaxf). */
static inline float rmax(float a, float b) { return fmaxf(a, b); }

/* -------------------------------------------------------------------------
 * sampler.rs:31-128  sample_with_rng, with the uniform r injected (the draw
 * `rng.random_range(0.0..1.0)` at :118 is the only RNG use; r is passed in).
 * Returns the sampled id. `work` must hold 3*V floats + V pairs (caller
 * provides via zo_sample_with_r which allocates).
 * Parity: pinned by sampler.rs tests (:134-192), closed forms (T<=0 argmax,
 * top_k>=V no-op, top_p>=1 no-op) and brute force in tests/.
 * ------------------------------------------------------------------------- */
ZO_API uint32_t zo_sample_with_r(const float* logits_in, uint32_t V, float temperature,
                                 uint32_t top_k, float top_p, float min_p, float r) {
    if (V == 0) return 0;
    /* :35-42 greedy: max_by(partial_cmp, unwrap_or(Equal)) -> last maximal
     * element; cmp::max_by returns v2 unless compare(v1, v2) == Greater. */
    if (temperature <= 0.0f) {
        uint32_t best = 0;
        float bv = logits_in[0];
        for (uint32_t i = 1; i < V; i++) {
            float v = logits_in[i];
            int greater = (bv > v); /* partial_cmp(best, v) == Greater */
            if (!greater) { best = i; bv = v; }
        }
        return best;
    }
    float* l = (float*)malloc(sizeof(float) * V);
    float* probs = (float*)malloc(sizeof(float) * V);
    pair_t* idx = (pair_t*)malloc(sizeof(pair_t) * V);
    memcpy(l, logits_in, sizeof(float) * V);
    /* :47-51 temperature */
    if (temperature != 1.0f)
        for (uint32_t i = 0; i < V; i++) l[i] = l[i] / temperature;
    /* :54-64 top-k: stable sort desc by total_cmp, threshold = sorted[k-1] */
    if (top_k > 0 && top_k < V) {
        for (uint32_t i = 0; i < V; i++) { idx[i].idx = i; idx[i].val = l[i]; }
        qsort(idx, V, sizeof(pair_t), cmp_desc_total);
        float thr = idx[top_k - 1].val;
        for (uint32_t i = 0; i < V; i++)
            if (l[i] < thr) l[i] = -INFINITY;
    }
    /* :67-69 softmax with sequential f32 sum */
    float m = -INFINITY;
    for (uint32_t i = 0; i < V; i++) m = rmax(m, l[i]);
    float s = -0.0f;
    for (uint32_t i = 0; i < V; i++) s = s + expf(l[i] - m);
    for (uint32_t i = 0; i < V; i++) probs[i] = expf(l[i] - m) / s;
    /* :72-88 min-p */
    if (min_p > 0.0f) {
        float pmax = 0.0f;
        for (uint32_t i = 0; i < V; i++) pmax = rmax(pmax, probs[i]);
        float cutoff = min_p * pmax;
        float kept = 0.0f;
        for (uint32_t i = 0; i < V; i++) {
            if (probs[i] < cutoff) probs[i] = 0.0f;
            else kept += probs[i];
        }
        if (kept > 0.0f)
            for (uint32_t i = 0; i < V; i++) probs[i] /= kept;
    }
    /* :91-115 top-p */
    if (top_p < 1.0f) {
        for (uint32_t i = 0; i < V; i++) { idx[i].idx = i; idx[i].val = probs[i]; }
        qsort(idx, V, sizeof(pair_t), cmp_desc_total);
        float* filtered = l; /* reuse */
        for (uint32_t i = 0; i < V; i++) filtered[i] = 0.0f;
        float cumsum = 0.0f;
        for (uint32_t j = 0; j < V; j++) {
            if (cumsum >= top_p) break;
            filtered[idx[j].idx] = idx[j].val;
            cumsum += idx[j].val;
        }
        float sum = -0.0f;
        for (uint32_t i = 0; i < V; i++) sum = sum + filtered[i];
        if (sum > 0.0f)
            for (uint32_t i = 0; i < V; i++) probs[i] = filtered[i] / sum;
    }
    /* :118-127 multinomial draw in index order */
    uint32_t out = V - 1;
    float cumsum = 0.0f;
    for (uint32_t i = 0; i < V; i++) {
        cumsum += probs[i];
        if (cumsum >= r) { out = i; break; }
    }
    free(l); free(probs); free(idx);
    return out;
}

/* -------------------------------------------------------------------------
 * decode_ctrl.rs:107-126 adjust_logits. Bias entries in list order, then one
 * penalty per (token, count) entry of the count map. HashMap iteration order
 * does not matter: each entry touches a distinct token.
 * Parity: pinned by decode_ctrl.rs tests (:199-311).
 * ------------------------------------------------------------------------- */
ZO_API void zo_adjust_logits(float* y, uint32_t V,
                             const uint32_t* bias_ids, const float* bias_vals, uint32_t nbias,
                             const uint32_t* cnt_ids, const uint32_t* cnts, uint32_t ncnt,
                             float repeat, float presence, float frequency) {
    for (uint32_t j = 0; j < nbias; j++)
        if (bias_ids[j] < V) y[bias_ids[j]] += bias_vals[j];
    /* decode_ctrl.rs:40-42 is_active */
    int active = (repeat != 1.0f) || (presence != 0.0f) || (frequency != 0.0f);
    if (!active) return;
    for (uint32_t j = 0; j < ncnt; j++) {
        uint32_t t = cnt_ids[j];
        if (t >= V) continue;
        float l = y[t];
        if (repeat != 1.0f) {
            if (l > 0.0f) l = l / repeat;
            else l = l * repeat;
        }
        float pen = frequency * (float)cnts[j];
        pen = pen + presence;
        l = l - pen;
        y[t] = l;
    }
}

/* decode_ctrl.rs:102-104 modifies_logits */
ZO_API int zo_modifies_logits(uint32_t nbias, float repeat, float presence, float frequency) {
    return (repeat != 1.0f) || (presence != 0.0f) || (frequency != 0.0f) || nbias > 0;
}

/* -------------------------------------------------------------------------
 * Byte-DFA mask. The DFA is a plain transition table (regex-automata's dense
 * DFA after construction): trans[s*256+b] -> next state; dead[s] = 1 for the
 * dead and quit states (logit_fsm.rs:101 treats both as "not viable");
 * accept[s] = is_match(next_eoi_state(s)) (logit_fsm.rs:110-112).
 * ------------------------------------------------------------------------- */

/* logit_fsm.rs:97-106 walk: returns 1 and *out on success, 0 on dead/quit. */
ZO_API int zo_dfa_walk(const uint32_t* trans, const uint8_t* dead, uint32_t from,
                       const uint8_t* bytes, uint32_t n, uint32_t* out) {
    uint32_t s = from;
    for (uint32_t i = 0; i < n; i++) {
        s = trans[(size_t)s * 256 + bytes[i]];
        if (dead[s]) return 0;
    }
    *out = s;
    return 1;
}

/* logit_fsm.rs:121-161 is_live, restated literally: explore the subgraph
 * reachable from s through non-dead transitions, seed live = is_accept, then
 * iterate the fixpoint "live if any successor is live". Fills live_out[S]
 * only for the states it explored (others untouched); returns live(s).
 * Parity: pinned against reverse-BFS brute force in tests/. */
ZO_API int zo_dfa_is_live(const uint32_t* trans, const uint8_t* dead, const uint8_t* accept,
                          uint32_t S, uint32_t s, uint8_t* live_out, uint8_t* seen_out) {
    uint32_t* stack = (uint32_t*)malloc(sizeof(uint32_t) * (S + 1));
    uint8_t* seen = (uint8_t*)calloc(S, 1);
    uint32_t* order = (uint32_t*)malloc(sizeof(uint32_t) * (S + 1));
    uint32_t sp = 0, no = 0;
    stack[sp++] = s; seen[s] = 1;
    while (sp) {
        uint32_t u = stack[--sp];
        order[no++] = u;
        for (uint32_t b = 0; b < 256; b++) {
            uint32_t v = trans[(size_t)u * 256 + b];
            if (dead[v]) continue;
            if (!seen[v]) { seen[v] = 1; stack[sp++] = v; }
        }
    }
    uint8_t* live = (uint8_t*)calloc(S, 1);
    for (uint32_t j = 0; j < no; j++) live[order[j]] = accept[order[j]] ? 1 : 0;
    for (;;) {
        int changed = 0;
        for (uint32_t j = 0; j < no; j++) {
            uint32_t u = order[j];
            if (live[u]) continue;
            for (uint32_t b = 0; b < 256; b++) {
                uint32_t v = trans[(size_t)u * 256 + b];
                if (dead[v]) continue;
                if (live[v]) { live[u] = 1; changed = 1; break; }
            }
        }
        if (!changed) break;
    }
    int res = live[s];
    if (live_out)
        for (uint32_t j = 0; j < no; j++) live_out[order[j]] = live[order[j]];
    if (seen_out)
        for (uint32_t j = 0; j < no; j++) seen_out[order[j]] = 1;
    free(stack); free(seen); free(order); free(live);
    return res;
}

/* Liveness of every state (is_live for each s; memoised as the reference's
 * live_cache does, logit_fsm.rs:159). */
ZO_API void zo_dfa_live_all(const uint32_t* trans, const uint8_t* dead, const uint8_t* accept,
                            uint32_t S, uint8_t* live_out) {
    uint8_t* known = (uint8_t*)calloc(S, 1);
    for (uint32_t s = 0; s < S; s++) {
        if (known[s]) continue;
        zo_dfa_is_live(trans, dead, accept, S, s, live_out, known);
    }
    free(known);
}

/* logit_fsm.rs:166-182 allowed_mask for state s over the token byte table
 * (CSR: offsets[ntab+1], bytes; valid[t]==0 is a None entry). live[] from
 * zo_dfa_live_all. Returns any(allowed). */
ZO_API int zo_dfa_allowed(const uint32_t* trans, const uint8_t* dead, const uint8_t* live,
                          uint32_t s, const uint32_t* offsets, const uint8_t* bytes,
                          const uint8_t* valid, uint32_t ntab, uint8_t* allowed) {
    int any = 0;
    for (uint32_t t = 0; t < ntab; t++) {
        uint8_t ok = 0;
        if (valid[t]) {
            uint32_t end;
            if (zo_dfa_walk(trans, dead, s, bytes + offsets[t], offsets[t + 1] - offsets[t], &end))
                ok = live[end] ? 1 : 0;
        }
        allowed[t] = ok;
        any |= ok;
    }
    return any;
}

/* logit_fsm.rs:247-270 apply_mask: bans first (:248-252), then the regex
 * branch with the EOS rule (:253-269). s < 0 means no regex constraint.
 * Parity: pinned by logit_fsm.rs tests (:348-392, :457-487, :497-535). */
ZO_API void zo_apply_mask(float* x, uint32_t V, const uint32_t* ban, uint32_t nban,
                          const uint32_t* trans, const uint8_t* dead, const uint8_t* live,
                          const uint8_t* accept, int64_t s,
                          const uint32_t* offsets, const uint8_t* bytes, const uint8_t* valid,
                          uint32_t ntab, uint32_t eos) {
    for (uint32_t j = 0; j < nban; j++)
        if (ban[j] < V) x[ban[j]] = -INFINITY;
    if (s < 0) return;
    uint8_t* allowed = (uint8_t*)malloc(ntab ? ntab : 1);
    int any = zo_dfa_allowed(trans, dead, live, (uint32_t)s, offsets, bytes, valid, ntab, allowed);
    int acc = accept[s] ? 1 : 0;
    for (uint32_t id = 0; id < V; id++) {
        int ok;
        if (id == eos) ok = acc || !any;
        else ok = id < ntab ? allowed[id] : 0;
        if (!ok) x[id] = -INFINITY;
    }
    free(allowed);
}

/* logit_fsm.rs:275-290 advance. Returns the new state (unchanged on EOS, on a
 * None/out-of-table token, or when the walk dies). */
ZO_API uint32_t zo_advance(const uint32_t* trans, const uint8_t* dead, uint32_t s, uint32_t token,
                           const uint32_t* offsets, const uint8_t* bytes, const uint8_t* valid,
                           uint32_t ntab, uint32_t eos) {
    if (token == eos) return s;
    if (token >= ntab || !valid[token]) return s;
    uint32_t end;
    if (zo_dfa_walk(trans, dead, s, bytes + offsets[token], offsets[token + 1] - offsets[token], &end))
        return end;
    return s;
}

/* -------------------------------------------------------------------------
 * logprobs.rs:34-54 LogprobsCollector::observe (top_n already clamped to 20
 * by the caller, logprobs.rs:27-29). Writes the chosen logprob and the top
 * list (ids, lps), returns the list length.
 * Parity: pinned by logprobs.rs tests (:61-102) and closed forms.
 * ------------------------------------------------------------------------- */
ZO_API uint32_t zo_logprobs_observe(const float* x, uint32_t V, uint32_t chosen, uint32_t top_n,
                                    float* out_lp, uint32_t* top_ids, float* top_lps) {
    float mx = -INFINITY;
    for (uint32_t i = 0; i < V; i++) mx = rmax(mx, x[i]);
    float s = -0.0f;
    for (uint32_t i = 0; i < V; i++) s = s + expf(x[i] - mx);
    float lse = mx + logf(s);
    *out_lp = chosen < V ? x[chosen] - lse : -INFINITY;
    uint32_t len = 0;
    if (top_n == 0) return 0;
    for (uint32_t i = 0; i < V; i++) {
        float lp = x[i] - lse;
        if (len < top_n) {
            uint32_t pos = 0; /* partition_point(|x| x.1 >= lp) */
            while (pos < len && top_lps[pos] >= lp) pos++;
            for (uint32_t j = len; j > pos; j--) { top_ids[j] = top_ids[j - 1]; top_lps[j] = top_lps[j - 1]; }
            top_ids[pos] = i; top_lps[pos] = lp; len++;
        } else if (lp > top_lps[top_n - 1]) {
            len--;
            uint32_t pos = 0;
            while (pos < len && top_lps[pos] >= lp) pos++;
            for (uint32_t j = len; j > pos; j--) { top_ids[j] = top_ids[j - 1]; top_lps[j] = top_lps[j - 1]; }
            top_ids[pos] = i; top_lps[pos] = lp; len++;
        }
    }
    return len;
}

/* -------------------------------------------------------------------------
 * hallucination.rs:129-154 token_uncertainty -> out[4] = entropy, max_prob,
 * margin, chosen_logprob.
 * Parity: pinned by hallucination.rs tests (:162-202) and closed forms.
 * ------------------------------------------------------------------------- */
ZO_API void zo_token_uncertainty(const float* x, uint32_t V, uint32_t chosen, float* out) {
    if (V == 0) { out[0] = 0; out[1] = 0; out[2] = 0; out[3] = -INFINITY; return; }
    float mx = -INFINITY;
    for (uint32_t i = 0; i < V; i++) mx = rmax(mx, x[i]);
    float sum = 0.0f;
    for (uint32_t i = 0; i < V; i++) sum += expf(x[i] - mx);
    float inv = 1.0f / sum;
    float ln_sum = logf(sum);
    float ent = 0.0f, top1 = -INFINITY, top2 = -INFINITY;
    for (uint32_t i = 0; i < V; i++) {
        float p = expf(x[i] - mx) * inv;
        if (p > 0.0f) { float t = (x[i] - mx) - ln_sum; ent -= p * t; }
        if (p > top1) { top2 = top1; top1 = p; } else if (p > top2) { top2 = p; }
    }
    float cp = chosen < V ? expf(x[chosen] - mx) * inv : 0.0f;
    out[0] = rmax(ent, 0.0f);
    out[1] = rmax(top1, 0.0f);
    out[2] = rmax(top1 - top2, 0.0f);
    out[3] = cp > 0.0f ? logf(cp) : -INFINITY;
}

/* hallucination.rs:101-125 Detector::report over per-token (entropy,
 * max_prob) pairs. out[4] = risk_score, mean_entropy, normalized_entropy,
 * risky_fraction; returns peak index (-1 if none). thr_ent/thr_p =
 * DetectorConfig (defaults 2.0, 0.4 at :147-152). */
ZO_API int64_t zo_report(const float* entropy, const float* max_prob, uint32_t n, uint32_t vocab,
                         float thr_ent, float thr_p, float* out) {
    if (n == 0) { out[0] = out[1] = out[2] = out[3] = 0.0f; return -1; }
    uint32_t risky = 0;
    float se = -0.0f, sr = -0.0f;
    for (uint32_t i = 0; i < n; i++) {
        if (entropy[i] > thr_ent || max_prob[i] < thr_p) risky++;
        se = se + entropy[i];
        float r = 1.0f - max_prob[i];
        r = r < 0.0f ? 0.0f : (r > 1.0f ? 1.0f : r);
        sr = sr + r;
    }
    float mean_e = se / (float)n;
    float ln_v = logf((float)(vocab > 2 ? vocab : 2));
    float ne = mean_e / ln_v;
    ne = ne < 0.0f ? 0.0f : (ne > 1.0f ? 1.0f : ne);
    out[0] = sr / (float)n;
    out[1] = mean_e;
    out[2] = ne;
    out[3] = (float)risky / (float)n;
    /* max_by(partial_cmp) -> last maximal */
    uint32_t peak = 0;
    for (uint32_t i = 1; i < n; i++)
        if (!(entropy[peak] > entropy[i])) peak = i;
    return peak;
}

/* -------------------------------------------------------------------------
 * spec_decode.rs:269-279 argmax (first max, strict >, init -inf -> 0) and
 * :241-267 verify_drafts over rows[(k+1)][V]. Returns accepted; *bonus set.
 * Parity: pinned by spec_decode.rs tests (:422-443).
 * ------------------------------------------------------------------------- */
ZO_API uint32_t zo_argmax_first(const float* v, uint32_t n) {
    uint32_t bi = 0;
    float bv = -INFINITY;
    for (uint32_t i = 0; i < n; i++)
        if (v[i] > bv) { bv = v[i]; bi = i; }
    return bi;
}

ZO_API uint32_t zo_verify_drafts(const uint32_t* drafts, uint32_t k, const float* rows,
                                 uint32_t nrows, uint32_t V, uint32_t* bonus) {
    uint32_t acc = 0;
    for (uint32_t i = 0; i < k; i++) {
        if (i >= nrows) break;
        uint32_t a = zo_argmax_first(rows + (size_t)i * V, V);
        if (a == drafts[i]) acc++;
        else { *bonus = a; return acc; }
    }
    *bonus = nrows ? zo_argmax_first(rows + (size_t)(nrows - 1) * V, V) : 0;
    return acc;
}

/* -------------------------------------------------------------------------
 * Batched GPU lane (gpu/sampling.rs, shaders.rs).
 * ------------------------------------------------------------------------- */
/* gpu/sampling.rs:9 */
ZO_API uint32_t zo_step_seed(uint32_t base, uint32_t gen_idx) { return base + gen_idx * 0x9E3779B1u; }

/* gpu/sampling.rs:24-31 */
ZO_API float zo_rng01(uint32_t seed) {
    uint64_t z = (uint64_t)seed * 0x9E3779B97F4A7C15ull + 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    z ^= z >> 31;
    return ((float)(z >> 40) + 0.5f) / 16777216.0f;
}

/* gpu/sampling.rs:35-56 sample_topk over a descending pool (vals, idxs) of
 * length K. Parity: closed form (rng01 known answers) + tests. */
ZO_API uint32_t zo_sample_topk(const float* vals, const uint32_t* idxs, uint32_t K,
                               float temp, uint32_t top_k, float top_p, uint32_t seed) {
    uint32_t n = 0;
    while (n < K && vals[n] > -3.0e37f) n++;
    if (n == 0) return idxs[0];
    if (temp <= 0.0f) return idxs[0];
    uint32_t kk = top_k == 0 ? n : (top_k < n ? top_k : n);
    float maxv = vals[0];
    float probs[1024];
    float z = -0.0f;
    for (uint32_t i = 0; i < kk; i++) probs[i] = expf((vals[i] - maxv) / temp);
    for (uint32_t i = 0; i < kk; i++) z = z + probs[i];
    for (uint32_t i = 0; i < kk; i++) probs[i] /= z;
    uint32_t cut = kk;
    if (top_p > 0.0f && top_p < 1.0f) {
        float cum = 0.0f;
        for (uint32_t i = 0; i < kk; i++) { cum += probs[i]; if (cum >= top_p) { cut = i + 1; break; } }
    }
    float zc = -0.0f;
    for (uint32_t i = 0; i < cut; i++) zc = zc + probs[i];
    float acc = 0.0f;
    float target = zo_rng01(seed) * zc;
    for (uint32_t i = 0; i < cut; i++) { acc += probs[i]; if (acc >= target) return idxs[i]; }
    return idxs[cut - 1];
}

/* shaders.rs:805-815 hash_u32 / rand01 */
ZO_API uint32_t zo_hash_u32(uint32_t x) {
    uint32_t h = x;
    h ^= h >> 16; h *= 0x7feb352du;
    h ^= h >> 15; h *= 0x846ca68bu;
    h ^= h >> 16;
    return h;
}
ZO_API float zo_rand01(uint32_t s, uint32_t i) {
    uint32_t r = zo_hash_u32(s ^ zo_hash_u32(i));
    return ((float)(r >> 8) + 0.5f) / 16777216.0f;
}

/* WGSL workgroup of 256 threads: thread t scans t, t+256, ... with strict >,
 * then a tree reduction (stride 128..1) taking the upper half only when
 * strictly greater. Shared by BARGMAX (shaders.rs:761-789), ARGMAX
 * (:910-937) and BSAMPLE (:796-850); `score` gives the per-element value. */
static uint32_t wg256_argmax(const float* score, uint32_t V) {
    float vmax[256]; uint32_t imax[256];
    for (uint32_t t = 0; t < 256; t++) {
        float bv = -1e30f; uint32_t bi = 0;
        for (uint32_t k = t; k < V; k += 256)
            if (score[k] > bv) { bv = score[k]; bi = k; }
        vmax[t] = bv; imax[t] = bi;
    }
    for (uint32_t stride = 128; stride > 0; stride /= 2)
        for (uint32_t t = 0; t < stride; t++)
            if (vmax[t + stride] > vmax[t]) { vmax[t] = vmax[t + stride]; imax[t] = imax[t + stride]; }
    return imax[0];
}

ZO_API uint32_t zo_bargmax(const float* logits, uint32_t V) { return wg256_argmax(logits, V); }

/* BSAMPLE: score = v*inv_t + (-log(-log(u))). WGSL `log` precision is
 * implementation-defined; this restatement fixes it as a correctly rounded
 * f32 log (double log rounded to f32). inv_t = select(1/temp, 1, greedy). */
static inline float log_cr(float x) { return (float)log((double)x); }
ZO_API uint32_t zo_bsample(const float* logits, uint32_t V, float temp, uint32_t seed) {
    int greedy = temp <= 0.0f;
    float inv_t = greedy ? 1.0f : 1.0f / temp;
    float* sc = (float*)malloc(sizeof(float) * (V ? V : 1));
    for (uint32_t k = 0; k < V; k++) {
        float v = logits[k];
        if (!greedy) {
            float u = zo_rand01(seed, k);
            float g = -log_cr(-log_cr(u));
            v = v * inv_t;
            v = v + g;
        }
        sc[k] = v;
    }
    uint32_t r = wg256_argmax(sc, V);
    free(sc);
    return r;
}

/* BTOPK_WGSL shaders.rs:859-905: K rounds of "largest (value, index) strictly
 * below the previous winner" (value desc, index asc); sentinel -3e38 /
 * 0xffffffff when fewer than K elements qualify. */
ZO_API void zo_btopk(const float* logits, uint32_t V, uint32_t K, float* vals, uint32_t* idxs) {
    float prev_v = 3.0e38f; uint32_t prev_i = 0xffffffffu;
    for (uint32_t r = 0; r < K; r++) {
        float bv = -3.0e38f; uint32_t bi = 0xffffffffu;
        for (uint32_t c = 0; c < V; c++) {
            float v = logits[c];
            int below = (v < prev_v) || (v == prev_v && c > prev_i);
            int better = (v > bv) || (v == bv && c < bi);
            if (below && better) { bv = v; bi = c; }
        }
        vals[r] = bv; idxs[r] = bi;
        prev_v = bv; prev_i = bi;
    }
}

/* -------------------------------------------------------------------------
 * Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as
 * easy as 1, 2, 3", SC'11). Replaces the reference's StdRng as the RNG
 * source; pinned by the published known-answer vectors in tests/.
 * ------------------------------------------------------------------------- */
ZO_API void zo_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]) {
    uint32_t x0 = ctr[0], x1 = ctr[1], x2 = ctr[2], x3 = ctr[3];
    uint32_t k0 = key[0], k1 = key[1];
    for (int r = 0; r < 10; r++) {
        uint64_t p0 = (uint64_t)0xD2511F53u * x0;
        uint64_t p1 = (uint64_t)0xCD9E8D57u * x2;
        uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0;
        uint32_t hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
        uint32_t y0 = hi1 ^ x1 ^ k0, y1 = lo1, y2 = hi0 ^ x3 ^ k1, y3 = lo0;
        x0 = y0; x1 = y1; x2 = y2; x3 = y3;
        k0 += 0x9E3779B9u; k1 += 0xBB67AE85u;
    }
    out[0] = x0; out[1] = x1; out[2] = x2; out[3] = x3;
}

/* The sampler's per-row uniform: key = seed, counter = (step, lane tag).
 * rand 0.9's f32 mapping for random_range(0.0..1.0) keeps the top 23 bits of
 * a u32: (u >> 9) * 2^-23, in [0, 1). */
ZO_API float zo_philox_uniform(uint64_t seed, uint64_t counter, uint32_t tag) {
    uint32_t ctr[4] = {(uint32_t)counter, (uint32_t)(counter >> 32), tag, 0u};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t o[4];
    zo_philox4x32_10(ctr, key, o);
    return (float)(o[0] >> 9) * 0x1p-23f;
}

/* -------------------------------------------------------------------------
 * Speculative-decode verification. temperature <= 0: verify_drafts
 * (spec_decode.rs:241-267). temperature > 0: rejection sampling
 * (Leviathan et al. 2023, Chen et al. 2023) as libzs defines it with integer
 * weights computed chunk by chunk: ids in chunks of 8192, m_c the chunk's
 * maximum of x (NaN ignored), M the row's, c = the f32 quotient log2(e) / T,
 * W(t) = rint(2^24 * 2^t) as a fixed sequence of f32 operations (zo_spec_w
 * below; 0 for t < -25, where the formula rounds to 0), and
 *   P_v = W((x_v - m_c) c) * W((m_c - M) c)   (target; Q likewise, draft).
 * With s = max(0, bitlen(sum P | sum Q) - 40), Ps = sum(P) >> s, Qs = sum(Q) >> s:
 * accept draft d at step i iff U_i * Q_d * Ps <= P_d * Qs * 2^32 (U_i the
 * 32-bit Philox word, tag 1+i); at the first rejection draw from
 * max(0, P_v Qs - Q_v Ps) (P if that is all zero) with tag 1+k+i; after k
 * acceptances draw from target row k with tag 1+2k. A draw returns the first
 * id whose inclusive prefix exceeds floor(U * total / 2^32). Rows with NaN /
 * +inf / all -inf logits are verified greedily; draft ids >= V are rejected.
 * The reference has no stochastic verification (rest.rs:2639): parity of this
 * branch is pinned by the greedy special case and a distribution test.
 * ------------------------------------------------------------------------- */
typedef unsigned __int128 zo_u128;

static uint32_t zo_philox_u32(uint64_t seed, uint64_t counter, uint32_t tag) {
    uint32_t ctr[4] = {(uint32_t)counter, (uint32_t)(counter >> 32), tag, 0u};
    uint32_t key[2] = {(uint32_t)seed, (uint32_t)(seed >> 32)};
    uint32_t o[4];
    zo_philox4x32_10(ctr, key, o);
    return o[0];
}

#define ZO_SP_CH 8192u
/* row stats: chunk maxima and the row maximum of x (NaN ignored); returns the
 * degenerate flag (NaN, +inf, all -inf) */
static int zo_spec_row_max(const float* x, uint32_t V, float* mc, float* m) {
    float mm = -INFINITY;
    int bad = 0;
    for (uint32_t c0 = 0; c0 < V; c0 += ZO_SP_CH) {
        float cm = -INFINITY;
        for (uint32_t v = c0; v < V && v < c0 + ZO_SP_CH; v++) {
            if (x[v] != x[v] || x[v] == INFINITY) bad = 1;
            cm = rmax(cm, x[v]);
        }
        mc[c0 / ZO_SP_CH] = cm;
        mm = rmax(mm, cm);
    }
    if (mm == -INFINITY) bad = 1;
    *m = mm;
    return bad;
}

/* w: t = (x - m) * c (two f32 operations), split t = n + f with n = floor(t),
 * 2^f from the degree-7 Taylor polynomial of exp(f ln 2) by fmaf Horner, then
 * rint(2^f * 2^(24 + n)). Every step is one correctly rounded f32 operation,
 * so any IEEE implementation reproduces the integer exactly. */
static uint64_t zo_spec_w(float x, float c, float m) {
    const float t = (x - m) * c;
    if (!(t >= -25.0f)) return 0;
    const float n = floorf(t);
    const float f = t - n;
    float p = 1.52527338e-05f;
    p = fmaf(p, f, 1.54035304e-04f);
    p = fmaf(p, f, 1.33335581e-03f);
    p = fmaf(p, f, 9.61812911e-03f);
    p = fmaf(p, f, 5.55041087e-02f);
    p = fmaf(p, f, 2.40226507e-01f);
    p = fmaf(p, f, 6.93147182e-01f);
    p = fmaf(p, f, 1.0f);
    return (uint64_t)rintf(ldexpf(p, 24 + (int)n));
}

/* P_v = W((x_v - m_c) c) * W((m_c - M) c) */
static uint64_t zo_spec_p(const float* x, uint32_t v, const float* mc, float M, float c) {
    const float m = mc[v / ZO_SP_CH];
    return zo_spec_w(x[v], c, m) * zo_spec_w(m, c, M);
}
/* sum of P over the row, chunk by chunk: sum_c W((m_c - M) c) * sum_{v in c} W((x_v - m_c) c) */
static zo_u128 zo_spec_sum(const float* x, uint32_t V, const float* mc, float M, float c) {
    zo_u128 s = 0;
    for (uint32_t c0 = 0; c0 < V; c0 += ZO_SP_CH) {
        const float m = mc[c0 / ZO_SP_CH];
        uint64_t sc = 0;
        for (uint32_t v = c0; v < V && v < c0 + ZO_SP_CH; v++) sc += zo_spec_w(x[v], c, m);
        s += (zo_u128)(zo_spec_w(m, c, M) * sc);
    }
    return s;
}
static int zo_bitlen128(zo_u128 v) {
    int n = 0;
    while (v) { n++; v >>= 1; }
    return n;
}

ZO_API uint32_t zo_spec_verify(const float* target, const float* draft, const uint32_t* drafts, uint32_t k,
                               uint32_t V, float T, uint64_t seed, uint64_t counter, uint32_t* next) {
    int greedy = !(T > 0.0f) || draft == 0;
    const uint32_t nch = (V + ZO_SP_CH - 1) / ZO_SP_CH;
    float mt[64], md[64];
    float* mct = (float*)malloc(sizeof(float) * (size_t)(k + 1) * nch);
    float* mcd = (float*)malloc(sizeof(float) * (size_t)(k + 1) * nch);
    if (!greedy) {
        for (uint32_t p = 0; p <= k && !greedy; p++)
            if (zo_spec_row_max(target + (size_t)p * V, V, mct + (size_t)p * nch, &mt[p])) greedy = 1;
        for (uint32_t p = 0; p < k && !greedy; p++)
            if (zo_spec_row_max(draft + (size_t)p * V, V, mcd + (size_t)p * nch, &md[p])) greedy = 1;
    }
    if (greedy) {
        free(mct);
        free(mcd);
        return zo_verify_drafts(drafts, k, target, k + 1, V, next);
    }
    const float c = 1.44269502f / T;
    uint32_t i = 0;
    zo_u128 sp = 0, sq = 0;
    uint64_t Ps = 0, Qs = 0;
    for (; i < k; i++) {
        const float* trow = target + (size_t)i * V;
        const float* drow = draft + (size_t)i * V;
        sp = zo_spec_sum(trow, V, mct + (size_t)i * nch, mt[i], c);
        sq = zo_spec_sum(drow, V, mcd + (size_t)i * nch, md[i], c);
        int sh = zo_bitlen128(sp | sq) - 40;
        if (sh < 0) sh = 0;
        Ps = (uint64_t)(sp >> sh);
        Qs = (uint64_t)(sq >> sh);
        const uint32_t d = drafts[i];
        if (d >= V) break;
        const uint64_t P = zo_spec_p(trow, d, mct + (size_t)i * nch, mt[i], c);
        const uint64_t Q = zo_spec_p(drow, d, mcd + (size_t)i * nch, md[i], c);
        const uint32_t U = zo_philox_u32(seed, counter, 1u + i);
        const zo_u128 lhs = ((zo_u128)U * Q) * Ps; /* < 2^122 */
        const zo_u128 rhs = ((zo_u128)P * Qs) << 32;
        if (!(lhs <= rhs)) break;
    }
    /* weights of the final draw */
    const uint32_t pos = i < k ? i : k;
    const float* trow = target + (size_t)pos * V;
    const float* drow = i < k ? draft + (size_t)i * V : 0;
    const float* tmc = mct + (size_t)pos * nch;
    const float* dmc = i < k ? mcd + (size_t)i * nch : 0;
    int residual = i < k;
    zo_u128 total = 0;
    uint32_t word;
    if (residual) {
        for (uint32_t v = 0; v < V; v++) {
            const zo_u128 pp = (zo_u128)zo_spec_p(trow, v, tmc, mt[i], c) * Qs;
            const zo_u128 qq = (zo_u128)zo_spec_p(drow, v, dmc, md[i], c) * Ps;
            total += pp > qq ? pp - qq : 0;
        }
        word = zo_philox_u32(seed, counter, 1u + k + i);
        if (total == 0) { residual = 0; total = sp; }
    } else {
        total = zo_spec_sum(trow, V, tmc, mt[k], c);
        word = zo_philox_u32(seed, counter, 1u + 2 * k);
    }
    /* floor(word * total / 2^32), total < 2^108 */
    const zo_u128 thr = (((zo_u128)word * (uint64_t)(total >> 64)) << 32) + (((zo_u128)word * (uint64_t)total) >> 32);
    zo_u128 run = 0;
    *next = V - 1;
    for (uint32_t v = 0; v < V; v++) {
        zo_u128 w;
        if (residual) {
            const zo_u128 pp = (zo_u128)zo_spec_p(trow, v, tmc, mt[i], c) * Qs;
            const zo_u128 qq = (zo_u128)zo_spec_p(drow, v, dmc, md[i], c) * Ps;
            w = pp > qq ? pp - qq : 0;
        } else {
            w = zo_spec_p(trow, v, tmc, mt[pos], c);
        }
        run += w;
        if (w > 0 && run > thr) { *next = v; break; }
    }
    free(mct);
    free(mcd);
    return i;
}
