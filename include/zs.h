/*
 * zs.h -- C ABI of libzs, the MI355X (gfx950) logits post-processing and
 * sampling path that replaces fankh/zllm's per-step sampler and
 * constrained-decoding engine (src/engine/{sampler,decode_ctrl,logit_fsm,
 * logprobs,hallucination,spec_decode}.rs and the batched-lane helpers in
 * src/backend/gpu/{sampling,shaders}.rs).
 *
 * Conventions
 *  - Every entry point returns int status: 0 = ok, < 0 = error (ZS_E*). The
 *    message of the last error is kept per context (zs_last_error). Nothing
 *    aborts or throws across the boundary.
 *  - Pointers named d_* are device memory (hipMalloc'd by the caller) and are
 *    read or written asynchronously on `stream` (a hipStream_t passed as void*;
 *    NULL = the default stream). The caller synchronises. Host pointers (h_*)
 *    are read before the call returns.
 *  - A context is not thread-safe: use one per host thread. zs_ctx_create
 *    sizes all device scratch for (max_rows, max_vocab); zs_sample and
 *    zs_dfa_mask allocate nothing per call.
 *  - Vocab ids are uint32; logits are fp32 rows of width V with row stride ld
 *    (elements, ld >= V, ld % 4 == 0, base 16-byte aligned).
 */
#ifndef ZS_H
#define ZS_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ZS_ABI_VERSION 2   /* 2: zs_batch gained pass_event */

#define ZS_OK 0
#define ZS_EINVAL (-1)   /* bad argument (null pointer, size out of range) */
#define ZS_EHIP (-2)     /* HIP runtime error */
#define ZS_ENOMEM (-3)   /* device allocation failed */
#define ZS_ELIMIT (-4)   /* request exceeds a documented limit */

typedef struct zs_ctx zs_ctx;
typedef struct zs_vocab zs_vocab;
typedef struct zs_dfa zs_dfa;

/* ABI version of the library (compare with ZS_ABI_VERSION). New entry point;
 * the reference has no FFI (docs/PLUGIN_PLAN.md:93-136 sketches a versioned
 * C ABI that was never implemented). */
int zs_abi_version(void);

/* Layout of the ABI's structs as this library was compiled: `which` is one of
 * ZS_LAYOUT_*; writes sizeof into *size and the offset of each field, in
 * declaration order, into offsets[0 .. min(cap, nfields)); returns the number
 * of fields, or ZS_EINVAL for an unknown `which`. A binding (Rust, ctypes)
 * checks its own #[repr(C)] / Structure layout against it once at load time.
 * New entry point; no counterpart in the reference (docs/PLUGIN_PLAN.md:101-131
 * asks for a versioned ABI). */
#define ZS_LAYOUT_BATCH 0
#define ZS_LAYOUT_ROW_PARAMS 1
#define ZS_LAYOUT_SPEC_BATCH 2
#define ZS_LAYOUT_LANE_STREAM 3
#define ZS_LAYOUT_HALLUC_REPORT 4
int zs_struct_layout(int which, size_t* size, size_t* offsets, size_t cap);

/* Context on HIP device `device`, with scratch sized for batches of up to
 * max_rows rows of up to max_vocab logits. */
int zs_ctx_create(int device, uint32_t max_rows, uint32_t max_vocab, zs_ctx** out);
void zs_ctx_destroy(zs_ctx* ctx);
const char* zs_last_error(const zs_ctx* ctx);

/* ---- token byte table -------------------------------------------------
 * Replaces TokenByteTable (src/engine/logit_fsm.rs:43-46): token t has bytes
 * h_bytes[h_offsets[t] .. h_offsets[t+1]); h_valid[t] == 0 marks a None entry
 * (special / non-UTF-8 piece, never allowed under a grammar). ntab entries,
 * `eos` the end-of-sequence id (may be >= ntab, as in the reference tests).
 * Each token is at most 255 bytes. */
int zs_vocab_create(zs_ctx* ctx, const uint32_t* h_offsets, const uint8_t* h_bytes,
                    const uint8_t* h_valid, uint32_t ntab, uint32_t eos, zs_vocab** out);
void zs_vocab_destroy(zs_vocab* vocab);

/* ---- byte DFA ---------------------------------------------------------
 * Replaces RegexEngine (logit_fsm.rs:54-183) over an already-built dense DFA:
 * h_trans[s*256 + b] = next state; h_dead[s] != 0 for the dead and quit
 * states (logit_fsm.rs:101); h_accept[s] != 0 iff the text consumed so far is
 * a complete match, i.e. is_match(next_eoi_state(s)) (logit_fsm.rs:110-112).
 * Liveness (logit_fsm.rs:121-161) is computed here, once, on the host. */
int zs_dfa_create(zs_ctx* ctx, const uint32_t* h_trans, uint32_t nstates, const uint8_t* h_dead,
                  const uint8_t* h_accept, zs_dfa** out);
void zs_dfa_destroy(zs_dfa* dfa);
/* logit_fsm.rs:121 is_live / :110 is_accept for one state (host). */
int zs_dfa_is_live(const zs_dfa* dfa, uint32_t state);
int zs_dfa_is_accept(const zs_dfa* dfa, uint32_t state);
/* logit_fsm.rs:275-290 advance: the state after committing `token` (unchanged
 * for eos, a None/out-of-table token, or a walk into the dead state; *viable
 * is set to 0 in the last case, the reference's warning). Host-side. */
int zs_dfa_advance(const zs_dfa* dfa, const zs_vocab* vocab, uint32_t state, uint32_t token,
                   uint32_t* out_state, int* viable);

/* logit_fsm.rs:247-270 apply_mask (regex branch) + :166-182 allowed_mask,
 * vocab-parallel on the GPU for B rows at once. Row r is at DFA state
 * d_states[r] (int32; < 0 = row unconstrained: all bits set). Writes the
 * packed allow bitset d_out_bits[r*words + w] (bit i of word w = id 32w+i is
 * allowed, words = ceil(V/32)), with the EOS rule applied: eos is allowed iff
 * is_accept(state) or no table token is viable. Ids >= ntab other than eos
 * are disallowed. d_any (optional, uint32[B]) receives any(allowed).
 * Like the reference's per-state cache (logit_fsm.rs:166-182, the HashMap
 * that allowed_mask fills), the DFA keeps a device memo of walked bitsets per
 * state for the last (vocab, V) pair used with it: a row whose state was
 * walked by an earlier call copies the stored bitset, and rows sharing a state
 * in one call share one walk. Calls on one DFA must be ordered on one stream
 * (or synchronised); two calls that overlap on different streams with
 * different vocabularies or V race on the memo. */
int zs_dfa_mask(zs_ctx* ctx, const zs_dfa* dfa, const zs_vocab* vocab, const int32_t* d_states,
                uint32_t B, uint32_t V, uint32_t* d_out_bits, uint32_t* d_any, void* stream);
/* Drops every memoised bitset of the DFA (host only, no GPU work): the next
 * zs_dfa_mask walks all its rows. The reference has no call for this (its
 * cache lives as long as the engine); it is for timing the walk. */
void zs_dfa_memo_clear(zs_dfa* dfa);
/* The form zs_dfa_mask walks the table in (host only): 0 bit-packed rows in
 * LDS, 1 sparse rows in LDS, 2 displaced rows in LDS, 3 none fits the LDS
 * budget (the L2-resident walk). No counterpart in the reference (its DFA
 * walk is on the CPU); for tests and tuning. */
int zs_dfa_table_form(const zs_dfa* dfa);

/* ---- grammar compilers (host only: no context, no GPU) -----------------
 * Replace regex-automata's dense::Builder (logit_fsm.rs:62-88: anchored start,
 * MatchKind::All, minimised, 24 MB limit) and the schema compiler of
 * json_schema.rs. The DFA recognises "the whole text matches the pattern";
 * any DFA of that language yields the reference's masks, EOS rule and
 * advance (liveness is recomputed by zs_dfa_create). Errors go to err
 * (NUL-terminated, truncated to errcap) and return ZS_EINVAL. */
typedef struct zs_grammar zs_grammar;
/* RegexEngine::compile (logit_fsm.rs:62-91): pattern (len bytes, UTF-8) to a
 * host DFA; state 0 is dead, zs_grammar_info gives the start state. Feed
 * zs_grammar_trans / _dead / _accept to zs_dfa_create. */
int zs_regex_compile(const char* pattern, size_t len, zs_grammar** out, char* err, size_t errcap);
void zs_grammar_destroy(zs_grammar* g);
int zs_grammar_info(const zs_grammar* g, uint32_t* nstates, uint32_t* start);
const uint32_t* zs_grammar_trans(const zs_grammar* g);  /* [nstates * 256] */
const uint8_t* zs_grammar_accept(const zs_grammar* g);  /* [nstates] */
const uint8_t* zs_grammar_dead(const zs_grammar* g);    /* [nstates] */
/* json_schema.rs:78-80 schema_to_regex: the schema (JSON text) to an anchored
 * regex. String outputs: *need = length + 1; ZS_ELIMIT (nothing written) when
 * cap is smaller. */
int zs_json_schema_regex(const char* schema, size_t len, char* out, size_t cap, size_t* need, char* err,
                         size_t errcap);
/* json_schema.rs:84-91 any_json_regex(depth) (depth capped at 32; the
 * reference's `json:` mode uses depth 5). */
int zs_any_json_regex(uint32_t depth, char* out, size_t cap, size_t* need);
/* json_schema.rs:99-112 tool_call_envelope_regex over n (name, schema JSON). */
int zs_tool_call_envelope_regex(const char* const* names, const char* const* schemas, uint32_t n,
                                char* out, size_t cap, size_t* need, char* err, size_t errcap);

/* ---- grammar byte table of a real vocabulary (host only) ----------------
 * LlamaTokenizer::token_bytes_table (tokenizer.rs:108-117): per id below
 * get_vocab_size(true), the bytes of decode([id]) with special tokens
 * skipped, or None (valid = 0) when that text is empty or holds U+FFFD. From
 * a tokenizer.json document (len bytes) or from the vocab embedded in a GGUF
 * file (gguf_vocab.rs:75-171, byte-level BPE only). The CSR arrays feed
 * zs_vocab_create; eos is eos_token_id (tokenizer.rs:52-57) or -1. */
typedef struct zs_token_table zs_token_table;
int zs_token_table_from_json(const char* json, size_t len, zs_token_table** out, char* err, size_t errcap);
int zs_token_table_from_gguf(const char* path, zs_token_table** out, char* err, size_t errcap);
int zs_token_table_info(const zs_token_table* t, uint32_t* ntab, uint32_t* nbytes, int64_t* eos);
const uint32_t* zs_token_table_offsets(const zs_token_table* t);  /* [ntab + 1] */
const uint8_t* zs_token_table_bytes(const zs_token_table* t);     /* [nbytes] */
const uint8_t* zs_token_table_valid(const zs_token_table* t);     /* [ntab] */
/* decode([id]) text of every id (U+FFFD pieces and the "" of specials kept),
 * for the logprobs JSON (rest.rs:1714): offsets [ntab + 1] into bytes. */
int zs_token_table_text(const zs_token_table* t, const uint32_t** offsets, const uint8_t** bytes);
void zs_token_table_destroy(zs_token_table* t);

/* ---- OpenAI wire output (host only) ---------------------------------------
 * Detector::report (hallucination.rs:101-125) over per-token entropy /
 * max_prob (zs_sample's d_entropy / d_max_prob), vocab = row width, with the
 * DetectorConfig thresholds (defaults 2.0 and 0.4, hallucination.rs:44-50).
 * peak_token = -1 for an empty report. */
typedef struct zs_halluc_report {
    float risk_score, mean_entropy, normalized_entropy, risky_fraction;
    int64_t peak_token;
    uint64_t n_tokens;
} zs_halluc_report;
int zs_hallucination_report(const float* entropy, const float* max_prob, uint64_t n, uint64_t vocab,
                            float entropy_threshold, float max_prob_threshold, zs_halluc_report* out);
/* hallucination_json (rest.rs:1494-1503); `flagged` = risk_score >=
 * risk_threshold (the server uses 0.5). String outputs as zs_json_schema_regex. */
int zs_hallucination_json(const zs_halluc_report* r, float risk_threshold, char* out, size_t cap, size_t* need);
/* chat_logprobs_json / legacy_logprobs_json (rest.rs:1710-1744) over n
 * generated tokens: ids[i], logprobs[i] (zs_sample's d_token / d_logprob) and
 * top_count[i] alternatives top_ids / top_logprobs [i * top_stride + k]
 * (d_top_n / d_top_ids / d_top_lps), token texts from zs_token_table_text. */
#define ZS_LOGPROBS_CHAT 0
#define ZS_LOGPROBS_LEGACY 1
int zs_logprobs_json(int kind, uint32_t n, const uint32_t* ids, const float* logprobs, const uint32_t* top_count,
                     uint32_t top_stride, const uint32_t* top_ids, const float* top_logprobs,
                     const uint32_t* text_offsets, const uint8_t* text, uint32_t ntext, char* out, size_t cap,
                     size_t* need);

/* ---- sampler ------------------------------------------------------------
 * Per-row knobs: SamplerConfig (sampler.rs:3-22) + PenaltyConfig
 * (decode_ctrl.rs:21-43) + LogprobsCollector::top_n (logprobs.rs:27, clamped
 * to 20). */
typedef struct zs_row_params {
    float temperature;     /* <= 0: greedy (sampler.rs:35) */
    uint32_t top_k;        /* 0 = off */
    float top_p;           /* >= 1 = off */
    float min_p;           /* 0 = off */
    float repeat;          /* 1 = off */
    float presence;        /* 0 = off */
    float frequency;       /* 0 = off */
    uint32_t top_logprobs; /* N alternatives to report, clamped to 20 */
    uint32_t flags;        /* ZS_ROW_* */
    uint32_t pad;
} zs_row_params;

#define ZS_ROW_MASKED 1u       /* apply the row's allow bitset (grammar mask) */
#define ZS_ROW_LOGPROBS 2u     /* logprob of the token + top_logprobs list (logprobs.rs:34-54) */
#define ZS_ROW_UNCERTAINTY 4u  /* entropy / max_prob / margin / chosen_lp (hallucination.rs:129-154) */

/* Output status bits per row (d_status). */
#define ZS_ST_GREEDY 1u        /* temperature <= 0: argmax path */
#define ZS_ST_NONFINITE 2u     /* NaN/+inf/all -inf after adjustment: id V-1 (sampler.rs:127) */
#define ZS_ST_SMALL 4u         /* survivors fit the on-chip exact path */
#define ZS_ST_TOPLP_AMBIG 8u   /* top_logprobs order depends on the last bit of lse */
#define ZS_ST_LIMIT 0x100u     /* reserved (ABI 1 refused rows with over 4096 merged
                                  ban / bias / count entries; every row is served now) */

/* One step over B rows (the decode loop order of rest.rs:2594-2624):
 *   mask (bans, then the allow bitset)  -> x~        (observers see x~)
 *   bias + penalties over the count map -> y         (decode_ctrl.rs:107-126)
 *   sample_with_rng(y, params, r)       -> token     (sampler.rs:31-128)
 *   logprobs(x~, token), token_uncertainty(x~, token)
 * r is the row's Philox4x32-10 uniform for (seed, counter) -- the reference
 * draws it from StdRng; parity is defined with the same r injected.
 * CSR lists are indexed by row: entries off[r] .. off[r+1]. Count-map ids
 * must be distinct within a row; bias entries apply in list order. */
typedef struct zs_batch {
    uint32_t B, V;
    uint64_t ld;
    const float* d_logits;            /* [B][ld] */
    const zs_row_params* d_params;    /* [B] */
    const uint32_t* d_cnt_off;        /* [B+1] count map (token, count) */
    const uint32_t* d_cnt_ids;
    const uint32_t* d_cnt_vals;
    const uint32_t* d_bias_off;       /* [B+1] logit_bias (token, bias) */
    const uint32_t* d_bias_ids;
    const float* d_bias_vals;
    const uint32_t* d_ban_off;        /* [B+1] ban: ids */
    const uint32_t* d_ban_ids;
    const uint32_t* d_allow_bits;     /* [B][allow_words] or NULL */
    uint32_t allow_words;
    uint32_t top_stride;              /* >= max top_logprobs */
    /* Philox key per row. The reference seeds StdRng from the request seed
     * and falls back to the thread RNG when there is none (sampler.rs:26-29,
     * decode_ctrl.rs:73); libzs has no entropy source of its own, so for an
     * unseeded request the caller passes a fresh random 64-bit seed (drawn
     * from the OS entropy source once per request, distinct per row) and
     * keeps it for the request's later steps. Rows sharing a seed and a
     * counter draw the same uniform. */
    const uint64_t* d_seed;           /* [B] */
    const uint64_t* d_counter;        /* [B] step index of the row's request */
    /* outputs */
    uint32_t* d_token;                /* [B] */
    /* observer outputs are written for rows that request them (ZS_ROW_LOGPROBS
     * / ZS_ROW_UNCERTAINTY); other rows get NaN / top_n = 0 */
    float* d_logprob;                 /* [B] ln p(token) (logprobs.rs:37) */
    uint32_t* d_top_ids;              /* [B][top_stride] */
    float* d_top_lps;                 /* [B][top_stride] */
    uint32_t* d_top_n;                /* [B] entries written */
    float* d_entropy;                 /* [B] hallucination.rs:129-154 */
    float* d_max_prob;
    float* d_margin;
    float* d_chosen_lp;               /* [B] token_uncertainty.chosen_logprob */
    uint32_t* d_status;               /* [B] ZS_ST_* */
    /* optional hipEvent_t, recorded on `stream` where the sampler's kernels
     * begin: independent work (draft verification of the same step) made to
     * wait on it runs beside the sampler, on the CUs its per-row workgroups
     * leave idle (rows finish at different times), instead of after it.
     * NULL: no event. */
    void* pass_event;
} zs_batch;

/* The ban, bias and count lists of a row may hold any number of entries (ids
 * >= V are ignored); a bias list may name an id more than once, its entries
 * then add in list order (decode_ctrl.rs:108-112). */

int zs_sample(zs_ctx* ctx, const zs_batch* batch, void* stream);

/* ---- speculative decoding ------------------------------------------------
 * Verification of k draft tokens per row (k <= ZS_SPEC_KMAX). temperature <= 0
 * (or d_draft == NULL) is greedy verification exactly as verify_drafts
 * (spec_decode.rs:241-279): d_accepted = accepted drafts, d_next = the bonus /
 * corrected token. temperature > 0 is rejection sampling against the draft
 * distributions (the reference has none, rest.rs:2639); probabilities are
 * exact integer weights, computed in one read of the logits: with chunks of
 * 8192 ids, chunk maxima m_c, row maximum M, c = log2(e) / T and
 * W(t) = rint(2^24 * 2^t) from a fixed f32 operation sequence (0 below
 * t = -25), P_v = W((x_v - m_c) c) * W((m_c - M) c); the accept test and the
 * residual use the row sums shifted to 40 significant bits. Uniforms are
 * Philox words of (seed, counter, tag) -- tag 1+i for the test of draft i,
 * 1+k+i for the replacement draw at a rejection at i, 1+2k for the bonus
 * draw. Rows are read with 16-byte loads: ld >= V, ld % 4 == 0, both bases
 * 16-byte aligned. */
#define ZS_SPEC_KMAX 16
typedef struct zs_spec_batch {
    uint32_t B, V, k;
    uint64_t ld;
    const float* d_target;          /* [B][k+1][ld] target logits per position */
    const float* d_draft;           /* [B][k][ld] draft logits, or NULL */
    const uint32_t* d_draft_ids;    /* [B][k] */
    const float* d_temperature;     /* [B] */
    const uint64_t* d_seed;         /* [B] */
    const uint64_t* d_counter;      /* [B] */
    uint32_t* d_accepted;           /* [B] */
    uint32_t* d_next;               /* [B] */
    uint32_t flags;                 /* 0 or ZS_SPEC_BACKGROUND */
} zs_spec_batch;
/* ZS_SPEC_BACKGROUND: the chunk statistics and weight sums run as one
 * workgroup per (row, position) and at most one per CU, leaving most of each
 * CU to other work on other streams; slower alone. Results are identical.
 * (No reference counterpart: a scheduling hint of this implementation.) */
#define ZS_SPEC_BACKGROUND 1u
int zs_spec_verify(zs_ctx* ctx, const zs_spec_batch* batch, void* stream);

/* zs_spec_verify without a context and without any allocation: the same
 * kernels and results, with their scratch (per-chunk records and per-row
 * state) in a fixed device array of the library, one per GPU, held until the
 * process ends. No counterpart in the reference: it is for callers that
 * cannot allocate device memory (code under HIP graph capture, serving loops
 * that forbid hipMalloc). Runs on the current device. Limits: B <=
 * ZS_SPEC_STATIC_MAX_ROWS and B * npos * ceil(V / 8192) <=
 * ZS_SPEC_STATIC_MAX_RECORDS (npos = 2k+1 with draft logits, else k+1);
 * beyond them ZS_ELIMIT and nothing runs. Returns ZS_EINVAL for the argument
 * errors zs_spec_verify reports (no error string: there is no context), and
 * ZS_EHIP for a launch failure. Calls that overlap on one GPU (other streams,
 * other host threads) share the array and race: serialise them. */
#define ZS_SPEC_STATIC_MAX_ROWS 4096
#define ZS_SPEC_STATIC_MAX_RECORDS 65536   /* 40 bytes each: 2.5 MiB per GPU */
int zs_spec_verify_static(const zs_spec_batch* batch, void* stream);

/* ---- batched lane (continuous batching, gpu/batch.rs:176-192) --------------
 * Device-side versions of the WGSL sampling kernels with their exact
 * semantics: BARGMAX (shaders.rs:761-789), BSAMPLE Gumbel-max (:796-850; WGSL
 * `log` fixed as the correctly rounded f32 log), BTOPK (:859-905, K <= 1024),
 * and sample_topk over the top-K pool (gpu/sampling.rs:35-56) so the lane needs
 * no readback of candidate pools. */
int zs_lane_argmax(zs_ctx* ctx, const float* d_logits, uint32_t B, uint32_t V, uint64_t ld, uint32_t* d_out,
                   void* stream);
int zs_lane_sample(zs_ctx* ctx, const float* d_logits, uint32_t B, uint32_t V, uint64_t ld,
                   const float* d_temperature, const uint32_t* d_seed, uint32_t* d_out, void* stream);
int zs_lane_topk(zs_ctx* ctx, const float* d_logits, uint32_t B, uint32_t V, uint64_t ld, uint32_t K,
                 float* d_vals, uint32_t* d_idxs, void* stream);
int zs_lane_sample_topk(zs_ctx* ctx, const float* d_vals, const uint32_t* d_idxs, uint32_t B, uint32_t K,
                        const float* d_temperature, const uint32_t* d_top_k, const float* d_top_p,
                        const uint32_t* d_seed, uint32_t* d_out, void* stream);
/* gpu/sampling.rs:9 step_seed: base + gen_idx * 0x9E3779B1 (wrapping). */
uint32_t zs_step_seed(uint32_t base, uint32_t gen_idx);

/* One active stream of the continuous batcher: SamplingParams
 * (gpu/sampling.rs:14-21; temp <= 0 greedy, top_k 0 = none, top_p >= 1 or 0 =
 * none) and its seeding (base seed, tokens generated so far). */
typedef struct zs_lane_stream {
    float temp;
    uint32_t top_k;
    float top_p;
    uint32_t base_seed;
    uint32_t gen_index;
} zs_lane_stream;
#define ZS_LANE_ARGMAX 0
#define ZS_LANE_SAMPLE 1
#define ZS_LANE_TOPK 2
/* ContinuousBatcher::step's selection (gpu/batch.rs:176-192) for m streams
 * over d_logits[m][ld]: the cheapest path serving every stream -- top-64
 * pool + nucleus draw (step_slotted_topk, gpu/mod.rs:2213-2229) if any stream
 * needs top-k / top-p, else Gumbel temperature sampling (BSAMPLE) if any temp
 * > 0, else argmax (BARGMAX) -- with seeds step_seed(base_seed, gen_index),
 * all on the device: writes d_out[m], reads nothing back (the reference reads
 * m x 64 candidates back and samples on the CPU). h_streams is read before the
 * call returns; *path (optional) receives the ZS_LANE_* path taken. Calls on
 * one context must be issued in order on one stream. m <= max_rows. */
int zs_lane_step(zs_ctx* ctx, const float* d_logits, uint32_t m, uint32_t V, uint64_t ld,
                 const zs_lane_stream* h_streams, uint32_t* d_out, int* path, void* stream);

/* ---- profiling ----------------------------------------------------------
 * When enabled, zs_sample and zs_spec_verify record a HIP event around their
 * kernel launches (no synchronisation is added; zs_sample then runs every
 * kernel on the caller's stream). zs_last_timings waits for the last calls'
 * events and writes up to `cap` kernel names / durations (ms), zs_sample's
 * first; returns the number written. Stands in for the reference's
 * in-process timing (Cargo feature `profile`, Cargo.toml:121-126). */
int zs_set_profiling(zs_ctx* ctx, int on);
int zs_last_timings(zs_ctx* ctx, const char** names, float* ms, int cap);

#ifdef __cplusplus
}
#endif
#endif
