// zs_internal.h -- context and scratch layout shared by the host code and the
// HIP kernels of libzs.
#pragma once
#include <stdint.h>
#include "../../include/zs.h"

// Chunks of 8192 ids: the granularity of per-row scratch records (kept-set
// counts, draft-verification and batched-lane chunk records).
#define ZS_P1_CH 8192
// Largest top-k the row kernel selects by its sorted candidate list (above
// it the big-row engine selects the threshold).
#define ZS_KS 128
// Largest vocabulary a context accepts (the row kernel's patch bitmap and
// the per-row chunk records are sized for it).
#define ZS_MAX_VOCAB 262144
#define ZS_DFA_LDS_BYTES 138544  // packed DFA table budget in LDS (135.3 KB)
#define ZS_DFA_MEMO_BYTES (256ull << 20)  // per-DFA device memo of allow bitsets (cap)
#define ZS_WALK_TILE 2048        // ids per tile of the vocab-parallel DFA walk
#define ZS_DFA_MAXROWS 1024      // rows of the LDS-table DFA walk (constrained-row list in LDS)
#define ZS_DFA_RD_ROWS ZS_DFA_MAXROWS  // displaced rows: per-row u16 bases at the end of the table budget
#define ZS_MAX_CHUNKS (ZS_MAX_VOCAB / ZS_P1_CH)
// Big-row engine: 1024 threads, 4 consecutive elements per thread.
#define ZS_BIG_NT 1024
#define ZS_BIG_G 4096
#define ZS_SORT_CAP 8192
// top-K pool of the batched lane (gpu/mod.rs:1846 TOPK_K)
#define ZS_LANE_K 64

// Patch flags (merged bias / count-map / ban list, one entry per token id).
#define ZS_PF_BAN 1u
#define ZS_PF_Y 2u

// Chunk-stat flags.
#define ZS_CF_OBS_NAN 1u
#define ZS_CF_Z_NAN 2u
#define ZS_CF_Z_PINF 4u
#define ZS_CF_OBS_PINF 8u


// Sub-chunks of 1024 logits: the unit of the parallel exact-sum rounds.
// Sub-chunk j of pass-1 chunk c is the j-th float4 of every pass-1 thread.
#define ZS_SUB 1024
#define ZS_SUBS_PER_CHUNK (ZS_P1_CH / ZS_SUB)
#define ZS_MAX_SUBS (ZS_MAX_VOCAB / ZS_SUB)


// Sums reproduced by the rounds.
#define ZS_SUM_OBS_S 0
#define ZS_SUM_SAMP_S 1
#define ZS_SUM_OBS_H 2
#define ZS_NSUM 3

// Per (row, sum, sub-chunk): predicted grid exponent of the running sum at the
// sub-chunk start and the sub-chunk's total increment on that grid.
#define ZS_SF_FRAGILE 1u  // prediction unsafe (binade crossing nearby): process exactly
#define ZS_SF_TIE 2u      // an exact half-way term met: process exactly
#define ZS_SF_DONE 4u     // total valid
struct zs_sub_sum {
    int32_t eg;
    uint32_t flags;
    uint32_t total;
    uint32_t pad;
};

// Row modes decided by the row kernel.
#define ZS_MODE_DONE 1u   // token final (greedy / non-finite / small path)
#define ZS_MODE_BIG 2u    // big-row engine must run

#define ZS_OBS_CAND 28
#define ZS_ROW_PART 560   // u64 per (row, half) slot of a split row in zs_k_row

// Observer needs (zs_row_state.obs_need).
#define ZS_OBS_S 1u   // exact sequential sum S = sum exp(x~ - max)
#define ZS_OBS_H 2u   // exact sequential entropy sum

struct zs_row_state {
    float z_max;
    uint32_t thr_key;     // top-k threshold key (total order), valid if has_thr
    uint32_t has_thr;     // 0: no top-k; 1: thr_key valid; 2: big engine must select it
    uint32_t mode;
    uint32_t token;
    uint32_t status;
    // observers over x~
    float obs_max;
    uint32_t obs_special; // lse is NaN (NaN / +inf / all -inf row)
    uint32_t obs_need;
    uint32_t rounds;      // ZS_SUM_* bits: the sums zs_sums.hip computes for the row
    uint32_t g_n;         // masked rows: allowed ids gathered to row scratch (0: none, the sums read the row)
    float samp_S;         // sampler softmax denominator (sampler.rs:68) when computed by the rounds
    float obs_S;          // sequential f32 sum (hallucination.rs:134-135, logprobs.rs:36)
    float obs_H;          // sequential f32 entropy (hallucination.rs:139-144)
    // big rows: the kept set (top-p cut, or every positive p1) compacted in index
    // order, whose sum and draw run as parallel rounds (zs_k_roundK / zs_k_stitchK)
    uint32_t klist;       // 1: list ready
    uint32_t nk;          // list length
    uint32_t vstar, istar;  // kept: p > v*, or p == v* and id <= i*
    uint32_t kpend;       // 1: the kept list is compacted by zs_k_kcount / zs_k_kwrite
    uint32_t kident;      // 1: the kept list is the row's p in index order (every positive p, no
                          //    min-p; its zeros add nothing): zs_k_kcount only sums its sub-chunks
    uint32_t krank;       // rank of the top-p stop among the values equal to v*
    uint32_t kminp;       // min-p applies: p1 = p < kcut ? 0 : p / kkept
    uint32_t knorm;       // 1: the draw runs on p1 / sum2 (top-p renormalisation); 0: on p1 (no sum2)
    float kcut, kkept;
    float sum2;           // sequential sum of the kept set (sampler.rs:107)
    uint32_t n_cand;      // observer candidates by (x~ desc, id asc)
    uint32_t cand_id[ZS_OBS_CAND];
    float cand_x[ZS_OBS_CAND];
};

// Top-p walk on bucket totals: the probabilities of a row bucketed by their
// 13 high bits (rank 0 = the largest values). Per bucket: element count,
// approximate mass, start / gather cursor in the row's bucket layout, the
// predicted grid exponent of the running sum and flags (meta), and the total
// integer increment of its elements on that grid.
#define ZS_TP_NB 2048
#define ZS_TP_CAND 64
#define ZS_TP_CL (2 + ZS_TP_CAND)
struct zs_tp_bucket {
    uint32_t cnt;
    float mass;
    uint32_t start, cur, meta, pad;
    unsigned long long tot;
};

// Speculative-decode verification scratch (zs_spec.hip).
#define ZS_SPEC_KMAX 16
struct zs_spec_chunk {
    float xmax;           // chunk maximum of x (NaN ignored)
    uint32_t flags;
    float amax_val;
    uint32_t amax_idx;
    unsigned long long wsum;      // sum of the weights relative to the chunk maximum
    unsigned long long rlo, rhi;  // residual weight sum (position slot 0 of a row)
};
struct zs_spec_row {
    uint32_t mode, pos, residual, word;
    float m_t, m_d;                     // row maxima of the draw's target / draft positions
    unsigned long long ps, qs;          // their weight sums shifted to 40 bits (residual draw)
    unsigned long long sum_lo, sum_hi;  // the target's weight sum (draw from P)
};

struct zs_spec_args {
    uint32_t B, V, k;
    uint64_t ld;
    const float* target;        // [B][k+1][ld]
    const float* draft;         // [B][k][ld] or null
    const uint32_t* draft_ids;  // [B][k]
    const float* temperature;   // [B]
    const uint64_t* seed;
    const uint64_t* counter;
    uint32_t* accepted;
    uint32_t* next;
    zs_spec_chunk* cst;         // scratch [B][npos_max][nch]
    zs_spec_row* rs;            // scratch [B]
    uint32_t nch, npos_max;
    uint32_t background;        // ZS_SPEC_BACKGROUND: the fused one-workgroup-per-CU passes
};

struct zs_ctx {
    int device;
    uint32_t num_cus;
    uint32_t max_rows, max_vocab, max_chunks;
    char err[512];
    // device scratch
    uint32_t* p_cnt;
    uint32_t* p_id;
    uint32_t* p_flags;
    float* p_y;
    zs_row_state* rst;
    uint32_t* pairs;       // big-row gather area [rows][max_vocab][2]
    uint32_t* pv;          // big-row probabilities (f32 bits) [rows][max_vocab]
    void* mask_scratch;    // DFA mask viability flags [rows]
    uint32_t mask_epoch;   // last epoch handed to the packed DFA mask
    double* k_ap;                // [rows][max_subs] approximate sums of the kept list per sub-chunk
    zs_sub_sum* k_sum;           // [3][rows][2][max_subs] kept-list rounds (sum2, draw), then crossing records
    zs_sub_sum* s_rec;           // [3][rows][ZS_NSUM][max_subs] row-sum sub-chunk records (zs_k_sround), then crossing records
    float* gath;                 // [rows][2 * max_vocab + 16] masked rows' gathered allowed ids (x~, y, ids)
    float* s_hterm;              // [rows][max_vocab + 8] exact terms of the side-stream sums (S_obs, then entropy)
    float* s_apx;                // [rows][max_subs][8] approximate row-sum parts per sub-chunk (zs_k_sapx)
    zs_tp_bucket* tp_bk;         // [rows][ZS_TP_NB] top-p buckets (zs_k_tp_*)
    uint32_t* tp_cl;             // [rows][ZS_TP_CL] row flags, candidate count, candidate buckets
    uint32_t* tp_pre;            // [rows][2][max_vocab] increment prefixes of presorted buckets
    uint32_t* kcnt;              // [rows][2 * max_chunks] kept-set counts per 4096-id group
    unsigned long long* rw_part; // [rows][2][ZS_ROW_PART] the two halves of a split row (zs_k_row)
    uint32_t* rw_ctr;            // [rows] halves finished (0 between calls)
    uint32_t* tp_task;           // [1 + rows * ZS_TP_CAND] buckets to presort: count, then (row << 8 | candidate)
    uint32_t* p_sub;             // [rows][max_subs+1] patch index range per sub-chunk
    uint32_t max_subs;
    zs_spec_chunk* spec_chunks;  // [rows][2*ZS_SPEC_KMAX+1][max_chunks]
    zs_spec_row* spec_rows;      // [rows]
    // side stream for the observers' entropy chain, which runs beside the big
    // rows (fork / join by events on the caller's stream; default priority)
    void* side_stream;     // hipStream_t
    void* fork_event;      // hipEvent_t
    void* join_event;      // hipEvent_t
    // profiling (zs_set_profiling)
    int profiling;
    int n_timed;
    void* events[24];      // hipEvent_t
    const char* timed_names[24];
    // batched lane (zs_lane_step): per-stream knobs staged through pinned
    // host memory, top-K pool of every stream
    float* lane_temp;            // [4][rows] block: temp, then top_k, top_p, seed (below point into it)
    uint32_t* lane_topk;         // [rows]
    float* lane_topp;            // [rows]
    uint32_t* lane_seed;         // [rows]
    float* lane_vals;            // [rows][ZS_LANE_K]
    uint32_t* lane_idxs;         // [rows][ZS_LANE_K]
    unsigned long long* lane_ck; // [rows][chunks][ZS_LANE_K] chunk top-K lists (two-phase BTOPK)
    uint32_t* lane_cn;           // [rows][chunks]
    uint32_t* lane_ih;           // [max_vocab + 4] hash of every id (the id half of BSAMPLE's uniforms)
    unsigned long long* lane_keys;  // [rows] BSAMPLE's per-row best key (zero between calls)
    uint32_t* lane_host;         // pinned [2][4][rows]: temp, top_k, top_p, seed (two areas, alternating)
    void* lane_event[2];         // hipEvent_t: the staging copy from each area done
    uint32_t lane_slot;          // the area the next call fills
    int n_spec_timed;      // the same for the last zs_spec_verify call
    void* spec_events[8];
    const char* spec_names[8];
};

struct zs_vocab {
    zs_ctx* ctx;
    uint32_t serial;       // unique per context: keys the DFA memo
    uint32_t ntab, eos, nbytes;
    uint32_t* d_offsets;   // [ntab+1]
    uint8_t* d_bytes;
    uint8_t* d_valid;
    uint32_t* d_packed;    // per token: (offset << 8) | len, len==0xff... see zs_dfa.hip
    uint32_t maxlen;
    // walk order: inside every tile of ZS_WALK_TILE ids, the ids sorted by byte
    // length, with their first 16 bytes and (id | walk length << 18); 0xffffffff
    // marks a slot with no token, length 0 a token that is never allowed and
    // length 0x3fff a valid token with no bytes
    uint32_t nwtile;
    uint32_t* d_wbytes;    // [nwtile * ZS_WALK_TILE][4]
    uint32_t* d_wmeta;     // [nwtile * ZS_WALK_TILE]
    // host copies for advance()
    uint32_t* h_offsets;
    uint8_t* h_bytes;
    uint8_t* h_valid;
};

struct zs_dfa {
    zs_ctx* ctx;
    uint32_t nstates;
    uint32_t ncls;         // byte classes of the folded table
    uint32_t* h_trans;     // [nstates*256] as given
    uint8_t* h_dead;
    uint8_t* h_accept;
    uint8_t* h_live;
    // device: class-compressed table with dead / quit / non-live targets
    // folded into the sentinel 0xffff (see zs_dfa.hip)
    uint16_t* d_trans;     // [nstates][ncls]
    uint8_t* d_cls;        // [256] byte -> class
    uint8_t* d_bad;        // [nstates] dead or not live
    uint8_t* d_accept;     // [nstates]
    // bit-packed table for the LDS walk: good states renumbered 0..ngood-1 and
    // a sink row ngood (the fail value), entries of `bits` bits back to back,
    // state s / class c at bit s * rw + c * bits; rw = ncls * bits rounded up to 32
    uint32_t* d_packed;    // [packed_words]
    uint16_t* d_clsinfo;   // [256] class * bits
    uint16_t* d_remap;     // [nstates] good id or 0xffff
    uint32_t ngood, bits, rw, packed_words;
    int packed_lds;        // the packed table fits the LDS budget
    // sparse form instead (tables past the budget with at most 64 classes):
    // d_packed = {mask lo, mask hi, first target, 0} per good state + sink,
    // then u16 targets; d_clsinfo = class index
    // sparse == 2, displaced rows (tables past the budget): d_packed =
    // packed_words entries b_g + c -> b_g << 16 | b_target (0xffffffff: none),
    // then (not staged in LDS) the u16 base of every state by its original id,
    // rd_fail for bad states; d_clsinfo = class index
    uint32_t sparse;
    uint32_t rd_fail;
    uint32_t dense;        // over 30% of (good state, byte) transitions reach a good state
    // memo of allow bitsets per good state (logit_fsm.rs:166-182's cache):
    // slot g holds the walk's bitset for good state g (before the EOS rule)
    // and d_memo_any[g] = a token is viable; it is valid when
    // d_memo_key[g] == memo_tag << 32 | seq with seq not the current call's
    // (the EOS kernel fills the key after the walk; a slot is used from the
    // next call on, so every workgroup of a walk builds the same plan). The tag
    // is bumped when the vocabulary or V changes (or on zs_dfa_memo_clear),
    // which invalidates every slot at once.
    uint32_t* d_memo;                 // [memo_slots][memo_words]
    unsigned long long* d_memo_key;   // [memo_slots]
    uint32_t* d_memo_any;             // [memo_slots]
    uint32_t memo_slots, memo_words;
    mutable uint32_t memo_tag, memo_seq, memo_serial, memo_V;
    // for the vocabulary memo_serial: every good state's viability known
    // without the walk (all_quick), and that viability per good state
    mutable uint32_t all_quick;
    uint8_t* h_viable;                // [ngood]
    uint16_t* h_remap;                // [nstates] good id or 0xffff (host copy)
    uint8_t* d_viable;                // [ngood]
};

// Arguments of the DFA mask kernels (zs_dfa.hip).
struct dm_args {
    const uint16_t* trans;    // [nstates][ncls], DM_SENT = fail
    const uint8_t* cls;       // [256]
    const uint8_t* bad_start; // [nstates] 1 = start state can allow nothing
    const uint8_t* accept;    // [nstates]
    const uint32_t* tok16;    // [ntab][4] first 16 bytes
    const uint8_t* tlen;      // [ntab] length, 255 = longer than 254 (use CSR)
    const uint32_t* offsets;  // CSR for long tokens
    const uint8_t* bytes;
    const uint8_t* valid;
    uint32_t ntab, eos, nstates, ncls;
    const uint32_t* packed;
    uint32_t packed_words;
    const uint32_t* wbytes;
    const uint32_t* wmeta;
    uint32_t nwtile;
    const uint16_t* clsinfo;
    const uint16_t* remap;
    uint32_t ngood, bits, rw;
    uint32_t sparse;          // packed table in the sparse row form (1) or displaced rows (2)
    uint32_t rd_fail;         // displaced rows: the fail value (a base no state owns)
    const uint16_t* rdmap;    // displaced rows: [nstates] base of each state (rd_fail: bad)
    uint32_t dense;           // most (good state, byte) pairs lead to a good state
    const int32_t* states;
    uint32_t B, V, words;
    uint32_t* out;
    uint32_t* any;
    // packed path: viability flags hold the call's epoch (no clearing pass);
    // the EOS kernel writes the caller's 0/1 flags (any_user, optional)
    uint32_t epoch;
    uint32_t* any_user;
    // memo (packed path; memo_slots = 0 disables it): a constrained row whose
    // good state g < memo_slots has a valid slot copies it; the others are
    // walked, once per distinct state, and fill their slot
    uint32_t* memo;
    unsigned long long* memo_key;
    uint32_t* memo_any;
    uint32_t memo_slots, memo_words, memo_tag, memo_seq;
    // the viability of every good state is known without the walk
    // (viable[g], 0/1): the walk applies the EOS rule itself
    uint32_t eos_direct;
    const uint8_t* viable;
};

// Optional per-kernel event timing of a launch sequence (zs_set_profiling).
struct zs_prof {
    int on;
    void** events;       // hipEvent_t[n + 1]
    const char** names;
    int* n;
};

// Error helper (host).
int zs_set_error(zs_ctx* ctx, int code, const char* fmt, ...);
