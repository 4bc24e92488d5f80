// zs_dfa.hip -- vocab-parallel byte-DFA walk producing packed allow bitsets.
//
// Reference: logit_fsm.rs:97-106 (walk), :121-161 (is_live), :166-182
// (allowed_mask), :247-270 (apply_mask, EOS rule). A token is allowed from state
// s iff it has bytes, its walk never enters the dead/quit state, and it ends in a
// live state. Non-live states can never reach a live state again, so the host
// folds dead, quit and non-live states into one sentinel id: the walk fails as
// soon as it touches the sentinel, and a completed walk is always live.
//
// The transition table is byte-class compressed on the host (bytes with
// identical columns share a class). When nstates * nclasses u16 entries fit in
// LDS, every workgroup stages the table once and walks 2048 tokens for a slice
// of rows; otherwise the walk reads the table through L2.
#include <hip/hip_runtime.h>
#include "zs_internal.h"
#include "zs_dev.h"

#define DM_NT 256
#define DM_TPT 8                 // tokens per thread
#define DM_TOK (DM_NT * DM_TPT)  // tokens per workgroup
#define DM_ROWS 16               // rows per workgroup
#define DM_LDS_ENTRIES 32768     // u16 entries staged in LDS (64 KB)
#define DM_SENT 0xffffu


template <bool LDS>
__global__ __launch_bounds__(DM_NT) void zs_k_dfa_mask(dm_args a) {
    __shared__ uint16_t tab[LDS ? DM_LDS_ENTRIES : 1];
    __shared__ uint8_t cls[256];
    const int t = threadIdx.x;
    const uint32_t tok0 = blockIdx.x * DM_TOK;
    const uint32_t r0 = blockIdx.y * DM_ROWS;
    const uint32_t ncover = a.V > a.ntab ? a.V : a.ntab;
    if (tok0 >= ncover) return;
    for (int i = t; i < 256; i += DM_NT) cls[i] = a.cls[i];
    if (LDS) {
        const uint32_t n = a.nstates * a.ncls;
        for (uint32_t i = t; i < n; i += DM_NT) tab[i] = a.trans[i];
    }
    __syncthreads();
    const uint16_t* T = LDS ? tab : a.trans;
    // tokens: thread t owns ids tok0 + j*DM_NT + t (consecutive ids per wave)
    uint32_t w[DM_TPT][4];
    uint32_t len[DM_TPT];
#pragma unroll
    for (int j = 0; j < DM_TPT; j++) {
        uint32_t id = tok0 + j * DM_NT + t;
        len[j] = 0;
        w[j][0] = w[j][1] = w[j][2] = w[j][3] = 0;
        if (id < a.ntab && a.valid[id]) {
            len[j] = a.tlen[id];
            uint4 v = reinterpret_cast<const uint4*>(a.tok16)[id];
            w[j][0] = v.x; w[j][1] = v.y; w[j][2] = v.z; w[j][3] = v.w;
        } else {
            len[j] = 0xffffffffu;  // never allowed
        }
    }
    const uint32_t rend = min(a.B, r0 + DM_ROWS);
    for (uint32_t r = r0; r < rend; r++) {
        const int32_t st = a.states[r];
        uint32_t anyv = 0;
#pragma unroll
        for (int j = 0; j < DM_TPT; j++) {
            uint32_t id = tok0 + j * DM_NT + t;
            bool ok;
            if (st < 0) {
                ok = id < a.V;  // unconstrained row
            } else if (id >= a.ntab || len[j] == 0xffffffffu || a.bad_start[st]) {
                ok = false;
            } else {
                uint32_t s = (uint32_t)st;
                ok = true;
                uint32_t L = len[j];
                if (L <= 16) {
#pragma unroll
                    for (int i = 0; i < 16; i++) {
                        if ((uint32_t)i >= L) break;
                        uint32_t by = (w[j][i >> 2] >> (8 * (i & 3))) & 0xffu;
                        s = T[s * a.ncls + cls[by]];
                        if (s == DM_SENT) { ok = false; break; }
                    }
                } else {
                    const uint32_t o0 = a.offsets[id], o1 = a.offsets[id + 1];
                    for (uint32_t i = o0; i < o1; i++) {
                        s = T[s * a.ncls + cls[a.bytes[i]]];
                        if (s == DM_SENT) { ok = false; break; }
                    }
                }
            }
            if (st >= 0 && ok) anyv = 1;
            unsigned long long bal = __ballot(ok && id < a.V);
            // wave covers ids tok0 + j*DM_NT + 64*wid .. +63 -> two words
            uint32_t idw = tok0 + j * DM_NT + (t & ~63);
            if (zs_lane() == 0 && idw < a.V) {
                uint32_t wd = idw >> 5;
                uint32_t* o = a.out + (size_t)r * a.words;
                o[wd] = (uint32_t)bal;
                if (wd + 1 < a.words) o[wd + 1] = (uint32_t)(bal >> 32);
            }
        }
        if (st >= 0) {
            anyv = wave_or_u(anyv);
            if (zs_lane() == 0 && anyv) a.any[r] = a.epoch ? a.epoch : 1u;  // same value from every writer
        }
    }
}

// Persistent walk over the table staged in LDS, with the per-state memo. The
// table is in one of three forms: bit-packed rows (good states only,
// `bits`-bit entries, ngood = fail), sparse rows (a class mask per state and
// its targets, for tables past the budget with at most 64 classes) or
// displaced rows (every state is its base in one array of owner << 16 |
// target entries: one 32-bit read and a compare per step; the first choice for
// tables past the budget, since it reads a quarter of the sparse form's bytes
// per step and leaves the step one read deep). One workgroup per CU
// stages the table in LDS once and plans the call (every workgroup builds the
// same plan): each constrained row is either a memo hit (its state's slot is
// valid) or a walk, and rows sharing a state share one walk, whose result
// goes to all of them and to the state's memo slot. The walks are taken as
// items: a tile of ZS_WALK_TILE ids times a group of up to rg (<= 48)
// distinct states. Per item the workgroup first tabulates, for every byte,
// which of the item's states survive that byte as a first byte (one bit per
// state); a token reads its first byte's word and walks its remaining bytes
// only from the states whose bits are set, which is a small fraction of the
// pairs. Inside a tile the tokens come in length order (the vocabulary's walk
// order), so the lanes of a wave walk tokens of nearly equal length; allowed
// ids are set in an LDS bitmap of the tile and written out as whole words.
// Memo hits and unconstrained rows are written last, their words split over
// the workgroups.
#define DL_NT 1024
#define DL_TPT (ZS_WALK_TILE / DL_NT)
#define DL_RG 48                  // distinct states per item (bits of a first-byte word)
#define DL_TW (ZS_WALK_TILE / 32) // bitmap words per state and tile
#define DL_FREE 0xffffu           // row modes: unconstrained
#define DL_WALKED 0xfffcu         //            walked in this call, | 1: eos allowed (else: its memo slot)
#define DL_EMPTY 0x3fffu          // walk length of a valid token with no bytes

// Workgroup barrier that orders LDS accesses only (__syncthreads() would also
// wait for the next item's token loads, issued ahead on purpose)
__device__ __forceinline__ void dl_bar() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}
#define DL_WORDS (ZS_DFA_LDS_BYTES / 4)
#define DL_MAXROWS ZS_DFA_MAXROWS
#define DL_HASH (2 * DL_MAXROWS)  // plan hash table (state -> first row)
static_assert(DL_HASH <= DL_RG * DL_TW, "the plan's hash table lives in the bitmap");
static_assert(DL_MAXROWS <= DL_NT, "one row per thread in the plan");

__device__ __forceinline__ uint32_t dl_hash(uint32_t g) { return (g * 2654435761u) >> (32 - 11); }
static_assert(DL_HASH == 2048, "dl_hash yields 11 bits");

// SIDE states per token walked side by side, TG tokens together: 4 x 2 when
// few states survive a first byte, 8 x 1 for dense automata. FMT: 0
// bit-packed rows, 1 sparse rows, 2 displaced rows.
template <int FMT, int SIDE, int TG>
__global__ __launch_bounds__(DL_NT) void zs_k_dfa_mask_packed(dm_args a) {
    __shared__ uint32_t tab[DL_WORDS];
    __shared__ uint16_t ci[256];
    __shared__ uint32_t bm[DL_RG][DL_TW];   // the plan's hash table first
    __shared__ unsigned long long fb[256];  // per byte: the item's states alive after it
    __shared__ uint32_t wl[DL_MAXROWS];     // walks: good state << 16 | first row
    __shared__ uint32_t link[DL_MAXROWS];   // row -> next row of its state (0xffff: end)
    __shared__ uint32_t s0r[DL_RG + 1];     // the item's start states (packed ids); [DL_RG] = fail
    __shared__ uint16_t rmode[DL_MAXROWS];  // row: memo slot (hit), DL_WALKED or DL_FREE
    __shared__ uint32_t nwl;
    const int t = threadIdx.x;
    const uint32_t r = (uint32_t)t;
    const int32_t st = r < a.B ? a.states[r] : -1;   // issued before the table loads
    // stage the table with many 16-byte loads in flight per thread
    const uint32_t nq = a.packed_words / 4;  // the table is allocated in whole quads
    const uint4* src = reinterpret_cast<const uint4*>(a.packed);
    uint4* dst = reinterpret_cast<uint4*>(tab);
    uint32_t q0 = 0;
    for (; q0 + 8 * DL_NT <= nq; q0 += 8 * DL_NT) {
        uint4 v[8];
#pragma unroll
        for (int u = 0; u < 8; u++) v[u] = src[q0 + u * DL_NT + t];
#pragma unroll
        for (int u = 0; u < 8; u++) dst[q0 + u * DL_NT + t] = v[u];
    }
    for (uint32_t q = q0 + t; q < nq; q += DL_NT) dst[q] = src[q];
    for (int i = t; i < 256; i += DL_NT) ci[i] = a.clsinfo[i];
    // ---- plan: row t (B <= DL_MAXROWS <= DL_NT)
    uint32_t* hs = &bm[0][0];
    for (int i = t; i < DL_HASH; i += DL_NT) hs[i] = 0xffffffffu;
    if (t < DL_MAXROWS) link[t] = 0xffffu;
    if (t == 0) nwl = 0;
    const uint32_t g = st >= 0 ? a.remap[st] : 0xffffu;   // 0xffff: allows nothing
    // displaced rows: the row's start state as its base, after the table
    uint16_t* rbase = reinterpret_cast<uint16_t*>(tab + DL_WORDS - ZS_DFA_RD_ROWS / 2);
    if (FMT == 2 && t < DL_MAXROWS) rbase[t] = st >= 0 ? a.rdmap[st] : (uint16_t)a.rd_fail;
    // a hit needs this tag; the key also names the call that filled the slot
    // (never this one: keys are written by the EOS kernel after the walk, so
    // every workgroup builds the same plan)
    const unsigned long long key = g < a.memo_slots ? a.memo_key[g] : 0ull;
    const bool hit = st >= 0 && g < a.memo_slots && (uint32_t)(key >> 32) == a.memo_tag && (uint32_t)key != a.memo_seq;
    const bool walk = st >= 0 && !hit;
    // the EOS bit of a walked row when the state's viability is known without
    // the walk (eos_direct, viable[g]); a bad start state allows nothing, so
    // eos is allowed
    const uint32_t viab = a.eos_direct && g != 0xffffu ? a.viable[g] : 0u;
    const uint32_t eos_ok = g == 0xffffu ? 1u : (a.eos_direct && (a.accept[st] || !viab) ? 1u : 0u);
    if (t < DL_MAXROWS) rmode[t] = st < 0 ? DL_FREE : (hit ? (uint16_t)g : (uint16_t)(DL_WALKED | eos_ok));
    if (a.eos_direct && blockIdx.x == 0 && walk) {
        // viability is known now: the caller's flags, and the state's memo
        // slot (keyed with this call's sequence number: no workgroup of this
        // call takes it as a hit)
        if (a.any_user) a.any_user[r] = viab;
        if (g < a.memo_slots) {
            a.memo_any[g] = viab;
            a.memo_key[g] = ((unsigned long long)a.memo_tag << 32) | a.memo_seq;
        }
    }
    __syncthreads();
    // the first row of every walked state: insert g << 16 | row, keep the least
    uint32_t hpos = 0;
    if (walk) {
        const uint32_t hk = g << 16 | r;
        hpos = dl_hash(g);
        while (true) {
            const uint32_t old = atomicCAS(&hs[hpos], 0xffffffffu, hk);
            if (old == 0xffffffffu || (old >> 16) == g) {
                if (old != 0xffffffffu) atomicMin(&hs[hpos], hk);
                break;
            }
            hpos = (hpos + 1) & (DL_HASH - 1);
        }
    }
    __syncthreads();
    const uint32_t first = walk ? (hs[hpos] & 0xffffu) : 0u;
    const bool lead = walk && first == r;
    // the other rows of the state chain behind the first one
    if (walk && !lead) link[r] = atomicExch(&link[first], r);
    {
        uint32_t tot;
        const uint32_t pos = block_excl_scan_u<DL_NT>(lead ? 1u : 0u, reinterpret_cast<uint32_t*>(fb), &tot);
        if (lead) wl[pos] = g << 16 | r;
        if (t == 0) nwl = tot;
    }
    for (int i = t; i < DL_RG * DL_TW; i += DL_NT) (&bm[0][0])[i] = 0;
    __syncthreads();
    const uint32_t nc = nwl;
    const uint32_t rwb = a.rw >> 3;  // bytes per state row (whole words)
    const uint32_t fmask = (1u << a.bits) - 1u;
    // entry of class bit offset cb in row st: the 32 bits from bit cb & 31 of
    // the two words from byte st * rwb + cbw, cbw = the byte offset of the word
    // holding bit cb
    const uint16_t* tgt16 = reinterpret_cast<const uint16_t*>(tab + 4 * (a.ngood + 1));
    const uint32_t fail = FMT == 2 ? a.rd_fail : a.ngood;  // the sink row
    auto step = [&](uint32_t s, uint32_t cb) -> uint32_t {
        if (FMT == 2) {
            // states are their bases: the entry at base + class names its
            // owner in the upper half
            const uint32_t e = tab[s + cb];
            return (e >> 16) == s ? (e & 0xffffu) : fail;
        }
        if (FMT == 1) {
            // class mask of the state, then the target at the rank of its class
            const uint4 rec = reinterpret_cast<const uint4*>(tab)[s];
            const unsigned long long mask = ((unsigned long long)rec.y << 32) | rec.x;
            if (!((mask >> cb) & 1ull)) return fail;
            return tgt16[rec.z + (uint32_t)__popcll(mask & ((1ull << cb) - 1ull))];
        }
        // states < 2^16, row bytes < 2^13: the byte address fits 24 bits
        const uint32_t ba = __umul24(s, rwb) + ((cb >> 3) & ~3u);
        const uint32_t* w = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(tab) + ba);
        return __builtin_amdgcn_alignbit(w[1], w[0], cb) & fmask;
    };
    const uint32_t ncover = a.V > a.ntab ? a.V : a.ntab;
    // states per item: as few groups as fill the grid once (every workgroup
    // builds the same nc, so the same split), at most DL_RG states a group
    const uint32_t ntt = (ncover + ZS_WALK_TILE - 1) / ZS_WALK_TILE;
    const uint32_t ngrp = gridDim.x / ntt > 1u ? gridDim.x / ntt : 1u;
    const uint32_t rg = min((uint32_t)DL_RG, max(1u, (nc + ngrp - 1) / ngrp));
    const uint32_t nrg = (nc + rg - 1) / rg;
    static_assert(DL_TPT == 2 && ZS_WALK_TILE == 2048 && DL_NT == 1024, "run pairing");
    // the thread's two slots of an item's tile: runs of 64 length-sorted
    // slots, wave w takes runs w and 31 - w (a short and a long run)
    const uint32_t wv = (uint32_t)t >> 6;
    const uint32_t sl_off[2] = {wv * 64 + (uint32_t)zs_lane(), (31u - wv) * 64 + (uint32_t)zs_lane()};
    auto fetch = [&](uint32_t w, uint32_t (&meta)[2], uint4 (&wb)[2]) {
        const uint32_t tt = w % ntt;
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const bool ok = w < ntt * nrg && tt < a.nwtile;
            const uint32_t sl = tt * ZS_WALK_TILE + sl_off[j];
            meta[j] = ok ? a.wmeta[sl] : 0xffffffffu;
            wb[j] = ok ? reinterpret_cast<const uint4*>(a.wbytes)[sl] : make_uint4(0, 0, 0, 0);
        }
    };
    uint32_t meta[2];
    uint4 wb[2];
    fetch(blockIdx.x, meta, wb);
    for (uint32_t w = blockIdx.x; w < ntt * nrg; w += gridDim.x) {
        const uint32_t tt = w % ntt, g0 = (w / ntt) * rg;
        const uint32_t nr = min(rg, nc - g0);
        const uint32_t tok0 = tt * ZS_WALK_TILE;
        // the item's start states, then the first-byte words: thread t takes
        // byte t & 255 for the states 16 * (t >> 8) .. + 15
        if (t <= DL_RG) {
            const uint32_t gg = (uint32_t)t < nr ? wl[g0 + t] >> 16 : 0xffffu;
            s0r[t] = gg == 0xffffu ? fail : FMT == 2 ? (uint32_t)rbase[wl[g0 + t] & 0xffffu] : gg;
        }
        dl_bar();
        {
            const uint32_t b = (uint32_t)t & 255u, q = (uint32_t)t >> 8;
            static_assert(DL_RG <= 64 && DL_NT == 1024, "four 16-state quarters per byte");
            if (q * 16 < nr) {
                // states past nr start in the sink row: no branches, so the
                // 16 reads of each kind are in flight together
                const uint32_t cb = ci[b];
                uint32_t m = 0;
#pragma unroll
                for (uint32_t k = 0; k < 16; k++)
                    if (step(s0r[q * 16 + k], cb) != fail) m |= 1u << k;
                reinterpret_cast<uint16_t*>(fb)[b * 4 + q] = (uint16_t)m;
            } else {
                reinterpret_cast<uint16_t*>(fb)[b * 4 + q] = 0;
            }
        }
        // this item's tokens (fetched during the previous item), the next
        // item's fetched now
        uint32_t cm[2] = {meta[0], meta[1]};
        uint4 cw[2] = {wb[0], wb[1]};
        fetch(w + gridDim.x, meta, wb);
        dl_bar();
        // both tokens' surviving states, DL_SIDE of each token at a time,
        // walked side by side (independent chains hide the LDS latency)
        uint32_t L[2], id[2], cb0[2];
        unsigned long long m[2];
#pragma unroll
        for (int j = 0; j < 2; j++) {
            L[j] = cm[j] == 0xffffffffu ? 0u : cm[j] >> 18;   // 0: never allowed
            id[j] = cm[j] & 0x3ffffu;
            m[j] = L[j] ? fb[cw[j].x & 0xffu] : 0ull;         // most tokens end here
            cb0[j] = ci[cw[j].x & 0xffu];
            if (L[j] == DL_EMPTY) {
                // no bytes: allowed from every (live) start state
                m[j] = 0ull;
                const uint32_t off = id[j] - tok0;
                for (uint32_t rr = 0; rr < nr; rr++)
                    if (s0r[rr] != fail) atomicOr(&bm[rr][off >> 5], 1u << (off & 31));
            }
        }
#pragma unroll
        for (int j0 = 0; j0 < 2; j0 += TG) {
            // tokens j0 .. j0 + TG - 1 together: up to SIDE states of each
            // (the ones taken leave m), walked side by side
            auto left = [&]() {
                unsigned long long x = 0ull;
#pragma unroll
                for (int jj = 0; jj < TG; jj++) x |= m[j0 + jj];
                return x;
            };
            while (left()) {
                uint32_t sv[TG][SIDE];
                unsigned long long taken[TG];
#pragma unroll
                for (int jj = 0; jj < TG; jj++) {
                    const int j = j0 + jj;
                    unsigned long long mm = m[j];
#pragma unroll
                    for (int k = 0; k < SIDE; k++) {
                        // no state left: the sink entry (no branch per state)
                        sv[jj][k] = step(s0r[mm ? (uint32_t)__builtin_ctzll(mm) : (uint32_t)DL_RG], cb0[j]);
                        mm &= mm - 1ull;
                    }
                    taken[jj] = m[j] & ~mm;
                    m[j] = mm;
                }
                // the class of the next byte is read while the current step's
                // table reads are in flight
                uint32_t cb[TG];
#pragma unroll
                for (int jj = 0; jj < TG; jj++) cb[jj] = ci[(cw[j0 + jj].x >> 8) & 0xffu];
#pragma unroll
                for (int i = 1; i < 16; i++) {
                    bool go[TG], any = false;
#pragma unroll
                    for (int jj = 0; jj < TG; jj++) {
                        bool live = false;
#pragma unroll
                        for (int k = 0; k < SIDE; k++) live |= sv[jj][k] != fail;
                        go[jj] = live && (uint32_t)i < L[j0 + jj];
                        any |= go[jj];
                    }
                    if (!any) break;
#pragma unroll
                    for (int jj = 0; jj < TG; jj++) {
                        if (!go[jj]) continue;
                        const uint4 w4 = cw[j0 + jj];
                        uint32_t cbn = 0;
                        if (i < 15) {
                            const int n = i + 1;
                            const uint32_t bw = n < 4 ? w4.x : n < 8 ? w4.y : n < 12 ? w4.z : w4.w;
                            cbn = ci[(bw >> (8 * (n & 3))) & 0xffu];
                        }
#pragma unroll
                        for (int k = 0; k < SIDE; k++) sv[jj][k] = step(sv[jj][k], cb[jj]);
                        cb[jj] = cbn;
                    }
                }
#pragma unroll
                for (int jj = 0; jj < TG; jj++) {
                    const int j = j0 + jj;
                    bool live = false;
#pragma unroll
                    for (int k = 0; k < SIDE; k++) live |= sv[jj][k] != fail;
                    if (L[j] > 16 && live) {
                        // bytes past the first 16 from the CSR copy (long tokens)
                        const uint32_t o0 = a.offsets[id[j]], o1 = a.offsets[id[j] + 1];
                        for (uint32_t i = o0 + 16; i < o1; i++) {
                            const uint32_t c = ci[a.bytes[i]];
#pragma unroll
                            for (int k = 0; k < SIDE; k++) sv[jj][k] = step(sv[jj][k], c);
                        }
                    }
                    const uint32_t off = id[j] - tok0;
                    unsigned long long tk = taken[jj];
#pragma unroll
                    for (int k = 0; k < SIDE; k++) {
                        if (tk && sv[jj][k] != fail) atomicOr(&bm[__builtin_ctzll(tk)][off >> 5], 1u << (off & 31));
                        tk &= tk - 1ull;
                    }
                }
            }
        }
        dl_bar();
        // whole words out to every row of the state and its memo slot (and
        // cleared for the next item); bits at ids >= V stay clear; viability
        // counts every table id of the tile
        for (int i = t; i < (int)(nr * DL_TW); i += DL_NT) {
            const uint32_t rr = i / DL_TW, wi = i % DL_TW;
            const uint32_t e = wl[g0 + rr];
            const uint32_t gg = e >> 16;
            const uint32_t word = bm[rr][wi];
            bm[rr][wi] = 0;
            const uint32_t gw = tok0 / 32 + wi;
            uint32_t v = word;
            if (gw == a.words - 1 && (a.V & 31)) v &= (1u << (a.V & 31)) - 1u;
            if (gg < a.memo_slots && gw < a.words) a.memo[(size_t)gg * a.memo_words + gw] = v;
            if (a.eos_direct && gw == (a.eos >> 5) && a.eos < a.V) {
                // the EOS rule here (the same for every row of the state)
                const uint32_t bit = 1u << (a.eos & 31);
                v = (rmode[e & 0xffffu] & 1u) ? (v | bit) : (v & ~bit);
            }
            for (uint32_t rw = e & 0xffffu; rw != 0xffffu; rw = link[rw]) {
                if (gw < a.words) a.out[(size_t)rw * a.words + gw] = v;
                if (word && !a.eos_direct) a.any[rw] = a.epoch;  // every writer stores the same value
            }
        }
    }
    // memo hits and unconstrained rows (the workgroups split the rows' words)
    const uint32_t nall = a.B * a.words;
    for (uint32_t i = blockIdx.x * DL_NT + t; i < nall; i += gridDim.x * DL_NT) {
        const uint32_t rr = i / a.words, wi = i - rr * a.words;
        const uint32_t mode = rmode[rr];
        if ((mode & ~1u) == DL_WALKED) continue;
        uint32_t v;
        if (mode == DL_FREE) {
            v = 0xffffffffu;
            if (wi == a.words - 1 && (a.V & 31)) v = (1u << (a.V & 31)) - 1u;
        } else {
            // the stored walk and its viability, then the EOS rule (here, or
            // by the EOS kernel)
            v = a.memo[(size_t)mode * a.memo_words + wi];
            if (a.eos_direct) {
                if (wi == 0 && a.any_user) a.any_user[rr] = a.memo_any[mode];
                if (a.eos < a.V && wi == (a.eos >> 5)) {
                    const uint32_t bit = 1u << (a.eos & 31);
                    v = (a.accept[a.states[rr]] || !a.memo_any[mode]) ? (v | bit) : (v & ~bit);
                }
            } else if (wi == 0 && a.memo_any[mode]) {
                a.any[rr] = a.epoch;
            }
        }
        a.out[(size_t)rr * a.words + wi] = v;
    }
}

__global__ void zs_k_fill_u32(uint32_t* p, uint32_t n, uint32_t v) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// EOS rule (logit_fsm.rs:258-262): eos allowed iff is_accept(s) or no token is
// viable; ids >= ntab other than eos stay disallowed. With epoch != 0 the
// viability flags hold the epoch of the call that found a viable token (the
// packed walk: no clearing pass), and the caller's 0/1 flags are written here.
__global__ void zs_k_dfa_eos(dm_args a) {
    uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.B) return;
    int32_t st = a.states[r];
    if (st < 0) return;
    const bool anyv = a.epoch ? a.any[r] == a.epoch : a.any[r] != 0;
    if (a.epoch && a.any_user) a.any_user[r] = anyv ? 1u : 0u;
    // the walk of this call is complete: the state's memo slot is valid from
    // the next call on (rows of one state store the same values)
    const uint32_t g = a.remap[st];
    if (g < a.memo_slots) {
        a.memo_any[g] = anyv ? 1u : 0u;
        a.memo_key[g] = ((unsigned long long)a.memo_tag << 32) | a.memo_seq;
    }
    if (a.eos >= a.V) return;
    bool ok = a.accept[st] || !anyv;
    uint32_t* o = a.out + (size_t)r * a.words + (a.eos >> 5);
    uint32_t bit = 1u << (a.eos & 31);
    *o = ok ? (*o | bit) : (*o & ~bit);
}

extern "C" int zs_dfa_mask_launch(const dm_args& a, bool packed_lds, uint32_t ncu, uint32_t* any_scratch,
                                  hipStream_t stream) {
    dm_args x = a;
    x.any = any_scratch;
    uint32_t ncover = a.V > a.ntab ? a.V : a.ntab;
    if (!packed_lds || a.B > DL_MAXROWS) {
        x.memo_slots = 0;      // the memo and the direct EOS rule are the packed walk's
        x.eos_direct = 0;
    }
    if (packed_lds && a.B <= DL_MAXROWS) {
        // one workgroup per CU, fewer when there are fewer (tile, state)
        // pairs (B bounds the distinct states; the kernel splits them)
        const uint32_t ntt = (ncover + ZS_WALK_TILE - 1) / ZS_WALK_TILE;
        const uint32_t items = ntt * a.B;
        const dim3 grid(min(items, ncu));
        if (a.sparse == 2)
            hipLaunchKernelGGL((zs_k_dfa_mask_packed<2, 4, 2>), grid, dim3(DL_NT), 0, stream, x);
        else if (a.sparse)
            hipLaunchKernelGGL((zs_k_dfa_mask_packed<1, 4, 2>), grid, dim3(DL_NT), 0, stream, x);
        else if (a.dense)
            hipLaunchKernelGGL((zs_k_dfa_mask_packed<0, 8, 1>), grid, dim3(DL_NT), 0, stream, x);
        else
            hipLaunchKernelGGL((zs_k_dfa_mask_packed<0, 4, 2>), grid, dim3(DL_NT), 0, stream, x);
        if (x.eos_direct) return hipGetLastError() == hipSuccess ? 0 : -1;   // the walk applied the EOS rule
    } else {
        // epoch 0: the caller's own 0/1 flags, cleared first; otherwise the
        // context's flags, compared with the epoch as in the packed walk
        if (!x.epoch) hipLaunchKernelGGL(zs_k_fill_u32, dim3((a.B + 255) / 256), dim3(256), 0, stream, any_scratch, a.B, 0u);
        dim3 grid((ncover + DM_TOK - 1) / DM_TOK, (a.B + DM_ROWS - 1) / DM_ROWS);
        hipLaunchKernelGGL(zs_k_dfa_mask<false>, grid, dim3(DM_NT), 0, stream, x);
    }
    hipLaunchKernelGGL(zs_k_dfa_eos, dim3((a.B + 63) / 64), dim3(64), 0, stream, x);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
