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

// Persistent walk over the bit-packed table (good states only, `bits`-bit
// entries, all ones = fail). One workgroup per CU stages the table in LDS once
// and then takes items: a tile of ZS_WALK_TILE ids times a group of DL_RG
// constrained rows. A thread walks DL_TPT tokens, each through all rows of the
// group at once: the byte and its class are read once per step and the rows'
// states advance side by side. Inside a tile the tokens come in length order
// (the vocabulary's walk order), so the lanes of a wave walk tokens of nearly
// equal length; allowed ids are set in an LDS bitmap of the tile and written
// out as whole words. A step costs one LDS class read and one 64-bit LDS
// table read per row.
#define DL_NT 1024
#define DL_TPT (ZS_WALK_TILE / DL_NT)
#define DL_RG 8                  // rows walked together
#define DL_TW (ZS_WALK_TILE / 32) // bitmap words per row and tile
#define DL_WORDS (ZS_DFA_LDS_BYTES / 4)
#define DL_MAXROWS ZS_DFA_MAXROWS
template <bool SPARSE>
__global__ __launch_bounds__(DL_NT) void zs_k_dfa_mask_packed(dm_args a) {
    __shared__ uint32_t tab[DL_WORDS];
    __shared__ uint16_t ci[256];
    __shared__ uint32_t bm[DL_RG][DL_TW];
    __shared__ uint16_t crow[DL_MAXROWS];  // constrained rows
    __shared__ uint16_t cst[DL_MAXROWS];   // their good start state (0xffff: none allowed)
    __shared__ uint16_t frow[DL_MAXROWS];  // unconstrained rows
    __shared__ uint32_t ncr, nfr;
    const int t = threadIdx.x;
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
    if (t == 0) ncr = nfr = 0;
    __syncthreads();
    // constrained and unconstrained rows in order (every workgroup builds the
    // same lists)
    for (uint32_t r0 = 0; r0 < a.B; r0 += DL_NT) {
        const uint32_t r = r0 + t;
        const int32_t st = r < a.B ? a.states[r] : 0;
        const bool c = r < a.B && st >= 0, f = r < a.B && st < 0;
        uint32_t tot;
        const uint32_t pos = block_excl_scan_u<DL_NT>(c ? 1u : 0u, reinterpret_cast<uint32_t*>(bm), &tot);
        if (c) {
            crow[ncr + pos] = (uint16_t)r;
            cst[ncr + pos] = a.remap[st];
        }
        uint32_t ftot;
        const uint32_t fpos = block_excl_scan_u<DL_NT>(f ? 1u : 0u, reinterpret_cast<uint32_t*>(bm), &ftot);
        if (f) frow[nfr + fpos] = (uint16_t)r;
        __syncthreads();
        if (t == 0) { ncr += tot; nfr += ftot; }
        __syncthreads();
    }
    const uint32_t nc = ncr;
    const uint32_t rwb = a.rw >> 3;  // bytes per state row (whole words)
    const uint32_t fmask = (1u << a.bits) - 1u;
    // entry of class bit offset cb in row st: the 32 bits from bit cb & 31 of
    // the two words from byte st * rwb + cbw, cbw = the byte offset of the word
    // holding bit cb (computed once per byte, shared by the rows)
    const uint16_t* tgt16 = reinterpret_cast<const uint16_t*>(tab + 4 * (a.ngood + 1));
    auto step = [&](uint32_t st, uint32_t cb, uint32_t cbw) -> uint32_t {
        if (SPARSE) {
            // class mask of the state, then the target at the rank of its class
            const uint4 rec = reinterpret_cast<const uint4*>(tab)[st];
            const unsigned long long mask = ((unsigned long long)rec.y << 32) | rec.x;
            if (!((mask >> cb) & 1ull)) return a.ngood;
            return tgt16[rec.z + (uint32_t)__popcll(mask & ((1ull << cb) - 1ull))];
        }
        // states < 2^16, row bytes < 2^13: the byte address fits 24 bits
        const uint32_t ba = __umul24(st, rwb) + cbw;
        const uint32_t* w = reinterpret_cast<const uint32_t*>(reinterpret_cast<const uint8_t*>(tab) + ba);
        return __builtin_amdgcn_alignbit(w[1], w[0], cb) & fmask;
    };
    const uint32_t fail = a.ngood;  // the sink row
    const uint32_t ncover = a.V > a.ntab ? a.V : a.ntab;
    const uint32_t ntt = (ncover + ZS_WALK_TILE - 1) / ZS_WALK_TILE, nrg = (nc + DL_RG - 1) / DL_RG;
    for (uint32_t w = blockIdx.x; w < ntt * nrg; w += gridDim.x) {
        const uint32_t tt = w % ntt, g0 = (w / ntt) * DL_RG;
        const uint32_t nr = min((uint32_t)DL_RG, nc - g0);
        const uint32_t tok0 = tt * ZS_WALK_TILE;
        for (int i = t; i < DL_RG * DL_TW; i += DL_NT) (&bm[0][0])[i] = 0;
        uint32_t s0[DL_RG];
#pragma unroll
        for (int rr = 0; rr < DL_RG; rr++) {
            const uint32_t g = (uint32_t)rr < nr ? cst[g0 + rr] : 0xffffu;
            s0[rr] = g == 0xffffu ? fail : g;
        }
        __syncthreads();
#pragma unroll
        for (int j = 0; j < DL_TPT; j++) {
            // runs of 64 length-sorted slots: wave w takes runs w and 31 - w, so
            // its lanes walk tokens of nearly one length and every wave gets a
            // short and a long run (the item waits for its slowest wave)
            static_assert(DL_TPT == 2 && ZS_WALK_TILE == 2048 && DL_NT == 1024, "run pairing");
            const uint32_t wv = (uint32_t)t >> 6;
            const uint32_t run = j == 0 ? wv : 31u - wv;
            const uint32_t slot = tok0 + run * 64 + (uint32_t)zs_lane();
            if (tt >= a.nwtile) break;
            const uint32_t meta = a.wmeta[slot];
            const uint4 wb = reinterpret_cast<const uint4*>(a.wbytes)[slot];  // issued with meta
            if (meta == 0xffffffffu) continue;
            const uint32_t id = meta & 0x3ffffu, L = meta >> 18;
            if (L == 0) continue;  // no bytes or not a token: never allowed
            const uint32_t bw[4] = {wb.x, wb.y, wb.z, wb.w};
            uint32_t s[DL_RG];
#pragma unroll
            for (int rr = 0; rr < DL_RG; rr++) s[rr] = s0[rr];
            // failed walks sit in the sink row: every row steps unconditionally
#pragma unroll
            for (int i = 0; i < 16; i++) {
                if ((uint32_t)i >= L) break;
                const uint32_t cb = ci[(bw[i >> 2] >> (8 * (i & 3))) & 0xffu];
                const uint32_t cbw = (cb >> 3) & ~3u;
#pragma unroll
                for (int rr = 0; rr < DL_RG; rr++) s[rr] = step(s[rr], cb, cbw);
            }
            if (L > 16) {
                // bytes past the first 16 from the CSR copy (long tokens)
                const uint32_t o0 = a.offsets[id], o1 = a.offsets[id + 1];
                for (uint32_t i = o0 + 16; i < o1; i++) {
                    const uint32_t cb = ci[a.bytes[i]];
                    const uint32_t cbw = (cb >> 3) & ~3u;
#pragma unroll
                    for (int rr = 0; rr < DL_RG; rr++) s[rr] = step(s[rr], cb, cbw);
                }
            }
            const uint32_t off = id - tok0;
#pragma unroll
            for (int rr = 0; rr < DL_RG; rr++)
                if (s[rr] != fail) atomicOr(&bm[rr][off >> 5], 1u << (off & 31));
        }
        __syncthreads();
        // whole words out; bits at ids >= V stay clear; viability counts every
        // table id of the tile
        for (int i = t; i < (int)(nr * DL_TW); i += DL_NT) {
            const uint32_t rr = i / DL_TW, wi = i % DL_TW;
            const uint32_t r = crow[g0 + rr];
            const uint32_t word = bm[rr][wi];
            const uint32_t gw = tok0 / 32 + wi;
            if (gw < a.words) {
                uint32_t v = word;
                if (gw == a.words - 1 && (a.V & 31)) v &= (1u << (a.V & 31)) - 1u;
                a.out[(size_t)r * a.words + gw] = v;
            }
            if (word) a.any[r] = a.epoch;  // every writer stores the same value
        }
        __syncthreads();
    }
    // unconstrained rows: every id below V (the workgroups split the words)
    const uint32_t nfw = nfr * a.words;
    for (uint32_t i = blockIdx.x * DL_NT + t; i < nfw; i += gridDim.x * DL_NT) {
        const uint32_t k = i / a.words, wi = i - k * a.words;
        uint32_t v = 0xffffffffu;
        if (wi == a.words - 1 && (a.V & 31)) v = (1u << (a.V & 31)) - 1u;
        a.out[(size_t)frow[k] * a.words + wi] = v;
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
    if (packed_lds && a.B <= DL_MAXROWS) {
        const uint32_t items = ((ncover + ZS_WALK_TILE - 1) / ZS_WALK_TILE) * ((a.B + DL_RG - 1) / DL_RG);
        if (a.sparse)
            hipLaunchKernelGGL(zs_k_dfa_mask_packed<true>, dim3(min(items, ncu)), dim3(DL_NT), 0, stream, x);
        else
            hipLaunchKernelGGL(zs_k_dfa_mask_packed<false>, dim3(min(items, ncu)), dim3(DL_NT), 0, stream, x);
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
