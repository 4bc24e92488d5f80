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
            if (zs_lane() == 0 && anyv) atomicOr(&a.any[r], 1u);
        }
    }
}

__global__ void zs_k_fill_u32(uint32_t* p, uint32_t n, uint32_t v) {
    uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = v;
}

// EOS rule (logit_fsm.rs:258-262): eos allowed iff is_accept(s) or no token is
// viable; ids >= ntab other than eos stay disallowed.
__global__ void zs_k_dfa_eos(dm_args a) {
    uint32_t r = blockIdx.x * blockDim.x + threadIdx.x;
    if (r >= a.B) return;
    int32_t st = a.states[r];
    if (st < 0) return;
    if (a.eos >= a.V) return;
    bool ok = a.accept[st] || a.any[r] == 0;
    uint32_t* o = a.out + (size_t)r * a.words + (a.eos >> 5);
    uint32_t bit = 1u << (a.eos & 31);
    *o = ok ? (*o | bit) : (*o & ~bit);
}

extern "C" int zs_dfa_mask_launch(const dm_args& a, bool lds, uint32_t* any_scratch, hipStream_t stream) {
    dm_args x = a;
    x.any = any_scratch;
    hipLaunchKernelGGL(zs_k_fill_u32, dim3((a.B + 255) / 256), dim3(256), 0, stream, any_scratch, a.B, 0u);
    uint32_t ncover = a.V > a.ntab ? a.V : a.ntab;
    dim3 grid((ncover + DM_TOK - 1) / DM_TOK, (a.B + DM_ROWS - 1) / DM_ROWS);
    if (lds) hipLaunchKernelGGL(zs_k_dfa_mask<true>, grid, dim3(DM_NT), 0, stream, x);
    else hipLaunchKernelGGL(zs_k_dfa_mask<false>, grid, dim3(DM_NT), 0, stream, x);
    hipLaunchKernelGGL(zs_k_dfa_eos, dim3((a.B + 63) / 64), dim3(64), 0, stream, x);
    return hipGetLastError() == hipSuccess ? 0 : -1;
}
