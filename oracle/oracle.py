"""ctypes binding of the CPU oracle (oracle/zs_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, always as the checker. The product never imports
this module.

`reference_step` chains the restated reference functions in the decode-loop
order of rest.rs:2594-2624 for one row.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")


def build():
    subprocess.run(["make", "-s", "-C", HERE], check=True)
    return LIB_PATH


def _load():
    if not os.path.exists(LIB_PATH):
        build()
    lib = C.CDLL(LIB_PATH)
    P = C.POINTER
    f32p, u32p, u8p = P(C.c_float), P(C.c_uint32), P(C.c_uint8)
    sig = {
        "zo_sample_with_r": (C.c_uint32, [f32p, C.c_uint32, C.c_float, C.c_uint32, C.c_float, C.c_float, C.c_float]),
        "zo_adjust_logits": (None, [f32p, C.c_uint32, u32p, f32p, C.c_uint32, u32p, u32p, C.c_uint32,
                                    C.c_float, C.c_float, C.c_float]),
        "zo_modifies_logits": (C.c_int, [C.c_uint32, C.c_float, C.c_float, C.c_float]),
        "zo_dfa_walk": (C.c_int, [u32p, u8p, C.c_uint32, u8p, C.c_uint32, u32p]),
        "zo_dfa_is_live": (C.c_int, [u32p, u8p, u8p, C.c_uint32, C.c_uint32, u8p, u8p]),
        "zo_dfa_live_all": (None, [u32p, u8p, u8p, C.c_uint32, u8p]),
        "zo_dfa_allowed": (C.c_int, [u32p, u8p, u8p, C.c_uint32, u32p, u8p, u8p, C.c_uint32, u8p]),
        "zo_apply_mask": (None, [f32p, C.c_uint32, u32p, C.c_uint32, u32p, u8p, u8p, u8p, C.c_int64,
                                 u32p, u8p, u8p, C.c_uint32, C.c_uint32]),
        "zo_advance": (C.c_uint32, [u32p, u8p, C.c_uint32, C.c_uint32, u32p, u8p, u8p, C.c_uint32, C.c_uint32]),
        "zo_logprobs_observe": (C.c_uint32, [f32p, C.c_uint32, C.c_uint32, C.c_uint32, f32p, u32p, f32p]),
        "zo_token_uncertainty": (None, [f32p, C.c_uint32, C.c_uint32, f32p]),
        "zo_report": (C.c_int64, [f32p, f32p, C.c_uint32, C.c_uint32, C.c_float, C.c_float, f32p]),
        "zo_argmax_first": (C.c_uint32, [f32p, C.c_uint32]),
        "zo_verify_drafts": (C.c_uint32, [u32p, C.c_uint32, f32p, C.c_uint32, C.c_uint32, u32p]),
        "zo_step_seed": (C.c_uint32, [C.c_uint32, C.c_uint32]),
        "zo_rng01": (C.c_float, [C.c_uint32]),
        "zo_sample_topk": (C.c_uint32, [f32p, u32p, C.c_uint32, C.c_float, C.c_uint32, C.c_float, C.c_uint32]),
        "zo_hash_u32": (C.c_uint32, [C.c_uint32]),
        "zo_rand01": (C.c_float, [C.c_uint32, C.c_uint32]),
        "zo_bargmax": (C.c_uint32, [f32p, C.c_uint32]),
        "zo_bsample": (C.c_uint32, [f32p, C.c_uint32, C.c_float, C.c_uint32]),
        "zo_btopk": (None, [f32p, C.c_uint32, C.c_uint32, f32p, u32p]),
        "zo_philox4x32_10": (None, [u32p, u32p, u32p]),
        "zo_philox_uniform": (C.c_float, [C.c_uint64, C.c_uint64, C.c_uint32]),
        "zo_spec_verify": (C.c_uint32, [f32p, f32p, u32p, C.c_uint32, C.c_uint32, C.c_float, C.c_uint64,
                                        C.c_uint64, u32p]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _f32(a):
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a, a.ctypes.data_as(C.POINTER(C.c_float))


def _u32(a):
    a = np.ascontiguousarray(a, dtype=np.uint32)
    return a, a.ctypes.data_as(C.POINTER(C.c_uint32))


def _u8(a):
    a = np.ascontiguousarray(a, dtype=np.uint8)
    return a, a.ctypes.data_as(C.POINTER(C.c_uint8))


# ---- sampler.rs / decode_ctrl.rs ------------------------------------------
def sample_with_r(logits, temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, r=0.5):
    x, xp = _f32(logits)
    return int(lib().zo_sample_with_r(xp, x.size, temperature, top_k, top_p, min_p, r))


def adjust_logits(logits, bias=(), counts=(), repeat=1.0, presence=0.0, frequency=0.0):
    """decode_ctrl.rs:107-126 on a copy. bias: [(id, b)], counts: [(id, cnt)]."""
    y, yp = _f32(np.array(logits, dtype=np.float32, copy=True))
    bi, bip = _u32([b[0] for b in bias] or [0])
    bv, bvp = _f32([b[1] for b in bias] or [0])
    ci, cip = _u32([c[0] for c in counts] or [0])
    cv, cvp = _u32([c[1] for c in counts] or [0])
    lib().zo_adjust_logits(yp, y.size, bip, bvp, len(bias), cip, cvp, len(counts), repeat, presence, frequency)
    return y


def modifies_logits(nbias, repeat=1.0, presence=0.0, frequency=0.0):
    return bool(lib().zo_modifies_logits(nbias, repeat, presence, frequency))


# ---- logit_fsm.rs -------------------------------------------------------------
class Dfa:
    """Dense DFA: trans[S,256] uint32, dead[S], accept[S] (see zs_oracle.c)."""

    def __init__(self, trans, dead, accept):
        self.trans, self.tp = _u32(np.asarray(trans).reshape(-1))
        self.S = self.trans.size // 256
        self.dead, self.dp = _u8(dead)
        self.accept, self.ap = _u8(accept)
        self.live = np.zeros(self.S, np.uint8)
        lib().zo_dfa_live_all(self.tp, self.dp, self.ap, self.S, self.live.ctypes.data_as(C.POINTER(C.c_uint8)))
        self.lp = self.live.ctypes.data_as(C.POINTER(C.c_uint8))

    def is_live_literal(self, s):
        return bool(lib().zo_dfa_is_live(self.tp, self.dp, self.ap, self.S, s, None, None))


class Vocab:
    """Token byte table: list of bytes or None per token id, plus eos."""

    def __init__(self, tokens, eos):
        self.ntab = len(tokens)
        self.eos = eos
        offs = [0]
        buf = bytearray()
        valid = []
        for t in tokens:
            if t is None:
                valid.append(0)
            else:
                valid.append(1)
                buf += t
            offs.append(len(buf))
        self.offsets, self.op = _u32(offs)
        self.bytes, self.bp = _u8(np.frombuffer(bytes(buf) or b"\0", np.uint8))
        self.valid, self.vp = _u8(valid or [0])


def dfa_allowed(dfa, vocab, state):
    out = np.zeros(max(vocab.ntab, 1), np.uint8)
    anyv = lib().zo_dfa_allowed(dfa.tp, dfa.dp, dfa.lp, state, vocab.op, vocab.bp, vocab.vp, vocab.ntab,
                                out.ctypes.data_as(C.POINTER(C.c_uint8)))
    return out[: vocab.ntab], bool(anyv)


def apply_mask(logits, ban=(), dfa=None, vocab=None, state=-1):
    x, xp = _f32(np.array(logits, dtype=np.float32, copy=True))
    bn, bnp = _u32(list(ban) or [0])
    if dfa is None:
        lib().zo_apply_mask(xp, x.size, bnp, len(ban), None, None, None, None, -1, None, None, None, 0, 0)
    else:
        lib().zo_apply_mask(xp, x.size, bnp, len(ban), dfa.tp, dfa.dp, dfa.lp, dfa.ap, int(state), vocab.op,
                            vocab.bp, vocab.vp, vocab.ntab, vocab.eos)
    return x


def mask_bits(V, ban=(), dfa=None, vocab=None, state=-1):
    """Allow bitset (uint32 words, bit i of word w = id 32w+i) implied by
    apply_mask over zero logits."""
    x = apply_mask(np.zeros(V, np.float32), ban, dfa, vocab, state)
    return pack_bits(~np.isneginf(x))


def pack_bits(ok):
    ok = np.asarray(ok, bool)
    words = (ok.size + 31) // 32
    pad = np.zeros(words * 32, np.uint64)
    pad[: ok.size] = ok
    w = (pad.reshape(words, 32) << np.arange(32, dtype=np.uint64)).sum(axis=1)
    return w.astype(np.uint32)


def advance(dfa, vocab, state, token):
    return int(lib().zo_advance(dfa.tp, dfa.dp, state, token, vocab.op, vocab.bp, vocab.vp, vocab.ntab, vocab.eos))


# ---- logprobs.rs / hallucination.rs -------------------------------------------
def logprobs_observe(logits, chosen, top_n):
    x, xp = _f32(logits)
    n = min(top_n, 20)
    lp = C.c_float()
    ids = np.zeros(max(n, 1), np.uint32)
    lps = np.zeros(max(n, 1), np.float32)
    k = lib().zo_logprobs_observe(xp, x.size, chosen, n, C.byref(lp), ids.ctypes.data_as(C.POINTER(C.c_uint32)),
                                  lps.ctypes.data_as(C.POINTER(C.c_float)))
    return lp.value, ids[:k].copy(), lps[:k].copy()


def token_uncertainty(logits, chosen):
    x, xp = _f32(logits)
    out = np.zeros(4, np.float32)
    lib().zo_token_uncertainty(xp, x.size, chosen, out.ctypes.data_as(C.POINTER(C.c_float)))
    return out  # entropy, max_prob, margin, chosen_logprob


def report(entropy, max_prob, vocab, thr_ent=2.0, thr_p=0.4):
    e, ep = _f32(entropy)
    m, mp = _f32(max_prob)
    out = np.zeros(4, np.float32)
    peak = lib().zo_report(ep, mp, e.size, vocab, thr_ent, thr_p, out.ctypes.data_as(C.POINTER(C.c_float)))
    return out, (None if peak < 0 else int(peak))


# ---- spec_decode.rs ------------------------------------------------------------
def argmax_first(v):
    x, xp = _f32(v)
    return int(lib().zo_argmax_first(xp, x.size))


def verify_drafts(drafts, rows):
    rows = np.ascontiguousarray(rows, np.float32)
    d, dp = _u32(list(drafts) or [0])
    r, rp = _f32(rows.reshape(-1))
    bonus = C.c_uint32(0)
    nrows = rows.shape[0] if rows.ndim == 2 else 0
    V = rows.shape[1] if rows.ndim == 2 else 0
    acc = lib().zo_verify_drafts(dp, len(drafts), rp, nrows, V, C.byref(bonus))
    return int(acc), int(bonus.value)


# ---- gpu/sampling.rs, shaders.rs ------------------------------------------------
def step_seed(base, gen_idx):
    return int(lib().zo_step_seed(base & 0xFFFFFFFF, gen_idx & 0xFFFFFFFF))


def rng01(seed):
    return float(lib().zo_rng01(seed & 0xFFFFFFFF))


def sample_topk(vals, idxs, temp, top_k, top_p, seed):
    v, vp = _f32(vals)
    i, ip = _u32(idxs)
    return int(lib().zo_sample_topk(vp, ip, v.size, temp, top_k, top_p, seed & 0xFFFFFFFF))


def hash_u32(x):
    return int(lib().zo_hash_u32(x & 0xFFFFFFFF))


def rand01(s, i):
    return float(lib().zo_rand01(s & 0xFFFFFFFF, i & 0xFFFFFFFF))


def bargmax(logits):
    x, xp = _f32(logits)
    return int(lib().zo_bargmax(xp, x.size))


def bsample(logits, temp, seed):
    x, xp = _f32(logits)
    return int(lib().zo_bsample(xp, x.size, temp, seed & 0xFFFFFFFF))


def btopk(logits, K):
    x, xp = _f32(logits)
    vals = np.zeros(K, np.float32)
    idxs = np.zeros(K, np.uint32)
    lib().zo_btopk(xp, x.size, K, vals.ctypes.data_as(C.POINTER(C.c_float)), idxs.ctypes.data_as(C.POINTER(C.c_uint32)))
    return vals, idxs


# ---- Philox ---------------------------------------------------------------------
def philox4x32_10(ctr, key):
    c, cp = _u32(ctr)
    k, kp = _u32(key)
    out = np.zeros(4, np.uint32)
    lib().zo_philox4x32_10(cp, kp, out.ctypes.data_as(C.POINTER(C.c_uint32)))
    return out


def philox_uniform(seed, counter, tag=0):
    return float(lib().zo_philox_uniform(seed & (2**64 - 1), counter & (2**64 - 1), tag))


def spec_verify(target, draft, drafts, temperature, seed=0, counter=0):
    """target [k+1, V], draft [k, V] or None -> (accepted, next)."""
    t, tp = _f32(np.asarray(target, np.float32).reshape(-1))
    k = len(drafts)
    V = t.size // (k + 1)
    if draft is None:
        dp = None
    else:
        d, dp = _f32(np.asarray(draft, np.float32).reshape(-1))
    ids, ip = _u32(list(drafts) or [0])
    nxt = C.c_uint32(0)
    acc = lib().zo_spec_verify(tp, dp, ip, k, V, temperature, seed & (2**64 - 1), counter & (2**64 - 1),
                               C.byref(nxt))
    return int(acc), int(nxt.value)


# ---- one row through the reference decode-loop order ------------------------------
def reference_step(x, params, ban=(), bias=(), counts=(), dfa=None, vocab=None, state=-1, seed=0, counter=0):
    """Returns dict(token, logprob, top_ids, top_lps, entropy, max_prob, margin,
    chosen_lp, r) for one row (rest.rs:2594-2624 order).

    params: dict with temperature, top_k, top_p, min_p, repeat, presence,
    frequency, top_logprobs.
    """
    xm = apply_mask(x, ban, dfa, vocab, state)
    rep, pres, freq = params.get("repeat", 1.0), params.get("presence", 0.0), params.get("frequency", 0.0)
    if modifies_logits(len(bias), rep, pres, freq):
        y = adjust_logits(xm, bias, counts, rep, pres, freq)
    else:
        y = xm
    T = params.get("temperature", 1.0)
    r = philox_uniform(seed, counter, 0)
    tok = sample_with_r(y, T, params.get("top_k", 0), params.get("top_p", 1.0), params.get("min_p", 0.0), r)
    lp, ids, lps = logprobs_observe(xm, tok, params.get("top_logprobs", 0))
    unc = token_uncertainty(xm, tok)
    return dict(token=tok, logprob=lp, top_ids=ids, top_lps=lps, entropy=float(unc[0]), max_prob=float(unc[1]),
                margin=float(unc[2]), chosen_lp=float(unc[3]), r=r, masked=xm)
