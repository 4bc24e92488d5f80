"""Known-answer tests that pin the CPU oracle to the reference.

Each test transcribes a reference unit test (cited) or checks a closed form /
brute-force property chosen so that a plausible restatement mistake fails.
CPU only.
"""
import itertools
import math

import numpy as np
import pytest

from oracle import oracle as O
from tests.tiny import (TINY_EOS, TINY_TOKENS, dfa_ab_opt, dfa_ab_plus_c, dfa_ab_star_c, dfa_abc, masked)


# ---------------------------------------------------------------- sampler.rs
def test_temperature_zero_is_argmax():  # sampler.rs:134-141
    for r in (0.0, 0.3, 0.99):
        assert O.sample_with_r([0.1, 0.5, 0.9, 0.2, 0.7], 0.0, 0, 1.0, 0.0, r) == 2


def test_temperature_zero_ties_are_deterministic():  # sampler.rs:143-152
    # max_by returns the LAST maximal element
    assert O.sample_with_r([1.0] * 8, 0.0, 0, 1.0, 0.0, 0.5) == 7


def test_greedy_nan_restarts_fold():
    # partial_cmp(NaN, x) is None -> Equal -> the later element is kept
    x = [5.0, float("nan"), 1.0, 2.0]
    assert O.sample_with_r(x, 0.0, 0, 1.0, 0.0, 0.5) == 3
    x = [5.0, 1.0, float("nan")]
    assert O.sample_with_r(x, 0.0, 0, 1.0, 0.0, 0.5) == 2


def test_min_p_prunes_the_tail():  # sampler.rs:154-165
    logits = [-10.0, 5.0, 4.9, -10.0]
    for r in np.linspace(1e-6, 0.9999, 200):
        assert O.sample_with_r(logits, 1.0, 0, 1.0, 0.5, float(r)) in (1, 2)


def test_seeded_stream_deterministic_and_seed_sensitive():  # sampler.rs:167-178
    logits = [1.0, 1.1, 1.2, 1.3, 1.4, 1.5]

    def run(seed):
        return [O.sample_with_r(logits, 1.0, 0, 1.0, 0.0, O.philox_uniform(seed, c)) for c in range(32)]

    assert run(42) == run(42)
    assert run(42) != run(43)


def test_high_temperature_explores():  # sampler.rs:180-192
    logits = [1.0, 1.01, 1.02, 1.03, 1.04, 1.05]
    seen = {O.sample_with_r(logits, 100.0, 0, 1.0, 0.0, O.philox_uniform(1, c)) for c in range(200)}
    assert len(seen) >= 2


def test_smoke_sampler_ranges():  # tests/test_smoke.rs:22-42
    assert O.sample_with_r([0.0] * 100, 1.0, 50, 0.9, 0.0, 0.5) < 100
    logits = [i * 0.01 for i in range(1000)]
    assert O.sample_with_r(logits, 2.0, 10, 0.9, 0.0, 0.5) < 1000


def _brute_sample(x, T, top_k, top_p, min_p, r):
    """Independent float32 restatement with numpy (sequential loops)."""
    x = np.asarray(x, np.float32)
    V = x.size
    if T <= 0:
        best = 0
        for i in range(1, V):
            if not (x[best] > x[i]):
                best = i
        return best
    l = x / np.float32(T) if T != 1.0 else x.copy()
    if 0 < top_k < V:
        order = sorted(range(V), key=lambda i: (-float(l[i]), i))
        thr = l[order[top_k - 1]]
        l = np.where(l < thr, np.float32(-np.inf), l).astype(np.float32)
    m = np.float32(np.max(l))
    s = np.float32(0)
    e = np.exp((l - m).astype(np.float32)).astype(np.float32)
    for v in e:
        s = np.float32(s + v)
    p = (e / s).astype(np.float32)
    if min_p > 0:
        cut = np.float32(np.float32(min_p) * np.max(p))
        kept = np.float32(0)
        for i in range(V):
            if p[i] < cut:
                p[i] = 0
            else:
                kept = np.float32(kept + p[i])
        if kept > 0:
            p = (p / kept).astype(np.float32)
    if top_p < 1.0:
        order = sorted(range(V), key=lambda i: (-float(p[i]), i))
        f = np.zeros(V, np.float32)
        cum = np.float32(0)
        for i in order:
            if cum >= np.float32(top_p):
                break
            f[i] = p[i]
            cum = np.float32(cum + p[i])
        s2 = np.float32(0)
        for v in f:
            s2 = np.float32(s2 + v)
        if s2 > 0:
            p = (f / s2).astype(np.float32)
    cum = np.float32(0)
    for i in range(V):
        cum = np.float32(cum + p[i])
        if cum >= np.float32(r):
            return i
    return V - 1


@pytest.mark.parametrize("seed", range(12))
def test_sampler_matches_brute_force(seed):
    # numpy's exp is not glibc expf, so compare on inputs whose exp values are
    # exactly representable: logits from {0, -ln2 * k} would still round; use
    # small vocabularies and accept only when both agree on a reference with
    # exact powers of two: x = k*ln(2) makes exp(x-m) = 2^(k-kmax) exactly in
    # glibc and numpy alike.
    rng = np.random.default_rng(seed)
    V = int(rng.integers(2, 40))
    k = rng.integers(-20, 3, size=V)
    x = (k.astype(np.float64) * math.log(2)).astype(np.float32)
    for T, top_k, top_p, min_p in [(1.0, 0, 1.0, 0.0), (1.0, 3, 1.0, 0.0), (1.0, 0, 0.7, 0.0),
                                   (1.0, 0, 1.0, 0.05), (1.0, 5, 0.9, 0.01), (0.0, 0, 1.0, 0.0)]:
        for r in rng.random(6).astype(np.float32):
            got = O.sample_with_r(x, T, top_k, top_p, min_p, float(r))
            exp = _brute_sample(x, T, top_k, top_p, min_p, float(r))
            assert got == exp, (x, T, top_k, top_p, min_p, r)


def test_topk_ge_vocab_and_top_p_one_are_noops():
    rng = np.random.default_rng(3)
    x = rng.normal(0, 2, 50).astype(np.float32)
    for r in rng.random(20):
        a = O.sample_with_r(x, 0.9, 0, 1.0, 0.0, float(r))
        assert O.sample_with_r(x, 0.9, 50, 1.0, 0.0, float(r)) == a
        assert O.sample_with_r(x, 0.9, 500, 1.0, 0.0, float(r)) == a


def test_nonfinite_row_returns_last_index():
    # exp_sum is NaN: no cumsum >= r (sampler.rs:127)
    assert O.sample_with_r([0.0, float("nan"), 1.0], 1.0, 0, 1.0, 0.0, 0.5) == 2
    assert O.sample_with_r([-np.inf] * 4, 1.0, 0, 1.0, 0.0, 0.5) == 3


def test_r_zero_returns_index_zero():
    assert O.sample_with_r([-np.inf, 1.0, 2.0], 1.0, 0, 1.0, 0.0, 0.0) == 0


def test_top_p_nonpositive_keeps_unfiltered():
    x = np.array([0.0, 1.0, 2.0], np.float32)
    for r in (0.1, 0.5, 0.9):
        assert O.sample_with_r(x, 1.0, 0, 0.0, 0.0, r) == O.sample_with_r(x, 1.0, 0, 1.0, 0.0, r)


# ---------------------------------------------------------------- decode_ctrl.rs
def test_passthrough_leaves_logits_alone():  # decode_ctrl.rs:199-207
    assert not O.modifies_logits(0)
    x = [0.5, -0.5, 2.0]
    assert list(O.adjust_logits(x)) == x


def test_repeat_penalty_flips_greedy_choice():  # decode_ctrl.rs:209-222
    x = [1.0, 0.9]
    assert O.sample_with_r(O.adjust_logits(x, counts=[], repeat=2.0), 0.0) == 0
    y = O.adjust_logits(x, counts=[(0, 1)], repeat=2.0)
    assert y[0] == np.float32(0.5)
    assert O.sample_with_r(y, 0.0) == 1


def test_frequency_penalty_scales_with_count():  # decode_ctrl.rs:224-239
    y = O.adjust_logits([0.0, 1.0], counts=[(1, 2)], presence=0.1, frequency=0.3)
    assert abs(y[1] - 0.3) < 1e-6
    assert y[0] == 0.0


def test_negative_logits_penalized_away_from_zero():  # decode_ctrl.rs:241-253
    y = O.adjust_logits([-1.0, -3.0], counts=[(0, 1)], repeat=2.0)
    assert abs(y[0] - -2.0) < 1e-6


def test_logit_bias_applies_and_can_ban():  # decode_ctrl.rs:255-266
    y = O.adjust_logits([10.0, 1.0, 6.0], bias=[(0, -100.0), (2, 5.0)])
    assert O.sample_with_r(y, 0.0) == 2


def test_prompt_tail_seeds_repeat_window():  # decode_ctrl.rs:298-311
    x = [0.0] * 8
    x[7] = 1.0
    y = O.adjust_logits(x, counts=[(5, 1), (6, 1), (7, 1)], repeat=2.0)
    assert abs(y[7] - 0.5) < 1e-6


def test_bias_out_of_range_skipped_and_order_kept():
    y = O.adjust_logits([1.0, 2.0], bias=[(9, 3.0), (1, 1e8), (1, -1e8)])
    # (2 + 1e8) - 1e8 in f32 sequence, not 2 + (1e8 - 1e8)
    assert y[1] == np.float32(np.float32(2.0 + np.float32(1e8)) - np.float32(1e8))


# ---------------------------------------------------------------- logit_fsm.rs
def _fsm(dfa_fn):
    trans, dead, acc = dfa_fn()
    return O.Dfa(trans, dead, acc), O.Vocab(TINY_TOKENS, TINY_EOS)


def test_regex_masks_to_viable_prefixes():  # logit_fsm.rs:348-357
    d, v = _fsm(dfa_ab_star_c)
    x = O.apply_mask(np.zeros(6), dfa=d, vocab=v, state=0)
    assert masked(x) == [False, True, False, True, True, True]


def test_regex_advance_transitions_and_accepts():  # logit_fsm.rs:359-373
    d, v = _fsm(dfa_ab_star_c)
    s = O.advance(d, v, 0, 0)
    assert masked(O.apply_mask(np.zeros(6), dfa=d, vocab=v, state=s)) == [True, False, True, False, True, True]
    s = O.advance(d, v, s, 1)
    s = O.advance(d, v, s, 3)
    assert masked(O.apply_mask(np.zeros(6), dfa=d, vocab=v, state=s)) == [True, True, True, True, True, False]


def test_regex_multibyte_token_walks_whole_surface():  # logit_fsm.rs:375-383
    d, v = _fsm(dfa_abc)
    s = O.advance(d, v, 0, 2)
    assert masked(O.apply_mask(np.zeros(6), dfa=d, vocab=v, state=s)) == [True, True, True, False, True, True]


def test_regex_optional_suffix_allows_eos_and_continuation():  # logit_fsm.rs:385-392
    d, v = _fsm(dfa_ab_opt)
    s = O.advance(d, v, 0, 0)
    assert masked(O.apply_mask(np.zeros(6), dfa=d, vocab=v, state=s)) == [True, False, True, True, True, False]


def test_regex_constrains_a_greedy_loop_end_to_end():  # logit_fsm.rs:497-536
    d, v = _fsm(dfa_ab_plus_c)
    prefs = [[3, 1, 0, 2, 4, 5], [0, 2, 1, 3, 4, 5], [3, 1, 0, 2, 4, 5], [0, 1, 2, 3, 4, 5]]
    s, out = 0, []
    for pref in prefs:
        x = np.zeros(6, np.float32)
        for rank, i in enumerate(pref):
            x[i] = 10.0 - rank
        x = O.apply_mask(x, dfa=d, vocab=v, state=s)
        pick = max(range(6), key=lambda i: (x[i], i))  # max_by(total_cmp): last max
        if pick == 5:
            break
        out.append(pick)
        s = O.advance(d, v, s, pick)
    assert out == [0, 1, 3]


def test_ban_mode_masks_listed_tokens():  # logit_fsm.rs:457-468
    x = O.apply_mask([0.5] * 5, ban=[1, 3])
    assert list(x[[0, 2, 4]]) == [0.5] * 3 and np.isneginf(x[1]) and np.isneginf(x[3])


def test_ban_mode_out_of_range_id_ignored():  # logit_fsm.rs:481-487
    assert list(O.apply_mask([0.5] * 4, ban=[99])) == [0.5] * 4


def test_dead_end_forces_eos():  # logit_fsm.rs:244-246, 261
    d, v = _fsm(dfa_ab_star_c)
    # state 3 is the post-match non-live state: nothing viable, not accepting
    x = O.apply_mask(np.zeros(6), dfa=d, vocab=v, state=3)
    assert masked(x) == [True, True, True, True, True, False]


def test_liveness_literal_fixpoint_equals_reverse_bfs():
    rng = np.random.default_rng(0)
    for trial in range(20):
        S = int(rng.integers(2, 30))
        trans = rng.integers(0, S, size=(S, 256)).astype(np.uint32)
        # sparse graph: most bytes go to the dead state 0
        keep = rng.random((S, 256)) < 0.02
        trans = np.where(keep, trans, 0).astype(np.uint32)
        dead = np.zeros(S, np.uint8)
        dead[0] = 1
        acc = (rng.random(S) < 0.15).astype(np.uint8)
        acc[0] = 0
        d = O.Dfa(trans, dead, acc)
        # brute force: reachability from u to an accepting state
        adj = [set(int(v) for v in trans[u] if not dead[v]) for u in range(S)]
        for u in range(S):
            seen, stack = {u}, [u]
            while stack:
                a = stack.pop()
                for b in adj[a]:
                    if b not in seen:
                        seen.add(b)
                        stack.append(b)
            want = any(acc[w] for w in seen)
            assert bool(d.live[u]) == want
            assert d.is_live_literal(u) == want


def test_allowed_mask_equals_brute_force_walk():
    rng = np.random.default_rng(1)
    S = 12
    trans = rng.integers(1, S, size=(S, 256)).astype(np.uint32)
    trans[rng.random((S, 256)) < 0.3] = 0
    trans[0, :] = 0
    dead = np.zeros(S, np.uint8)
    dead[0] = 1
    acc = (rng.random(S) < 0.3).astype(np.uint8)
    acc[0] = 0
    d = O.Dfa(trans, dead, acc)
    toks = [bytes(rng.integers(97, 101, size=int(rng.integers(1, 5))).astype(np.uint8)) for _ in range(60)] + [None]
    v = O.Vocab(toks, 61)
    for s in range(S):
        allowed, anyv = O.dfa_allowed(d, v, s)
        for t, tb in enumerate(toks):
            if tb is None:
                want = False
            else:
                u, ok = s, True
                for by in tb:
                    u = int(trans[u, by])
                    if dead[u]:
                        ok = False
                        break
                want = ok and bool(d.live[u])
            assert bool(allowed[t]) == want
        assert anyv == bool(allowed.any())


# ---------------------------------------------------------------- logprobs.rs
def test_logprobs_sum_to_one_and_rank_correctly():  # logprobs.rs:61-78
    lp, ids, lps = O.logprobs_observe([2.0, 1.0, 0.0, -1.0], 1, 3)
    p = float(np.exp(lps.astype(np.float64)).sum())
    assert 0.8 < p <= 1.0 + 1e-4
    assert ids[0] == 0 and ids[1] == 1
    assert abs(lps[list(ids).index(1)] - lp) < 1e-5
    assert all(lps[i] >= lps[i + 1] for i in range(len(lps) - 1))


def test_top_n_zero_gives_chosen_only():  # logprobs.rs:80-86
    lp, ids, lps = O.logprobs_observe([0.0, 5.0], 1, 0)
    assert len(ids) == 0 and lp > -0.01


def test_masked_tokens_never_enter_top():  # logprobs.rs:88-97
    lp, ids, lps = O.logprobs_observe([1.0, -np.inf, 0.5, -np.inf], 0, 4)
    assert ids[0] == 0 and ids[1] == 2


def test_top_n_clamped_to_openai_cap():  # logprobs.rs:99-102
    lp, ids, lps = O.logprobs_observe(np.arange(64, dtype=np.float32), 0, 50)
    assert len(ids) == 20


def test_logprob_ties_keep_lower_index():
    lp, ids, lps = O.logprobs_observe([1.0, 3.0, 3.0, 2.0, 3.0], 0, 3)
    assert list(ids) == [1, 2, 4]


def test_uniform_logprob_closed_form():
    V = 1000
    lp, ids, lps = O.logprobs_observe(np.zeros(V), 5, 5)
    assert abs(lp + math.log(V)) < 1e-5
    assert list(ids) == [0, 1, 2, 3, 4]


# ---------------------------------------------------------------- hallucination.rs
def test_one_hot_is_certain():  # hallucination.rs:163-172
    l = np.zeros(64, np.float32)
    l[7] = 50.0
    H, mp, mg, clp = O.token_uncertainty(l, 7)
    assert H < 1e-3 and abs(mp - 1) < 1e-3 and abs(mg - 1) < 1e-3 and clp > -1e-3


def test_uniform_is_maximally_uncertain():  # hallucination.rs:175-183
    H, mp, mg, clp = O.token_uncertainty(np.zeros(64), 0)
    assert abs(H - math.log(64)) < 1e-3 and abs(mp - 1 / 64) < 1e-4 and mg < 1e-4


def test_sharper_distribution_is_less_risky():  # hallucination.rs:186-194
    ud = O.token_uncertainty([0.0, 0.1, 0.2, 0.0], 2)
    up = O.token_uncertainty([0.0, 0.1, 6.0, 0.0], 2)
    assert up[0] < ud[0] and up[1] > ud[1]


def test_chosen_logprob_tracks_choice():  # hallucination.rs:197-202
    assert O.token_uncertainty([3.0, 1.0, 0.0], 0)[3] > O.token_uncertainty([3.0, 1.0, 0.0], 2)[3]


def test_entropy_closed_form_two_level():
    # two values a (n1 times), b (n2 times): H = -sum p ln p exactly
    n1, n2, a, b = 10, 90, 2.0, 0.0
    x = np.array([a] * n1 + [b] * n2, np.float32)
    ea, eb = math.exp(a), math.exp(b)
    Z = n1 * ea + n2 * eb
    H = -(n1 * (ea / Z) * math.log(ea / Z) + n2 * (eb / Z) * math.log(eb / Z))
    assert abs(O.token_uncertainty(x, 0)[0] - H) < 1e-5


def test_report_aggregates_and_flags():  # hallucination.rs:205-221
    sharp = np.zeros(32, np.float32)
    sharp[1] = 40.0
    us = [O.token_uncertainty(sharp, 1), O.token_uncertainty(sharp, 1), O.token_uncertainty(np.zeros(32), 0)]
    out, peak = O.report([u[0] for u in us], [u[1] for u in us], 32)
    risk, mean_e, norm_e, risky = out
    assert abs(risky - 1 / 3) < 1e-5 and peak == 2 and 0 < risk < 1 and 0 < norm_e <= 1
    assert risk >= 0.1 and not risk >= 0.99


def test_empty_report_is_zero():  # hallucination.rs:224-231
    out, peak = O.report([], [], 0)
    assert list(out) == [0, 0, 0, 0] and peak is None


# ---------------------------------------------------------------- spec_decode.rs
def _mk(V, peak):
    v = np.zeros(V, np.float32)
    v[peak] = 10.0
    return v


def test_verify_all_accept_returns_bonus():  # spec_decode.rs:422-433
    assert O.verify_drafts([5, 7], np.stack([_mk(16, 5), _mk(16, 7), _mk(16, 9)])) == (2, 9)


def test_verify_first_mismatch_returns_corrected():  # spec_decode.rs:435-443
    assert O.verify_drafts([5, 99], np.stack([_mk(8, 5), _mk(8, 7)])) == (1, 7)


def test_argmax_first_max():  # spec_decode.rs:269-279
    assert O.argmax_first([1.0, 3.0, 3.0]) == 1
    assert O.argmax_first([-np.inf, -np.inf]) == 0
    assert O.argmax_first([float("nan"), 1.0]) == 1


# ---------------------------------------------------------------- gpu/sampling.rs, shaders.rs
def test_step_seed_and_rng01_closed_form():  # gpu/sampling.rs:9, :24-31
    assert O.step_seed(1, 2) == (1 + 2 * 0x9E3779B1) & 0xFFFFFFFF
    M = (1 << 64) - 1

    def rng01(seed):
        z = (seed * 0x9E3779B97F4A7C15 + 0x9E3779B97F4A7C15) & M
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & M
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & M
        z ^= z >> 31
        return np.float32((np.float32(z >> 40) + np.float32(0.5)) / np.float32(16777216.0))

    for s in (0, 1, 42, 0xFFFFFFFF, 123456789):
        assert O.rng01(s) == rng01(s)
        assert 0.0 < O.rng01(s) < 1.0


def test_hash_u32_closed_form():  # shaders.rs:805-811
    def h(x):
        x ^= x >> 16
        x = (x * 0x7FEB352D) & 0xFFFFFFFF
        x ^= x >> 15
        x = (x * 0x846CA68B) & 0xFFFFFFFF
        x ^= x >> 16
        return x

    for x in (0, 1, 2, 12345, 0xFFFFFFFF):
        assert O.hash_u32(x) == h(x)


def _xorshift_logits(m, V):
    # gpu/mod.rs:3853-3858
    st = 0x2545F4914F6CDD1D
    M = (1 << 64) - 1
    out = np.zeros(m * V, np.float32)
    for i in range(m * V):
        st ^= (st << 13) & M
        st ^= st >> 7
        st ^= (st << 17) & M
        out[i] = np.float32(np.float32(st >> 40) / np.float32(16777216.0)) - np.float32(0.5)
    out = out.reshape(m, V)
    out[:, 100] = np.float32(0.4999)
    out[:, 4000] = np.float32(0.4999)
    return out


def test_btopk_matches_cpu_stable_sort():  # gpu/mod.rs:3847-3880
    logits = _xorshift_logits(3, 5000)
    for s in range(3):
        vals, idxs = O.btopk(logits[s], 64)
        order = sorted(range(5000), key=lambda i: (-float(logits[s, i]), i))[:64]
        assert list(idxs) == order


def test_sample_topk_greedy_and_nucleus():  # gpu/sampling.rs:35-56
    vals = np.array([3.0, 2.0, 1.0, -4e37], np.float32)
    idxs = np.array([10, 20, 30, 40], np.uint32)
    assert O.sample_topk(vals, idxs, 0.0, 0, 1.0, 5) == 10
    # top_p tiny -> only the first survives
    for seed in range(20):
        assert O.sample_topk(vals, idxs, 1.0, 0, 0.01, seed) == 10
    # sentinel entries never sampled
    for seed in range(50):
        assert O.sample_topk(vals, idxs, 5.0, 0, 1.0, seed) in (10, 20, 30)


def _wg256_argmax(x):
    """Independent restatement of the WGSL workgroup: per-thread strided scan
    with strict >, then the stride 128..1 tree."""
    vm = [np.float32(-1e30)] * 256
    im = [0] * 256
    for t in range(256):
        for k in range(t, len(x), 256):
            if x[k] > vm[t]:
                vm[t], im[t] = x[k], k
    stride = 128
    while stride:
        for t in range(stride):
            if vm[t + stride] > vm[t]:
                vm[t], im[t] = vm[t + stride], im[t + stride]
        stride //= 2
    return im[0]


def test_bargmax_tree_tie_break():  # shaders.rs:761-789
    # equal maxima in threads 44 (id 300) and 5 (id 5): decided by the tree
    x = np.zeros(1000, np.float32)
    x[300] = 1.0
    x[5] = 1.0
    assert O.bargmax(x) == _wg256_argmax(x) == 300
    # same thread: the first index
    x = np.zeros(1000, np.float32)
    x[7] = 1.0
    x[7 + 256] = 1.0
    assert O.bargmax(x) == 7
    # values <= -1e30 never win
    assert O.bargmax(np.full(10, -2e30, np.float32)) == 0
    rng = np.random.default_rng(5)
    for _ in range(5):
        x = rng.integers(0, 4, 3000).astype(np.float32)
        assert O.bargmax(x) == _wg256_argmax(x)


def test_bsample_greedy_equals_bargmax():  # shaders.rs:822-830
    x = np.random.default_rng(0).normal(size=777).astype(np.float32)
    assert O.bsample(x, 0.0, 123) == O.bargmax(x)


# ---------------------------------------------------------------- Philox4x32-10
def test_philox_known_answers():
    # Random123 kat_vectors, philox4x32 with 10 rounds
    assert list(O.philox4x32_10([0, 0, 0, 0], [0, 0])) == [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]
    assert list(O.philox4x32_10([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2)) == [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]
    assert list(O.philox4x32_10([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0])) == \
        [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]


def test_philox_uniform_range_and_mapping():
    for c in range(100):
        u = O.philox_uniform(7, c)
        w = int(O.philox4x32_10([c, 0, 0, 0], [7, 0])[0])
        assert u == np.float32((w >> 9) * 2.0 ** -23)
        assert 0.0 <= u < 1.0


# ---------------------------------------------------------------- spec decode (rejection sampling)
def test_spec_greedy_equals_verify_drafts():  # spec_decode.rs:422-443
    t = np.stack([_mk(16, 5), _mk(16, 7), _mk(16, 9)])
    assert O.spec_verify(t, None, [5, 7], 0.0) == (2, 9)
    t = np.stack([_mk(8, 5), _mk(8, 7), _mk(8, 1)])
    assert O.spec_verify(t, np.zeros((2, 8)), [5, 99], 0.0) == (1, 7)


def test_spec_rejection_sampling_preserves_target_distribution():
    # first emitted token ~ target distribution (Leviathan et al. 2023, Thm 1)
    rng = np.random.default_rng(0)
    V = 6
    tl = np.array([[1.0, 0.2, -1.0, 2.0, 0.5, 0.0], [0.0] * 6], np.float32)
    dl = np.array([[0.0, 1.5, 0.3, -0.5, 1.0, 0.2]], np.float32)

    def weights(x):
        e = np.array([np.float32(np.exp(np.float32(v - x.max()))) for v in x], np.float64)
        return np.rint(e * 2 ** 24)

    p = weights(tl[0]) / weights(tl[0]).sum()
    q = weights(dl[0]) / weights(dl[0]).sum()
    N = 30000
    counts = np.zeros(V)
    for c in range(N):
        d = int(rng.choice(V, p=q))
        acc, nxt = O.spec_verify(tl, dl, [d], 1.0, seed=11, counter=c)
        counts[d if acc == 1 else nxt] += 1
    chi2 = (((counts - N * p) ** 2) / (N * p)).sum()
    assert chi2 < 25.0, (chi2, counts / N, p)  # 5 dof: p(chi2 > 25) ~ 1e-4


def test_spec_rejection_sampling_k3_acceptance_and_bonus():
    """k = 3 drafts: the joint law of (accepted, next) over N trials against
    its closed form (Leviathan et al. 2023, Thm 1 applied position by
    position): with a_i = sum_x min(p_i, q_i), P(accepted = j, next = x) is
    prod_{i<j} a_i * (1 - a_j) * r_j(x) for j < 3, r_j = norm(max(0, p_j - q_j)),
    and prod_i a_i * p_3(x) for the all-accepted bonus draw from row k."""
    rng = np.random.default_rng(3)
    V, k = 4, 3
    tl = np.array([[1.0, 0.2, -1.0, 2.0], [0.0, 1.0, 0.5, -0.5], [0.3, 0.3, 1.2, 0.0], [2.0, 0.0, 0.5, 1.0]],
                  np.float32)
    dl = np.array([[0.0, 1.5, 0.3, -0.5], [0.5, 0.0, 1.0, 0.2], [0.0, 0.8, 0.6, -1.0]], np.float32)

    def weights(x):
        e = np.array([np.float32(np.exp(np.float32(v - x.max()))) for v in x], np.float64)
        return np.rint(e * 2 ** 24)

    p = [weights(r) / weights(r).sum() for r in tl]
    q = [weights(r) / weights(r).sum() for r in dl]
    a = [np.minimum(p[i], q[i]).sum() for i in range(k)]
    expect = np.zeros((k + 1, V))
    reach = 1.0
    for j in range(k):
        r = np.maximum(p[j] - q[j], 0.0)
        expect[j] = reach * (1.0 - a[j]) * r / r.sum()
        reach *= a[j]
    expect[k] = reach * p[k]
    assert abs(expect.sum() - 1.0) < 1e-9
    N = 40000
    counts = np.zeros((k + 1, V))
    for c in range(N):
        drafts = [int(rng.choice(V, p=q[i])) for i in range(k)]
        acc, nxt = O.spec_verify(tl, dl, drafts, 1.0, seed=5, counter=c)
        counts[acc, nxt] += 1
    m = expect > 0
    chi2 = (((counts[m] - N * expect[m]) ** 2) / (N * expect[m])).sum()
    assert counts[~m].sum() == 0
    dof = int(m.sum()) - 1
    assert chi2 < dof + 6.0 * np.sqrt(2.0 * dof), (chi2, dof, counts / N, expect)  # ~4.2 sigma
    # per-position acceptance (the marginal of `accepted`)
    acc_emp = counts.sum(1) / N
    acc_exp = expect.sum(1)
    assert np.all(np.abs(acc_emp - acc_exp) < 5 * np.sqrt(acc_exp * (1 - acc_exp) / N) + 1e-9), (acc_emp, acc_exp)
