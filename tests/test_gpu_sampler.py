"""GPU parity: zs_sample against the CPU oracle on the same seeded rows.

Tokens and top_logprobs ids must be bit-identical; logprobs / entropy /
max_prob / margin within 1e-5 relative (abs floors stated in gpu_util.close).
"""
import sys

import numpy as np
import pytest

from zllm_amd import synth

pytestmark = pytest.mark.gpu


def _run(x, params, allow_bits=None, allow=None):
    from tests.gpu_util import compare, run_gpu
    print(f"[case] B={x.shape[0]} V={x.shape[1]}", flush=True)
    out = run_gpu(x, params, allow_bits)
    errs = compare(x, params, out, allow)
    assert not errs, "\n".join(errs[:20])
    return out


def test_config1_single_row():
    x = synth.logits_c1(0)
    rng = np.random.default_rng(0)
    hist = rng.integers(0, 32000, 64)
    ids, cnt = np.unique(hist, return_counts=True)
    p = dict(temperature=0.8, top_k=40, top_p=0.95, repeat=1.1, counts=list(zip(ids.tolist(), cnt.tolist())),
             top_logprobs=5, seed=0)
    out = _run(x, [p])
    assert out["status"][0] & 4  # small path


@pytest.mark.parametrize("seed", [1, 2])
def test_mixed_rows_small_vocab(seed):
    B, V = 24, 5000
    x = synth.logits_powerlaw(B, V, seed)
    params = synth.mixed_params(B, V, seed, hist=64)
    rng = np.random.default_rng(seed)
    for i, p in enumerate(params):
        p["top_logprobs"] = int(rng.integers(0, 21))
        p["seed"] = 1000 + i
        p["counter"] = seed
        if i % 6 == 1:
            p["temperature"] = 0.0
        if i % 6 == 2:
            p["min_p"] = 0.05
        if i % 6 == 3:
            p["bias"] = [(int(rng.integers(0, V)), float(rng.normal(0, 5))) for _ in range(5)]
        if i % 6 == 4:
            p["ban"] = [int(v) for v in rng.integers(0, V, 50)]
    _run(x, params)


def test_big_rows_full_vocab():
    B, V = 6, 151936
    x = synth.logits_powerlaw(B, V, 11)
    params = [dict(temperature=t, top_k=0, top_p=tp, seed=i, top_logprobs=5)
              for i, (t, tp) in enumerate([(1.0, 1.0), (0.7, 0.9), (1.2, 0.95), (1.0, 0.8), (0.5, 0.99), (1.1, 1.0)])]
    out = _run(x, params)
    assert not any(out["status"] & 4)  # all through the big-row engine


def test_big_rows_min_p_and_flat():
    V = 20000
    x = synth.logits_normal(4, V, 5, sigma=0.3)
    params = [dict(temperature=1.0, top_k=0, top_p=0.5, min_p=0.2, seed=3),
              dict(temperature=2.0, top_k=0, top_p=0.9, seed=4),
              dict(temperature=1.0, top_k=300, top_p=0.9, seed=5),   # k beyond the candidate lists
              dict(temperature=0.9, top_k=0, top_p=1.0, min_p=0.01, seed=6)]
    _run(x, params)


def test_edge_rows():
    V = 3000
    rng = np.random.default_rng(9)
    x = rng.normal(0, 1, (8, V)).astype(np.float32)
    x[0, 17] = np.nan                      # NaN: sampler returns V-1, observers NaN
    x[1, :] = -np.inf                      # all masked
    x[2, :] = 1.0                          # all ties
    x[3, ::2] = -np.inf                    # half masked
    x[4, 100] = np.inf                     # +inf logit
    x[5, :] = np.float32(0.25)
    x[5, 7] = 3.0
    params = [dict(temperature=1.0, top_k=0, top_p=1.0, seed=1, top_logprobs=3),
              dict(temperature=1.0, top_k=10, top_p=0.9, seed=2, top_logprobs=3),
              dict(temperature=0.0, top_logprobs=4),
              dict(temperature=0.8, top_k=0, top_p=0.9, seed=3, top_logprobs=2),
              dict(temperature=1.0, top_k=5, seed=4, top_logprobs=2),
              dict(temperature=1.0, top_k=4, top_p=0.5, seed=5, top_logprobs=5),
              dict(temperature=1.0, top_k=0, top_p=0.0, seed=6),
              dict(temperature=1.0, top_k=1, seed=7, top_logprobs=1)]
    _run(x, params)


def test_allow_bits_rows():
    from oracle import oracle as O
    B, V = 8, 40000
    x = synth.logits_powerlaw(B, V, 21)
    rng = np.random.default_rng(21)
    allow = rng.random((B, V)) < np.array([0.5, 0.01, 0.001, 0.3, 1.0, 0.2, 0.0, 0.7])[:, None]
    bits = np.stack([O.pack_bits(a) for a in allow])
    params = [dict(temperature=0.9, top_k=0, top_p=0.9, seed=i, masked=True, top_logprobs=3) for i in range(B)]
    params[3]["top_k"] = 20
    params[2]["top_k"] = 100   # about 40 ids allowed: fewer than k
    params[5]["top_k"] = 3
    _run(x, params, allow_bits=bits, allow=allow)


@pytest.mark.parametrize("q", [0.5, 4.0])
def test_tied_values_topk_lists(q):
    """Quantized logits: many equal keys around each chunk's k-th value, so the
    per-chunk candidate selection runs its wave-sort, workgroup-sort and
    radix paths and the tie rule (key desc, index asc) decides membership."""
    B, V = 12, 60000
    x = np.round(synth.logits_powerlaw(B, V, 31) * q) / q
    x = x.astype(np.float32)
    rng = np.random.default_rng(31)
    params = []
    for i in range(B):
        params.append(dict(temperature=float([0.7, 1.0, 1.3][i % 3]), top_k=[20, 50, 128, 0][i % 4],
                           top_p=float([1.0, 0.9][i % 2]), seed=500 + i, top_logprobs=int(rng.integers(0, 21)),
                           detect_hallucination=bool(i % 2)))
    x[3, :] = 1.0                      # one value everywhere: every chunk ties completely
    x[7, ::3] = -np.inf                # a third masked out
    _run(x, params)


def test_unseeded_rows_draw_independently():
    """Unseeded requests (sampler.rs:26-29 draws from the thread RNG) get a
    fresh OS-entropy key each: 64 unseeded rows with identical logits draw
    independently, while rows with one explicit seed draw one token; every row
    matches the oracle under the key it was given."""
    from tests.gpu_util import compare, ctx, make_rows
    from zllm_amd.engine import BatchSampler
    import torch
    B, V = 64, 1000
    print(f"[case] unseeded B={B} V={V}", flush=True)
    x = np.zeros((B, V), np.float32)           # uniform: every draw is a fresh index
    unseeded = [dict(temperature=1.0, top_k=0, top_p=1.0, seed=None, logprobs=False,
                     detect_hallucination=False) for _ in range(B // 2)]
    seeded = [dict(temperature=1.0, top_k=0, top_p=1.0, seed=77, logprobs=False,
                   detect_hallucination=False) for _ in range(B // 2)]
    params = unseeded + seeded
    rows = make_rows(params)
    keys = [r.ctrl.seed for r in rows]
    assert len(set(keys[:B // 2])) == B // 2 and set(keys[B // 2:]) == {77}
    xs = torch.from_numpy(x).cuda()
    bs = BatchSampler(ctx())
    out = bs.run(xs, bs.pack(xs, rows))
    torch.cuda.synchronize()
    tok = out["token"].cpu().numpy().view(np.uint32)
    assert len(set(tok[:B // 2].tolist())) >= 24, tok[:B // 2]    # 32 draws from 1000 ids
    assert len(set(tok[B // 2:].tolist())) == 1
    for p, k in zip(params, keys):
        p["seed"] = k
    res = {k: v.cpu().numpy() for k, v in out.items()}
    errs = compare(x, params, res, check_stats=False)
    assert not errs, "\n".join(errs[:10])


def test_long_patch_lists_match_oracle():
    """Ban, bias and count lists of any length (decode_ctrl.rs:107-126,
    logit_fsm.rs:248-252): 6000 counted ids plus 2000 bans, a row past the
    4096-entry head the row kernel keeps on chip, and 5000 biases whose ids
    repeat (their adds happen in list order, where f32 rounding tells the
    orders apart) are sampled and observed exactly as the oracle does, and
    BatchSampler.step accepts them."""
    import torch

    from tests.gpu_util import compare, ctx, make_rows, run_gpu
    from zllm_amd.engine import BatchSampler
    B, V = 5, 32000
    print(f"[case] long patch lists B={B} V={V}", flush=True)
    rng = np.random.default_rng(7)
    x = synth.logits_powerlaw(B, V, 7)
    params = synth.mixed_params(B, V, 7, hist=64)
    for p in params:
        p["presence"], p["frequency"] = 0.3, 0.2   # counts are applied (penalties active)
        p["seed"] = 11
    ids = rng.permutation(V)
    params[1]["counts"] = [(int(t), 1 + int(t) % 3) for t in ids[:6000]]
    params[1]["ban"] = [int(t) for t in ids[6000:8000]]
    params[2]["counts"] = [(int(t), 2) for t in ids[:3096]]
    params[2]["ban"] = [int(t) for t in ids[3096:4096]]
    params[3]["counts"] = [(int(t), 1) for t in ids[:4500]]
    # 5000 biases on 1200 ids (most ids biased several times, magnitudes apart)
    bid = rng.choice(ids[4000:5200], 5000)
    params[3]["bias"] = [(int(t), float(np.float32(rng.normal(0, 4) * 10.0 ** rng.integers(-3, 2)))) for t in bid]
    params[3]["ban"] = [int(t) for t in bid[:300:7]]
    params[4]["bias"] = [(int(t), float(np.float32(rng.normal(0, 2)))) for t in ids[:4200]]
    params[4]["top_k"] = 0
    out = run_gpu(x, params)
    errs = compare(x, params, out)
    assert not errs, "\n".join(errs[:20])
    bs = BatchSampler(ctx(max(64, B), 151936))
    bs.step(torch.from_numpy(x).cuda(), make_rows(params))


def test_masked_rows_gathered_p1():
    """Masked rows with at most 2048 allowed ids take their statistics and
    lists from the gathered allowed ids; rows with fewer than 28 finite
    allowed values (the observers' list then ends with -inf ids of the whole
    row), more than 2048 allowed ids, greedy rows and NaN rows take the
    whole-row path. Bans, biases and counts on allowed and masked ids."""
    from oracle import oracle as O
    V = 30000
    rng = np.random.default_rng(41)
    x = synth.logits_powerlaw(10, V, 41)
    counts_allowed = [20, 500, 1500, 300, 2048, 2049, 100, 600, 30, 1200]
    allow = np.zeros((10, V), bool)
    for i, c in enumerate(counts_allowed):
        allow[i, rng.choice(V, c, replace=False)] = True
    ids1 = np.nonzero(allow[1])[0]
    x[1, ids1[7]] = np.nan                         # a NaN among the allowed ids
    ids8 = np.nonzero(allow[8])[0]
    x[8, ids8[:10]] = -np.inf                      # 20 finite allowed values: fewer than 28
    ids2 = np.nonzero(allow[2])[0]
    bits = np.stack([O.pack_bits(a) for a in allow])
    base = dict(temperature=0.9, top_k=0, top_p=0.95, masked=True, top_logprobs=5)
    params = [dict(base, seed=700 + i) for i in range(10)]
    params[2].update(ban=[int(v) for v in ids2[:40:3]], bias=[(int(ids2[5]), 2.5), (int(ids2[50]), -1.0), (3, 9.0)],
                     counts=[(int(v), 2) for v in ids2[100:140]], presence=0.3, frequency=0.2)
    params[3].update(temperature=0.0)
    params[4].update(top_k=50)
    params[5].update(top_k=20, top_p=0.8)
    params[6].update(top_k=200)
    params[7].update(min_p=0.05, top_p=1.0)
    params[9].update(counts=[(int(v), 1) for v in rng.choice(V, 64, replace=False)], repeat=1.3)
    _run(x, params, allow_bits=bits, allow=allow)


def test_helper_workgroups_match_one_per_row():
    """The sampler with helper workgroups (no pass_event) and with one
    workgroup per row (pass_event given) gives identical outputs."""
    import torch
    from tests.gpu_util import ctx, make_rows
    from zllm_amd.engine import BatchSampler
    B, V = 8, 151936
    x = synth.logits_powerlaw(B, V, 43)
    params = [dict(temperature=[0.7, 1.0, 1.3, 1.0][i % 4], top_k=0, top_p=[1.0, 0.9][i % 2], seed=800 + i,
                   top_logprobs=5, counts=[(i * 97 + j * 13, 1 + j % 3) for j in range(50)], presence=0.2)
              for i in range(B)]
    c = ctx(64, V)
    xs = torch.from_numpy(x).cuda()
    bs = BatchSampler(c)
    bufs = bs.pack(xs, make_rows(params))
    a = bs.run(xs, bufs)
    ev = torch.cuda.Event()
    ev.record()
    b = bs.run(xs, bufs, pass_event=ev)
    torch.cuda.synchronize()
    for k in a:
        assert np.array_equal(a[k].cpu().numpy().view(np.uint8), b[k].cpu().numpy().view(np.uint8)), k
    from tests.gpu_util import compare
    errs = compare(x, params, {k: v.cpu().numpy() for k, v in a.items()})
    assert not errs, "\n".join(errs[:20])


def test_top_logprobs_near_collisions():
    """top_logprobs ranks equal logprobs by id (logprobs.rs:41-51). Rows built
    so that many x~ map to one or two logprob values, with the boundary between
    them set by the last bits of lse: the ids must equal the oracle's in every
    row not flagged ZS_ST_TOPLP_AMBIG, and the rows must hold such ties."""
    from tests.gpu_util import compare, oracle_row, run_gpu
    rng = np.random.default_rng(7)
    B, V = 32, 8192
    x = np.full((B, V), -60.0, np.float32)
    for i in range(B):
        x[i, rng.integers(0, V)] = np.float32(30.0 + rng.normal() * 0.01)
        ids = rng.choice(V, 40, replace=False)
        base = np.float32(rng.uniform(1e-3, 2e-3))
        x[i, ids] = base + (rng.integers(0, 200, 40) * np.spacing(base)).astype(np.float32)
        x[i, rng.choice(V, 100, replace=False)] = rng.uniform(-12, -8, 100).astype(np.float32)
    params = [dict(temperature=1.0, top_k=0, top_p=1.0, top_logprobs=20, seed=i) for i in range(B)]
    for i in range(0, B, 2):   # bans among the tied ids (x~ = -inf there)
        tied_ids = np.flatnonzero((x[i] > 5e-4) & (x[i] < 5e-3))
        params[i]["ban"] = [int(v) for v in rng.choice(tied_ids, 6, replace=False)]
    refs = [oracle_row(x[i], params[i]) for i in range(B)]
    tied = sum(len(set(np.asarray(r["top_lps"]).tolist())) < len(r["top_lps"]) for r in refs)
    assert tied >= B // 2, tied
    print(f"[case] near-collision rows B={B} V={V} tied={tied}", flush=True)
    out = run_gpu(x, params)
    errs = compare(x, params, out, refs=refs)
    assert not errs, "\n".join(errs[:20])


def test_split_rows_across_halves():
    """Small batches stream each full row with two workgroups (halves of the
    row, merged by the one that finishes second): statistics, candidate lists
    and small-survivor sets that straddle the halves must merge to the
    oracle's results bit for bit."""
    B, V = 12, 151936
    mid = (V + 2047) // 2048 // 2 * 2048          # first id of the second half
    rng = np.random.default_rng(77)
    x = synth.logits_powerlaw(B, V, 77)
    x[0, mid + 5] = np.nan                        # greedy: a NaN in the second half restarts the fold there
    x[0, 10] = 40.0
    x[1, :] = -np.inf                             # 300 + 150 finite values over both halves: one small set
    x[1, rng.choice(mid, 300, replace=False)] = rng.normal(0, 2, 300)
    x[1, mid + rng.choice(V - mid, 150, replace=False)] = rng.normal(0, 2, 150)
    x[2, :] = -np.inf                             # 300 + 300: past the small-set cap
    x[2, rng.choice(mid, 300, replace=False)] = rng.normal(0, 2, 300)
    x[2, mid + rng.choice(V - mid, 300, replace=False)] = rng.normal(0, 2, 300)
    x[3, :] = -np.inf                             # fewer finite values than top_logprobs candidates
    x[3, [5, mid + 9]] = [1.0, 2.0]
    x[4, :] = 0.5                                 # equal values in both halves: ids decide
    x[5, mid:mid + 64] = 30.0                     # the top entries all in the second half
    x[6, mid - 32:mid + 32] = 25.0                # top entries across the boundary
    x[7, V - 1] = 50.0                            # the last id
    params = [dict(temperature=0.0, top_logprobs=5),
              dict(temperature=0.9, top_k=0, top_p=0.95, seed=1, top_logprobs=5),
              dict(temperature=0.9, top_k=0, top_p=0.95, seed=2, top_logprobs=5),
              dict(temperature=1.0, top_k=0, top_p=1.0, seed=3, top_logprobs=20),
              dict(temperature=1.0, top_k=20, top_p=0.9, seed=4, top_logprobs=20),
              dict(temperature=0.7, top_k=50, top_p=1.0, seed=5, top_logprobs=5),
              dict(temperature=1.2, top_k=128, top_p=0.9, seed=6, top_logprobs=10),
              dict(temperature=float("inf"), top_k=0, top_p=1.0, seed=7, top_logprobs=3),
              dict(temperature=1.0, top_k=300, top_p=0.8, seed=8, top_logprobs=5),
              dict(temperature=0.8, top_k=0, top_p=0.9, seed=9, top_logprobs=5, repeat=1.2,
                   counts=[(int(i), 2) for i in rng.choice(V, 1000, replace=False)]),
              dict(temperature=1.0, top_k=0, top_p=0.5, seed=10, top_logprobs=5, min_p=0.02),
              dict(temperature=0.0, top_logprobs=3)]
    x[11, [3, mid + 3]] = 60.0                    # greedy tie across the halves: the last one wins
    _run(x, params)
