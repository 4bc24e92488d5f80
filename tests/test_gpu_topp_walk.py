"""GPU parity of the top-p walk (sampler.rs:91-104) at full vocabulary size,
on rows chosen for the walk's cases: the bucket-total walk (bucket totals,
presorted candidate buckets resolved by prefix searches or one addition at a
time), its fallback to the workgroup walk, stops inside runs of equal
probabilities, top_p near 0 and 1, and grammar-masked rows. Tokens must equal
the oracle's (restated reference) bit for bit.
"""
import numpy as np
import pytest

from zllm_amd import synth

pytestmark = pytest.mark.gpu

V = 151936


def _run(x, params, allow_bits=None, allow=None):
    from tests.gpu_util import compare, run_gpu
    print(f"[case] B={x.shape[0]} V={x.shape[1]} top_p={[p['top_p'] for p in params]}", flush=True)
    out = run_gpu(x, params, allow_bits)
    errs = compare(x, params, out, allow)
    assert not errs, "\n".join(errs[:20])
    return out


def test_walk_spread_of_temperatures():
    """N(0, 2) logits over a range of temperatures and top_p: the running sum
    crosses many binades, at bucket edges and inside candidate buckets."""
    B = 12
    x = synth.logits_normal(B, V, 41, sigma=2.0)
    rng = np.random.default_rng(41)
    params = [dict(temperature=float(rng.uniform(0.8, 1.6)), top_k=0, top_p=float(rng.uniform(0.3, 0.995)),
                   seed=900 + i, top_logprobs=5) for i in range(B)]
    out = _run(x, params)
    assert not any(out["status"] & 4)  # every row through the big-row engine


@pytest.mark.parametrize("q", [4.0, 64.0])
def test_walk_equal_probabilities(q):
    """Quantised logits: probabilities repeat exactly, so the stop falls inside
    a run of equal values (its rank decides the kept set in index order) and
    half-way increments (ties) occur in the bucket totals."""
    B = 8
    x = (np.round(synth.logits_normal(B, V, 43, sigma=1.5) * q) / q).astype(np.float32)
    params = [dict(temperature=1.0, top_k=0, top_p=tp, seed=70 + i, top_logprobs=3)
              for i, tp in enumerate([0.5, 0.9, 0.99, 0.75, 0.3, 0.95, 0.6, 0.85])]
    _run(x, params)


def test_walk_flat_rows():
    """Nearly uniform rows: the largest bucket holds too many values to be
    presorted, so the row falls back to the workgroup walk; and a row whose
    sum reaches top_p only near the end of the vocabulary."""
    x = synth.logits_normal(4, V, 47, sigma=0.02)
    x[1] = np.float32(0.5)              # one value everywhere
    params = [dict(temperature=1.0, top_k=0, top_p=0.3, seed=1),
              dict(temperature=1.0, top_k=0, top_p=0.7, seed=2),
              dict(temperature=1.0, top_k=0, top_p=0.9999, seed=3),
              dict(temperature=0.9, top_k=0, top_p=0.05, seed=4)]
    _run(x, params)


def test_walk_extreme_top_p():
    """top_p just above the largest probability (the walk stops after a few
    values), tiny top_p (the peak alone), and top_p close to 1."""
    x = synth.logits_powerlaw(6, V, 53)
    params = [dict(temperature=1.2, top_k=0, top_p=tp, seed=10 + i, top_logprobs=5)
              for i, tp in enumerate([0.001, 0.02, 0.5, 0.999, 0.99999, 0.9])]
    _run(x, params)


def test_walk_masked_rows():
    """Grammar-masked big rows (allow bits): the walk sees only allowed ids."""
    from oracle import oracle as O
    B = 6
    x = synth.logits_normal(B, V, 59, sigma=2.0)
    rng = np.random.default_rng(59)
    allow = rng.random((B, V)) < np.array([0.9, 0.5, 0.2, 0.05, 0.7, 0.35])[:, None]
    bits = np.stack([O.pack_bits(a) for a in allow])
    params = [dict(temperature=float(t), top_k=0, top_p=float(tp), seed=30 + i, masked=True, top_logprobs=2)
              for i, (t, tp) in enumerate([(1.0, 0.9), (1.3, 0.8), (0.9, 0.95), (1.1, 0.99), (1.5, 0.7), (1.0, 0.6)])]
    _run(x, params, allow_bits=bits, allow=allow)
