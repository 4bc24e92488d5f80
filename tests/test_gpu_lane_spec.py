"""GPU parity for the batched lane (BARGMAX / BSAMPLE / BTOPK / sample_topk)
and for speculative-decode verification, against the oracle -- bit-exact ids."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.test_oracle_kat import _xorshift_logits
from zllm_amd import synth

pytestmark = pytest.mark.gpu


def _c():
    from tests.gpu_util import ctx
    return ctx()


def test_btopk_xorshift_reference_case():  # gpu/mod.rs:3847-3880
    from zllm_amd.engine import lane_topk
    print("[case] btopk xorshift m=3 V=5000", flush=True)
    x = _xorshift_logits(3, 5000)
    vals, idxs = lane_topk(_c(), torch.from_numpy(x).cuda(), 64)
    idxs = idxs.cpu().numpy().view(np.uint32)
    vals = vals.cpu().numpy()
    for s in range(3):
        ov, oi = O.btopk(x[s], 64)
        assert idxs[s].tolist() == oi.tolist()
        assert vals[s].tobytes() == ov.tobytes()


def test_btopk_edge_values():
    from zllm_amd.engine import lane_topk
    print("[case] btopk edges", flush=True)
    x = np.zeros((4, 3000), np.float32)
    x[1, :] = -np.inf
    x[1, 5:9] = [1.0, 3.5e38, -3.0e38, np.nan]
    x[2, ::3] = -0.0
    x[3] = np.random.default_rng(1).integers(0, 3, 3000).astype(np.float32)
    vals, idxs = lane_topk(_c(), torch.from_numpy(x).cuda(), 100)
    idxs = idxs.cpu().numpy().view(np.uint32)
    vals = vals.cpu().numpy()
    for s in range(4):
        ov, oi = O.btopk(x[s], 100)
        assert idxs[s].tolist() == oi.tolist(), s
        assert vals[s].tobytes() == ov.tobytes(), s


def test_bargmax_and_bsample():
    from zllm_amd.engine import lane_argmax, lane_sample
    print("[case] bargmax/bsample", flush=True)
    B, V = 16, 40000
    x = synth.logits_powerlaw(B, V, 3)
    x[0, :] = 0.0
    x[0, [300, 5, 7000]] = 2.0
    x[1, :] = -2e30
    x[2, 11] = np.nan
    x[3, :] = -np.inf            # two finite ids only
    x[3, [10, 20]] = 1.0
    x[4, 77] = np.inf
    x[5, :] = 1e33               # beyond the fast Gumbel bands: every id exact
    x[6, :] = 1.0                # only the Gumbel terms differ
    xs = torch.from_numpy(x).cuda()
    a = lane_argmax(_c(), xs).cpu().numpy()
    for s in range(B):
        assert int(a[s]) == O.bargmax(x[s]), s
    temp = np.array([0.0] + [0.5 + 0.05 * i for i in range(B - 1)], np.float32)
    seed = np.arange(B, dtype=np.uint32) * 7919 + 1
    g = lane_sample(_c(), xs, torch.from_numpy(temp).cuda(),
                    torch.from_numpy(seed.view(np.int32)).cuda()).cpu().numpy()
    for s in range(B):
        assert int(g[s]) == O.bsample(x[s], float(temp[s]), int(seed[s])), s


def test_sample_topk_on_device():
    from zllm_amd.engine import lane_sample_topk, lane_topk
    print("[case] sample_topk", flush=True)
    B, V, K = 32, 20000, 64
    x = synth.logits_powerlaw(B, V, 4)
    vals, idxs = lane_topk(_c(), torch.from_numpy(x).cuda(), K)
    rng = np.random.default_rng(4)
    temp = rng.uniform(0.0, 1.5, B).astype(np.float32)
    temp[:3] = 0.0
    topk = rng.choice([0, 5, 40, 64], B).astype(np.uint32)
    topp = rng.uniform(0.5, 1.0, B).astype(np.float32)
    seeds = np.array([O.step_seed(1234 + s, 17) for s in range(B)], np.uint32)
    out = lane_sample_topk(_c(), vals, idxs, torch.from_numpy(temp).cuda(),
                           torch.from_numpy(topk.view(np.int32)).cuda(), torch.from_numpy(topp).cuda(),
                           torch.from_numpy(seeds.view(np.int32)).cuda()).cpu().numpy().view(np.uint32)
    v_np, i_np = vals.cpu().numpy(), idxs.cpu().numpy().view(np.uint32)
    for s in range(B):
        want = O.sample_topk(v_np[s], i_np[s], float(temp[s]), int(topk[s]), float(topp[s]), int(seeds[s]))
        assert int(out[s]) == want, s


@pytest.mark.parametrize("background", [False, True])
@pytest.mark.parametrize("k,V", [(4, 3000), (4, 151936), (1, 50)])
def test_spec_verify_matches_oracle(k, V, background):
    from zllm_amd.engine import verify_drafts
    print(f"[case] spec k={k} V={V} background={background}", flush=True)
    B = 8
    rng = np.random.default_rng(k + V)
    target = synth.logits_powerlaw(B * (k + 1), V, 7).reshape(B, k + 1, V)
    draft = (target[:, :k, :] + rng.normal(0, 1.0, (B, k, V)).astype(np.float32)).astype(np.float32)
    ids = np.stack([np.argmax(draft[b], axis=1) for b in range(B)]).astype(np.uint32)
    ids[1, 0] = V + 3            # invalid draft id -> rejected
    temp = np.array([0.0, 1.0, 0.7, 1.3, 1.0, 0.9, 0.0, 2.0], np.float32)
    target[5, min(2, k), 9] = np.nan  # degenerate row -> greedy
    seeds = np.arange(B, dtype=np.uint64) + 100
    ctr = np.full(B, 3, np.uint64)
    t = lambda a, dt=None: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    acc, nxt = verify_drafts(_c(), t(target), t(ids.view(np.int32)), t(temp), t(seeds.view(np.int64)),
                             t(ctr.view(np.int64)), t(draft), background=background)
    acc, nxt = acc.cpu().numpy(), nxt.cpu().numpy().view(np.uint32)
    for b in range(B):
        want = O.spec_verify(target[b], draft[b], ids[b].tolist(), float(temp[b]), int(seeds[b]), int(ctr[b]))
        assert (int(acc[b]), int(nxt[b])) == want, (b, (acc[b], nxt[b]), want)


@pytest.mark.parametrize("mix", ["topk", "sample", "greedy"])
def test_lane_batcher_steps(mix):
    """LaneBatcher (ContinuousBatcher::step's selection, gpu/batch.rs:176-207)
    over several steps: every id equals the reference lane's choice for the
    path the batch takes (BTOPK + sample_topk, BSAMPLE or BARGMAX with
    step_seed(base, gen_index)); streams retire at eos / max_tokens."""
    from zllm_amd.engine import (ZS_LANE_ARGMAX, ZS_LANE_SAMPLE, ZS_LANE_TOPK, LaneBatcher, LaneSeq,
                                 SamplingParams)
    print(f"[case] lane batcher {mix}", flush=True)
    rng = np.random.default_rng({"topk": 1, "sample": 2, "greedy": 3}[mix])
    m, V = 24, 32000
    lb = LaneBatcher(_c())
    for i in range(m):
        if mix == "topk":
            sp = [SamplingParams(0.7, 40, 0.9), SamplingParams(1.0, 0, 0.8), SamplingParams.greedy(),
                  SamplingParams(0.5, 10, 1.0)][i % 4]
        elif mix == "sample":
            sp = SamplingParams.temperature([0.8, 0.0, 1.3][i % 3])
        else:
            sp = SamplingParams.greedy()
        lb.add(LaneSeq(i, sp, base_seed=1000 + 7 * i, eos=5, max_tokens=3 + i % 4, generated=[int(rng.integers(V))]))
    want_path = {"topk": ZS_LANE_TOPK, "sample": ZS_LANE_SAMPLE, "greedy": ZS_LANE_ARGMAX}[mix]
    for step in range(6):
        if not lb.active:
            break
        act = list(lb.active)
        x = (rng.standard_normal((len(act), V)) * 4).astype(np.float32)
        x[:, 5] = -1e9 if step < 2 else x[:, 5]  # eos only possible later
        seeds = [O.step_seed(s.base_seed, s.gen_index()) for s in act]
        res = lb.step(torch.from_numpy(x).cuda())
        assert lb.last_path == want_path
        for r, (s, (sid, tok, done)) in enumerate(zip(act, res)):
            if want_path == ZS_LANE_TOPK:
                vals, idxs = O.btopk(x[r], 64)
                want = O.sample_topk(vals, idxs, s.params.temp, s.params.top_k, s.params.top_p, seeds[r])
            elif want_path == ZS_LANE_SAMPLE:
                want = O.bsample(x[r], s.params.temp, seeds[r])
            else:
                want = O.bargmax(x[r])
            assert (sid, tok) == (s.id, want), (step, r)
            assert done == (tok == 5 or s.gen_index() >= s.max_tokens)
        assert all(not (s.generated[-1] == 5 or s.gen_index() >= s.max_tokens) for s in lb.active)
