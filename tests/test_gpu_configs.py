"""GPU parity at the full sizes of BASELINE.json's configs 2 and 5.

Config 5 is the bench workload itself (bench.build_workload / make_step, one
overlapped step): every one of the 256 rows' sampler outputs against the
oracle's reference_step with the same grammar state, every masked row's allow
bitset against the oracle's apply_mask (logit_fsm.rs:247-270), and every row's
draft verification against the oracle's spec_verify. Config 2: B=64 rows of
V=128256 with the mixed per-row knobs. Tokens, top ids and bitsets bit-exact;
float outputs within the tolerances of gpu_util.compare (1e-5 relative)."""
import os
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from zllm_amd import synth

pytestmark = pytest.mark.gpu

# the oracle's C calls release the GIL: rows in parallel on the host's cores
WORKERS = min(16, os.cpu_count() or 1)


def test_config2_full_size():
    from tests.gpu_util import compare, run_gpu
    B, V = 64, 128256
    print(f"[case] config 2 B={B} V={V}", flush=True)
    x = synth.logits_powerlaw(B, V, 2)
    params = synth.mixed_params(B, V, 2, hist=256)
    for i, p in enumerate(params):
        p["top_logprobs"] = 5
        p["seed"] = 300 + i
    out = run_gpu(x, params)
    from tests.gpu_util import oracle_row
    with ThreadPoolExecutor(WORKERS) as ex:
        refs = list(ex.map(lambda i: oracle_row(x[i], params[i]), range(B)))
    errs = compare(x, params, out, refs=refs)
    assert not errs, "\n".join(errs[:20])


def test_config5_bench_step():
    import torch

    import bench
    from oracle import oracle as O
    from tests.gpu_util import compare
    B, V, S = 256, 151936, 512
    print(f"[case] config 5 bench step B={B} V={V} dfa={S}", flush=True)
    W = bench.build_workload(B, V, S, 5)
    step, _ = bench.make_step(W, V)
    out, (acc, nxt) = step()
    torch.cuda.synchronize()
    out = {k: v.cpu().numpy() for k, v in out.items()}
    bits = W["bits"].cpu().numpy().view(np.uint32)
    acc, nxt = acc.cpu().numpy(), nxt.cpu().numpy().view(np.uint32)

    tokens = [bytes(W["data"][W["offs"][t]:W["offs"][t + 1]]) for t in range(V)]
    ov = O.Vocab(tokens, V - 1)
    od = O.Dfa(W["trans"], W["dead"], W["acc"])
    states = W["states"]
    params = []
    for i, p in enumerate(W["params"]):
        q = dict(p)
        q["top_logprobs"] = 5
        q["seed"] = 1000 + i
        params.append(q)

    def ref_row(i):
        st = int(states[i])
        p = params[i]
        return O.reference_step(W["x"][i], p, counts=p["counts"], dfa=od if st >= 0 else None,
                                vocab=ov if st >= 0 else None, state=st, seed=p["seed"], counter=0)

    def ref_bits(i):
        return O.mask_bits(V, dfa=od, vocab=ov, state=int(states[i]))

    tgt, dft = W["tgt"].cpu().numpy(), W["dft"].cpu().numpy()
    ids = W["draft_ids"].cpu().numpy().view(np.uint32)
    temp = W["spec_T"].cpu().numpy()

    def ref_spec(b):
        return O.spec_verify(tgt[b], dft[b], ids[b].tolist(), float(temp[b]), 5000 + b, 0)

    masked_rows = [i for i in range(B) if states[i] >= 0]
    with ThreadPoolExecutor(WORKERS) as ex:
        refs = list(ex.map(ref_row, range(B)))
        rbits = list(ex.map(ref_bits, masked_rows))
        rspec = list(ex.map(ref_spec, range(B)))
    assert len(masked_rows) == B // 2
    bad = [i for i, rb in zip(masked_rows, rbits) if not np.array_equal(bits[i], rb)]
    assert not bad, f"allow bitsets differ on rows {bad[:10]}"
    errs = compare(W["x"], params, out, refs=refs)
    assert not errs, "\n".join(errs[:20])
    got = [(int(acc[b]), int(nxt[b])) for b in range(B)]
    bad = [(b, got[b], rspec[b]) for b in range(B) if got[b] != rspec[b]]
    assert not bad, bad[:10]
    # the workload exercises acceptance, rejection and the bonus draw
    assert len({a for a, _ in got}) > 1


def _grammar_case(V, trans, dead, acc, nrows, seed):
    """Synthetic vocabulary of V tokens, GPU allow bitsets from random live
    states, and the oracle's bitsets for the same states."""
    import torch

    from oracle import oracle as O
    from tests.gpu_util import ctx
    from zllm_amd.engine import ByteDfa, TokenByteTable
    c = ctx(max(64, nrows), 151936)
    offs, data = synth.synthetic_vocab(V, seed)
    table = TokenByteTable.from_csr(c, offs, data, np.ones(V, np.uint8), eos=V - 1)
    dfa = ByteDfa(c, trans, dead, acc)
    rng = np.random.default_rng(seed)
    live = [s for s in range(trans.shape[0]) if dfa.is_live(s) and not dead[s]]
    states = rng.choice(live, nrows).astype(np.int32)
    bits = dfa.mask(table, torch.tensor(states, device="cuda"), V)
    torch.cuda.synchronize()
    got = bits.cpu().numpy().view(np.uint32)
    ov = O.Vocab([bytes(data[offs[t]:offs[t + 1]]) for t in range(V)], V - 1)
    od = O.Dfa(trans, dead, acc)
    with ThreadPoolExecutor(WORKERS) as ex:
        want = list(ex.map(lambda s: O.mask_bits(V, dfa=od, vocab=ov, state=int(s)), states))
    bad = [i for i in range(nrows) if not np.array_equal(got[i], want[i])]
    assert not bad, f"allow bitsets differ on rows {bad[:10]} (states {states[bad[:10]]})"
    allow = np.stack([np.unpackbits(w.view(np.uint8), bitorder="little")[:V].astype(bool) for w in want])
    return got, allow


def _sample_masked(x, params, bits, allow):
    from tests.gpu_util import compare, oracle_row, run_gpu
    out = run_gpu(x, params, allow_bits=bits)
    with ThreadPoolExecutor(WORKERS) as ex:
        refs = list(ex.map(lambda i: oracle_row(x[i], params[i], allow[i]), range(len(params))))
    errs = compare(x, params, out, allow, refs=refs)
    assert not errs, "\n".join(errs[:20])


def test_config3_regex_mask_and_sample():
    B, V = 32, 128256
    print(f"[case] config 3 B={B} V={V} dfa=64", flush=True)
    trans, dead, acc = synth.random_dfa(64, 3, dead_rate=0.3)
    bits, allow = _grammar_case(V, trans, dead, acc, B, 3)
    x = synth.logits_powerlaw(B, V, 3)
    params = [dict(temperature=1.0, top_k=0, top_p=1.0, seed=700 + i, masked=True, top_logprobs=5) for i in range(B)]
    _sample_masked(x, params, bits, allow)


def test_config4_json_schema_mask_ban_and_sample():
    B, V = 128, 151936
    print(f"[case] config 4 B={B} V={V} dfa=2048", flush=True)
    trans, dead, acc = synth.json_dfa(2048, 4)
    bits, allow = _grammar_case(V, trans, dead, acc, B, 4)
    x = synth.logits_powerlaw(B, V, 4)
    rng = np.random.default_rng(4)
    params = [dict(temperature=0.7, top_k=0, top_p=0.9, seed=900 + i, masked=True, top_logprobs=5,
                   ban=[int(v) for v in rng.choice(V, 500, replace=False)]) for i in range(B)]
    _sample_masked(x, params, bits, allow)
