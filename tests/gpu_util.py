"""Shared helpers for the GPU parity tests: run a batch through libzs and the
same rows through the oracle, and compare."""
import numpy as np
import torch

from oracle import oracle as O
from zllm_amd.engine import (BatchSampler, Context, DecodeControl, LogitFSM, PenaltyConfig, RowRequest,
                             SamplerConfig)

_CTX = {}


def ctx(max_rows=64, max_vocab=151936):
    key = (max_rows, max_vocab)
    if key not in _CTX:
        _CTX[key] = Context(0, max_rows, max_vocab)
    return _CTX[key]


def make_rows(params_list):
    rows = []
    for p in params_list:
        pen = PenaltyConfig(p.get("repeat", 1.0), p.get("presence", 0.0), p.get("frequency", 0.0))
        ctrl = DecodeControl(pen, p.get("bias", ()), p.get("seed", 0))
        ctrl.counter = p.get("counter", 0)
        for t, c in p.get("counts", ()):
            ctrl.counts[int(t)] = int(c)
        fsm = None
        if p.get("ban"):
            fsm = LogitFSM(banned=p["ban"])
        rows.append(RowRequest(SamplerConfig(p.get("temperature", 1.0), p.get("top_k", 0), p.get("top_p", 1.0),
                                             p.get("min_p", 0.0)), ctrl, fsm, p.get("top_logprobs", 0)))
        rows[-1].masked = bool(p.get("masked"))
        rows[-1].logprobs = p.get("logprobs", True)
        rows[-1].detect_hallucination = p.get("detect_hallucination", True)
    return rows


def run_gpu(x, params_list, allow_bits=None, c=None):
    c = c or ctx(max(64, len(params_list)), max(151936, x.shape[1]))
    xs = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    rows = make_rows(params_list)
    bs = BatchSampler(c)
    bufs = bs.pack(xs, rows)
    ab = None
    if allow_bits is not None:
        ab = allow_bits if isinstance(allow_bits, torch.Tensor) else torch.from_numpy(
            np.ascontiguousarray(allow_bits).view(np.int32)).cuda()
    out = bs.run(xs, bufs, ab)
    torch.cuda.synchronize()
    return {k: v.cpu().numpy() for k, v in out.items()}


def bits_to_ban_mask(bits, V):
    w = np.asarray(bits).view(np.uint32)
    ok = ((w[:, None] >> np.arange(32, dtype=np.uint32)) & 1).reshape(-1)[:V].astype(bool)
    return ok


def oracle_row(x, p, allow=None):
    """Reference step for one row. `allow` (bool[V]) stands for the grammar
    mask: disallowed ids are banned before the regular ban list."""
    x = np.asarray(x, np.float32)
    ban = list(p.get("ban", ()))
    xin = x.copy()
    if allow is not None:
        xin[~allow] = -np.inf
    return O.reference_step(xin, p, ban=ban, bias=p.get("bias", ()), counts=p.get("counts", ()),
                            seed=p.get("seed", 0), counter=p.get("counter", 0))


def close(a, b, rel=1e-5, abs_=1e-5):
    a, b = float(a), float(b)
    if np.isnan(a) or np.isnan(b):
        return np.isnan(a) and np.isnan(b)
    if np.isinf(a) or np.isinf(b):
        return a == b
    return abs(a - b) <= max(abs_, rel * abs(b))


AMBIG_FRAC = 0.02   # rows whose top_logprobs ids may be compared as a set at most


def compare(x, params_list, out, allow=None, check_stats=True, refs=None):
    """Asserts bit-exact tokens and top ids; tolerance on float outputs.
    refs: the oracle's results per row when the caller computed them.

    Rows flagged ZS_ST_TOPLP_AMBIG (their top_logprobs order depends on the
    last bit of lse, so the ranking is left unchecked) are counted
    and printed; more than AMBIG_FRAC of the rows (at least one allowed) is an
    error."""
    errs = []
    n_amb = int(np.count_nonzero(np.asarray(out["status"]).view(np.uint32) & 8))
    lim = max(1, int(np.ceil(AMBIG_FRAC * len(params_list))))
    print(f"[toplp-ambig] {n_amb} of {len(params_list)} rows", flush=True)
    if n_amb > lim:
        errs.append(f"{n_amb} rows flagged ZS_ST_TOPLP_AMBIG (limit {lim})")
    for i, p in enumerate(params_list):
        ref = refs[i] if refs is not None else oracle_row(x[i], p, None if allow is None else allow[i])
        tok = int(out["token"][i]) & 0xFFFFFFFF
        st = int(out["status"][i])
        if tok != ref["token"]:
            errs.append(f"row {i}: token gpu={tok} ref={ref['token']} status={st:#x} params={ {k: v for k, v in p.items() if k != 'counts'} }")
            continue
        if not p.get("logprobs", True):
            if int(out["top_n"][i]) != 0 or not np.isnan(out["logprob"][i]):
                errs.append(f"row {i}: logprobs written although not requested")
        elif not close(out["logprob"][i], ref["logprob"]):
            errs.append(f"row {i}: logprob {out['logprob'][i]} vs {ref['logprob']}")
        n = int(out["top_n"][i])
        if not p.get("logprobs", True):
            pass
        elif n != len(ref["top_ids"]):
            errs.append(f"row {i}: top_n {n} vs {len(ref['top_ids'])}")
        elif not (st & 8):  # ZS_ST_TOPLP_AMBIG
            gi = [int(v) for v in out["top_ids"][i][:n]]
            if gi != [int(v) for v in ref["top_ids"]]:
                errs.append(f"row {i}: top ids {gi} vs {list(ref['top_ids'])}")
            for a, b in zip(out["top_lps"][i][:n], ref["top_lps"]):
                if not close(a, b):
                    errs.append(f"row {i}: top lp {a} vs {b}")
                    break
        if check_stats and not p.get("detect_hallucination", True):
            if not np.isnan(out["entropy"][i]):
                errs.append(f"row {i}: uncertainty written although not requested")
        elif check_stats:
            if not close(out["entropy"][i], ref["entropy"], 1e-5, 2e-5):
                errs.append(f"row {i}: entropy {out['entropy'][i]} vs {ref['entropy']}")
            # max_prob is 1 / S_obs on both sides (f32 division): equal bits
            # iff the observers' exact sequential sum S_obs is
            if np.float32(out["max_prob"][i]).view(np.uint32) != np.float32(ref["max_prob"]).view(np.uint32):
                errs.append(f"row {i}: max_prob {out['max_prob'][i]!r} vs {ref['max_prob']!r} (bits)")
            if not close(out["margin"][i], ref["margin"], 1e-5, 2e-6):
                errs.append(f"row {i}: margin {out['margin'][i]} vs {ref['margin']}")
            if not close(out["chosen_lp"][i], ref["chosen_lp"], 1e-5, 1e-5):
                errs.append(f"row {i}: chosen_lp {out['chosen_lp'][i]} vs {ref['chosen_lp']}")
    return errs
