"""Benchmark: one batched sampler step of the headline workload (config 5 of
BASELINE.json) on one MI355X, plus the DFA-mask time, the roofline of the
dominant kernel and the CPU baseline.

A step = zs_dfa_mask for the grammar-masked rows + zs_sample for all rows
(mask, bias/penalties, temperature, top-k/top-p, Philox draw, logprobs with
top_logprobs=5, entropy / max_prob / margin), inputs resident in HBM.

    python bench.py [--gpus 1] [--steps K] [--warmup W]
Prints one JSON line.
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--B", type=int, default=256)
    ap.add_argument("--V", type=int, default=151936)
    ap.add_argument("--dfa-states", type=int, default=512)
    ap.add_argument("--seed", type=int, default=5)
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--dfa-only", action="store_true",
                    help="only time zs_dfa_mask (cold and warm) on the DFA configs and print one JSON line")
    ap.add_argument("--copy-probe", type=int, default=0,
                    help="only copy this many MiB device-to-device (calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE) and exit")
    return ap.parse_args()


def build_workload(B, V, S, seed):
    import numpy as np
    import torch
    from zllm_amd import synth
    from zllm_amd.engine import (BatchSampler, ByteDfa, Context, DecodeControl, PenaltyConfig, RowRequest,
                                 SamplerConfig, TokenByteTable)
    ctx = Context(0, B, V)
    x = synth.logits_powerlaw(B, V, seed)
    params = synth.mixed_params(B, V, seed, hist=256)
    offs, data = synth.synthetic_vocab(V, seed)
    valid = np.ones(V, np.uint8)
    # C5's grammar: a structured (JSON-schema) automaton of about S states
    trans, dead, acc = synth.json_dfa(S, seed)
    S = trans.shape[0]
    table = TokenByteTable.from_csr(ctx, offs, data, valid, eos=V - 1)
    dfa = ByteDfa(ctx, trans, dead, acc)
    rng = np.random.default_rng(seed)
    live = [s for s in range(S) if dfa.is_live(s) and not dead[s]]
    states = np.full(B, -1, np.int32)
    masked = np.zeros(B, bool)
    masked[1::2] = True                       # 50% grammar-masked rows
    states[masked] = rng.choice(live, int(masked.sum()))
    rows = []
    for i, p in enumerate(params):
        ctrl = DecodeControl(PenaltyConfig(1.0, p["presence"], p["frequency"]), (), seed=1000 + i)
        for t, c in p["counts"]:
            ctrl.counts[int(t)] = int(c)
        rq = RowRequest(SamplerConfig(p["temperature"], p["top_k"], p["top_p"], 0.0), ctrl, None, 5)
        rq.masked = bool(masked[i])
        rq.logprobs = True
        rq.detect_hallucination = True
        rows.append(rq)
    xs = torch.from_numpy(x).cuda()
    # speculative decoding, k=4 draft positions per row: target logits at k+1
    # positions and draft logits at k, both synthetic N(0, 2) plus a peak
    # shared by draft and target so that drafts are often accepted
    g = torch.Generator(device="cuda").manual_seed(seed + 99)
    K = SPEC_K
    peak_ids = torch.randint(0, V, (B, K + 1), device="cuda", generator=g)
    tgt = torch.randn((B, K + 1, V), device="cuda", generator=g) * 2.0
    tgt.scatter_add_(2, peak_ids[:, :, None], torch.full((B, K + 1, 1), 12.0, device="cuda"))
    dft = tgt[:, :K, :] + torch.randn((B, K, V), device="cuda", generator=g) * 0.5
    dft = dft.contiguous()
    draft_ids = peak_ids[:, :K].to(torch.int32).contiguous()
    spec_T = torch.tensor([float(p["temperature"]) for p in params], dtype=torch.float32, device="cuda")
    spec_seed = torch.arange(B, dtype=torch.int64, device="cuda") + 5000
    spec_ctr = torch.zeros(B, dtype=torch.int64, device="cuda")
    sampler = BatchSampler(ctx)
    bufs = sampler.pack(xs, rows)
    st = torch.from_numpy(states).cuda()
    bits = torch.empty((B, (V + 31) // 32), dtype=torch.int32, device="cuda")
    return dict(ctx=ctx, x=x, xs=xs, params=params, rows=rows, sampler=sampler, bufs=bufs, dfa=dfa, table=table,
                states=states, st=st, bits=bits, masked=masked, trans=trans, dead=dead, acc=acc, offs=offs,
                data=data, valid=valid, tgt=tgt, dft=dft, draft_ids=draft_ids, spec_T=spec_T, spec_seed=spec_seed,
                spec_ctr=spec_ctr)


def algorithmic_bytes_per_row(V, H, masked):
    # 4V logits + 4H count-map (ids+counts = 8 per entry, H distinct) + allow
    # bitset for masked rows + outputs (token 4, chosen lp 4, top-5 8*5, stats 12)
    b = 4 * V + 8 * H + 4 + 4 + 8 * 5 + 12
    if masked:
        b += 4 * ((V + 31) // 32)
    return b


SPEC_K = 4
# HBM bytes per launch of the C5 batch's dispatches, measured with rocprofv3
# --pmc FETCH_SIZE / WRITE_SIZE and scaled by the copy-kernel calibration
# (profiles/c5_kernels_counters.md, the tree of the commit that added it)
TRAFFIC = {"zs_k_spec_chunk": 1402.4e6, "zs_k_row": 107.8e6, "zs_k_sapx1": 26.6e6, "zs_k_sround1": 30.1e6,
           "zs_k_sapx2": 87.1e6, "zs_k_sround2": 97.2e6, "zs_k_sround3": 97.5e6, "zs_k_pv": 64.1e6,
           "zs_k_tp_inc": 36.4e6, "zs_k_big": 0.6e6}


def spec_bytes_per_row(V, k):
    # target logits at k+1 positions + draft logits at k positions + ids/outputs
    return 4 * V * (2 * k + 1) + 4 * k + 8


def lane_step_us(ctx, xs, params):
    """Mean time of one zs_lane_step over the C5 batch for each lane path:
    top-64 pool + nucleus (the C5 knobs), Gumbel sampling (temperatures
    only) and argmax (greedy)."""
    import ctypes as C
    import torch
    from zllm_amd._lib import LaneStream, lib
    B, V = xs.shape
    out = torch.empty(B, dtype=torch.int32, device="cuda")
    stream = torch.cuda.current_stream()
    res = {}
    for name in ("topk", "sample", "argmax"):
        st = (LaneStream * B)()
        for i, p in enumerate(params):
            st[i].temp = 0.0 if name == "argmax" else p["temperature"]
            st[i].top_k = p["top_k"] if name == "topk" else 0
            st[i].top_p = p["top_p"] if name == "topk" else 1.0
            st[i].base_seed, st[i].gen_index = 1000 + i, 3
        path = C.c_int()

        def call():
            rc = lib().zs_lane_step(ctx.h, xs.data_ptr(), B, V, xs.stride(0), st, out.data_ptr(), C.byref(path),
                                    stream.cuda_stream)
            assert rc == 0
        for _ in range(3):
            call()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(20):
            call()
        e1.record(stream)
        torch.cuda.synchronize()
        res[name] = round(e0.elapsed_time(e1) / 20 * 1000.0, 2)
    return res


def mask_config_us(ctx, V, rows, kind, S, seed):
    """Mean time of zs_dfa_mask over `rows` constrained rows (random current
    states) for one DFA config; synthetic vocabulary as in config C3."""
    import numpy as np
    import torch
    from zllm_amd import synth
    from zllm_amd.engine import ByteDfa, TokenByteTable
    offs, data = synth.synthetic_vocab(V, seed + S)
    table = TokenByteTable.from_csr(ctx, offs, data, np.ones(V, np.uint8), eos=V - 1)
    if kind == "random":
        trans, dead, acc = synth.random_dfa(S, seed + S, dead_rate=0.3)
    elif kind == "compiled":
        # the `json:` grammar (any JSON value, depth 5) through the native compiler
        from zllm_amd import grammar as G
        g = G.HostDfa(G.any_json_regex_default())
        trans, dead, acc = g.trans, g.dead, g.accept
    else:
        trans, dead, acc = synth.json_dfa(S, seed + S)
    dfa = ByteDfa(ctx, trans, dead, acc)
    rng = np.random.default_rng(seed + S + 1)
    live = [s for s in range(trans.shape[0]) if dfa.is_live(s) and not dead[s]]
    st = torch.tensor(rng.choice(live, rows).astype(np.int32), device="cuda")
    bits = torch.empty((rows, (V + 31) // 32), dtype=torch.int32, device="cuda")
    return mask_cold_warm_us(dfa, table, st, V, bits)


def mask_cold_warm_us(dfa, table, st, V, bits, iters=20):
    """(cold, warm) mean us of zs_dfa_mask: cold with the per-state memo
    dropped before every call (every row walked), warm with it filled (every
    row a memo hit, as when the rows revisit states, logit_fsm.rs:166-182)."""
    import torch
    stream = torch.cuda.current_stream()
    res = []
    for cold in (True, False):
        for _ in range(3):
            if cold:
                dfa.memo_clear()
            dfa.mask(table, st, V, out=bits)
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(iters):
            if cold:
                dfa.memo_clear()
            dfa.mask(table, st, V, out=bits)
        e1.record(stream)
        torch.cuda.synchronize()
        res.append(e0.elapsed_time(e1) / iters * 1000.0)
    return tuple(res)


def cpu_baseline(W, seconds, cores):
    """Oracle (C restatement of the reference, one row per thread) on a bounded
    sample of the same rows: rows/s."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    from oracle import oracle as O
    V = W["x"].shape[1]
    tokens = [bytes(W["data"][W["offs"][t]:W["offs"][t + 1]]) for t in range(V)]
    ov = O.Vocab(tokens, V - 1)
    od = O.Dfa(W["trans"], W["dead"], W["acc"])

    def one(i):
        p = dict(W["params"][i])
        p["top_logprobs"] = 5
        st = int(W["states"][i])
        return O.reference_step(W["x"][i], p, counts=p["counts"], dfa=od if st >= 0 else None,
                                vocab=ov if st >= 0 else None, state=st, seed=1000 + i, counter=0)["token"]

    done = 0
    t0 = time.time()
    with ThreadPoolExecutor(cores) as ex:
        i = 0
        while time.time() - t0 < seconds and i < 4 * len(W["params"]):
            batch = [(i + j) % len(W["params"]) for j in range(cores)]
            list(ex.map(one, batch))
            i += cores
            done += len(batch)
    el = time.time() - t0
    return done / el, done


def cpu_model():
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def build_config(ctx, name, seed):
    """Inputs of BASELINE.json configs 1-4 (the sampler part; C3 / C4 with
    their grammar masks): dict(x, rows, params, bits, dfa, table, states,
    masked, hist)."""
    import numpy as np
    import torch
    from zllm_amd import synth
    from zllm_amd.engine import (ByteDfa, DecodeControl, LogitFSM, PenaltyConfig, RowRequest, SamplerConfig,
                                 TokenByteTable)
    rng = np.random.default_rng(seed + 101)
    C = {"name": name, "dfa": None, "table": None, "states": None}
    if name == "c1":
        x = synth.logits_c1(0)
        V = x.shape[1]
        hist = rng.integers(0, V, 64)
        ids, cnt = np.unique(hist, return_counts=True)
        params = [dict(temperature=0.8, top_k=40, top_p=0.95, min_p=0.0, repeat=1.1, presence=0.0, frequency=0.0,
                       counts=list(zip(ids.tolist(), cnt.tolist())))]
    elif name == "c2":
        B, V = 64, 128256
        x = synth.logits_powerlaw(B, V, 2)
        params = synth.mixed_params(B, V, 2, hist=256)
    elif name == "c3":
        B, V = 32, 128256
        x = synth.logits_powerlaw(B, V, 3)
        params = [dict(temperature=1.0, top_k=0, top_p=1.0, min_p=0.0, repeat=1.0, presence=0.0, frequency=0.0,
                       counts=[]) for _ in range(B)]
        trans, dead, acc = synth.random_dfa(64, seed + 64, dead_rate=0.3)
    else:   # c4
        B, V = 128, 151936
        x = synth.logits_powerlaw(B, V, 4)
        params = [dict(temperature=0.7, top_k=0, top_p=0.9, min_p=0.0, repeat=1.0, presence=0.0, frequency=0.0,
                       counts=[], ban=[int(t) for t in rng.choice(V, 500, replace=False)]) for _ in range(B)]
        trans, dead, acc = synth.json_dfa(2048, seed + 2048)
    B, V = x.shape
    if name in ("c3", "c4"):
        offs, data = synth.synthetic_vocab(V, seed + V)
        C["table"] = TokenByteTable.from_csr(ctx, offs, data, np.ones(V, np.uint8), eos=V - 1)
        C["dfa"] = ByteDfa(ctx, trans, dead, acc)
        live = [q for q in range(trans.shape[0]) if C["dfa"].is_live(q) and not dead[q]]
        C["states"] = torch.tensor(rng.choice(live, B).astype(np.int32), device="cuda")
        C["trans"], C["dead"], C["acc"], C["offs"], C["data"] = trans, dead, acc, offs, data
    rows = []
    for i, p in enumerate(params):
        ctrl = DecodeControl(PenaltyConfig(p["repeat"], p["presence"], p["frequency"]), (), seed=900 + i)
        for t, c in p["counts"]:
            ctrl.counts[int(t)] = int(c)
        fsm = LogitFSM(banned=p["ban"]) if p.get("ban") else None
        rq = RowRequest(SamplerConfig(p["temperature"], p["top_k"], p["top_p"], p["min_p"]), ctrl, fsm, 5)
        rq.masked = C["dfa"] is not None
        rq.logprobs = True
        rq.detect_hallucination = True
        rows.append(rq)
    C.update(x=x, xs=torch.from_numpy(x).cuda(), params=params, rows=rows,
             bits=torch.zeros((B, (V + 31) // 32), dtype=torch.int32, device="cuda"),
             hist=[len(p["counts"]) + len(p.get("ban", ())) for p in params])
    return C


def config_measure(ctx, C, iters=20):
    """GPU: sampler us per step over the config's batch (the grammar mask
    separately), rows/s and the sampler's HBM fraction."""
    import torch
    from zllm_amd.engine import BatchSampler
    xs, bits = C["xs"], C["bits"]
    B, V = xs.shape
    sampler = BatchSampler(ctx)
    bufs = sampler.pack(xs, C["rows"], bits if C["dfa"] is not None else None)
    ab = bits if C["dfa"] is not None else None
    if C["dfa"] is not None:
        C["dfa"].mask(C["table"], C["states"], V, out=bits)
    out = None
    for _ in range(3):
        out = sampler.run(xs, bufs, ab, top_stride=5, out=out)
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(iters):
        out = sampler.run(xs, bufs, ab, top_stride=5, out=out)
    e1.record(stream)
    torch.cuda.synchronize()
    us = e0.elapsed_time(e1) / iters * 1000.0
    res = {"B": B, "V": V, "sampler_us": round(us, 2), "rows_per_s": round(B / (us * 1e-6), 1)}
    masked = C["dfa"] is not None
    nbytes = sum(algorithmic_bytes_per_row(V, C["hist"][i], masked) for i in range(B))
    res["sampler_hbm_frac"] = round(nbytes / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)
    if masked:
        cold, warm = mask_cold_warm_us(C["dfa"], C["table"], C["states"], V, bits, iters)
        res["mask_us"], res["mask_warm_us"] = round(cold, 2), round(warm, 2)
    res["toplp_ambig_rows"] = int(((out["status"].cpu().numpy().view("uint32") & 8) != 0).sum())
    return res


def config_cpu(C, seconds, cores):
    """CPU oracle on the same rows: rows/s on one core and on `cores` threads
    (bounded samples of about `seconds` each), and for grammar configs the
    CPU mask per row: cold (the DFA walk over every token) and warm (the
    per-state memo of logit_fsm.rs:166-182 hit: the cached mask applied)."""
    import numpy as np
    from concurrent.futures import ThreadPoolExecutor
    from oracle import oracle as O
    x = C["x"]
    B, V = x.shape
    od = ov = None
    st = None
    if C["dfa"] is not None:
        ov = O.Vocab([bytes(C["data"][C["offs"][t]:C["offs"][t + 1]]) for t in range(V)], V - 1)
        od = O.Dfa(C["trans"], C["dead"], C["acc"])
        st = C["states"].cpu().numpy()

    def one(i):
        p = dict(C["params"][i % B])
        p["top_logprobs"] = 5
        return O.reference_step(x[i % B], p, ban=p.get("ban", ()), counts=p["counts"], dfa=od,
                                vocab=ov, state=int(st[i % B]) if st is not None else -1, seed=900 + i,
                                counter=0)["token"]

    res = {}
    for n in (1, cores):
        done, t0 = 0, time.time()
        with ThreadPoolExecutor(n) as ex:
            while time.time() - t0 < seconds / 2 and done < 8 * B:
                list(ex.map(one, range(done, done + n)))
                done += n
        res[f"rows_per_s_{n}core" if n == 1 else "rows_per_s_ncore"] = round(done / (time.time() - t0), 2)
    if od is not None:
        t0 = time.time()
        k = 0
        cache = {}
        while time.time() - t0 < seconds / 4 and k < B:
            allowed, _ = O.dfa_allowed(od, ov, int(st[k]))
            cache[int(st[k])] = allowed.astype(bool)
            k += 1
        cold = (time.time() - t0) / k
        t0 = time.time()
        for j in range(k):
            xm = x[j].copy()
            xm[~cache[int(st[j])]] = -np.inf
        warm = (time.time() - t0) / k
        res["mask_cold_ms_per_row"] = round(cold * 1e3, 3)
        res["mask_warm_ms_per_row"] = round(warm * 1e3, 3)
    return res


def copy_probe(mib):
    """A plain device copy of known size: its FETCH_SIZE / WRITE_SIZE per
    dispatch against mib * 1024 KiB gives the counter scale."""
    import torch
    n = mib * (1 << 20) // 4
    src = torch.ones(n, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_probe_mib": mib}))


def make_step(W, V):
    """The timed step over workload W: DFA mask of the grammar rows, the
    sampler over all rows, draft verification. Returns (step, spec_stream);
    step(out=None, overlap=True) -> (sampler outputs, (accepted, next)).

    The draft verification is independent of this step's sampling: it runs on
    a second stream (default priority) from the point where the sampler's
    kernels begin (zs_batch.pass_event). The sampler's row kernel holds one
    workgroup per row and its rows finish at different times; the
    verification fills the CUs that frees. The step ends when both are done."""
    import torch
    from zllm_amd.engine import verify_drafts
    ctx, sampler, bufs, xs, bits = W["ctx"], W["sampler"], W["bufs"], W["xs"], W["bits"]
    stream = torch.cuda.current_stream()
    spec_stream = torch.cuda.Stream()
    pass_ev = torch.cuda.Event()
    pass_ev.record(stream)  # creates the event

    def step(out=None, overlap=True):
        if overlap:
            spec_stream.wait_stream(stream)
        W["dfa"].memo_clear()   # every step walks every grammar row (the memo's cold path)
        W["dfa"].mask(W["table"], W["st"], V, out=bits)
        out = sampler.run(xs, bufs, bits, top_stride=5, out=out, pass_event=pass_ev if overlap else None)
        bufs["counter"].add_(1)
        if overlap:
            with torch.cuda.stream(spec_stream):
                spec_stream.wait_event(pass_ev)
                spec = verify_drafts(ctx, W["tgt"], W["draft_ids"], W["spec_T"], W["spec_seed"], W["spec_ctr"],
                                     W["dft"])
                W["spec_ctr"].add_(1)
            stream.wait_stream(spec_stream)
        else:
            spec = verify_drafts(ctx, W["tgt"], W["draft_ids"], W["spec_T"], W["spec_seed"], W["spec_ctr"], W["dft"])
            W["spec_ctr"].add_(1)
        return out, spec

    return step, spec_stream


DFA_CONFIGS = [("c5_json512", 151936, 128, "json", 512), ("c4_json2048", 151936, 128, "json", 2048),
               ("c3_random64", 128256, 32, "random", 64), ("json_any_compiled", 151936, 128, "compiled", 0)]


def dfa_only(seed):
    """zs_dfa_mask alone over the DFA configs (in this order: 23 cold calls,
    then 23 warm calls each): {config: [cold us, warm us]}."""
    from zllm_amd.engine import Context
    ctx = Context(0, 256, 151936)
    res = {name: [round(v, 2) for v in mask_config_us(ctx, V, rows, kind, S, seed)]
           for name, V, rows, kind, S in DFA_CONFIGS}
    print(json.dumps({"dfa_mask_us_cold_warm": res}), flush=True)
    ctx.close()


def main():
    args = parse()
    if args.copy_probe:
        copy_probe(args.copy_probe)
        return
    if args.gpus != 1:
        print(json.dumps({"error": "this build targets one GPU: run with --gpus 1 (sharding is design-only)"}))
        sys.exit(2)
    if args.dfa_only:
        dfa_only(args.seed)
        return
    import numpy as np
    import torch
    B, V = args.B, args.V
    W = build_workload(B, V, args.dfa_states, args.seed)
    ctx, xs, bits = W["ctx"], W["xs"], W["bits"]
    stream = torch.cuda.current_stream()

    from zllm_amd.engine import verify_drafts

    step, spec_stream = make_step(W, V)

    out = None
    for _ in range(args.warmup):
        out, _ = step(out)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(stream)
    for _ in range(args.steps):
        out, _ = step(out)
    e1.record(stream)
    torch.cuda.synchronize()
    ms_step = e0.elapsed_time(e1) / args.steps

    # the step's DFA mask alone (C5: 128 grammar rows of 256), cold and warm
    us_mask, us_mask_warm = mask_cold_warm_us(W["dfa"], W["table"], W["st"], V, bits)
    # DFA-mask configs C3 (64-state random DFA, 32 rows, V=128256) and C4
    # (JSON-schema DFA of 2048 states, 128 rows, V=151936), untimed loops
    dfa_cfg = {"c5_json512": None, "c3_random64": mask_config_us(ctx, 128256, 32, "random", 64, args.seed),
               "c4_json2048": mask_config_us(ctx, 151936, 128, "json", 2048, args.seed)}

    dfa_cfg["json_any_compiled"] = mask_config_us(ctx, 151936, 128, "compiled", 0, args.seed)
    lane_us = lane_step_us(ctx, xs, W["params"])

    # spec verify alone (separate, untimed loop)
    s0, s1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s0.record(stream)
    for _ in range(10):
        verify_drafts(ctx, W["tgt"], W["draft_ids"], W["spec_T"], W["spec_seed"], W["spec_ctr"], W["dft"])
    s1.record(stream)
    torch.cuda.synchronize()
    us_spec = s0.elapsed_time(s1) / 10 * 1000.0

    # DFA mask alone and per-kernel timings of zs_sample (separate, untimed loops)
    ctx.set_profiling(True)
    acc = {}
    n_prof = 10
    for _ in range(n_prof):
        out, _ = step(out, overlap=False)  # one stream: events bracket single kernels
        for k, v in ctx.last_timings().items():
            acc[k] = acc.get(k, 0.0) + v / n_prof
    ctx.set_profiling(False)
    torch.cuda.synchronize()

    status = out["status"].cpu().numpy()
    H = [len(p["counts"]) for p in W["params"]]
    row_bytes = [algorithmic_bytes_per_row(V, H[i], W["masked"][i]) for i in range(B)]
    step_bytes = float(sum(row_bytes)) + B * spec_bytes_per_row(V, SPEC_K)
    dom = max(acc, key=acc.get)
    dom_ms = acc[dom]
    # algorithmic bytes of one launch of the dominant kernel: the rows it
    # processes times their per-row bytes (the logits it must read at least once)
    big_rows = [i for i in range(B) if not (status[i] & (1 | 2 | 4))]  # not greedy / non-finite / small
    per_kernel_bytes = {
        "zs_k_row": float(sum(row_bytes)),
        "zs_k_big": float(sum(row_bytes[i] for i in big_rows)),
        "zs_k_pv": float(sum(4 * V + 4 * V for i in big_rows)),   # read logits, write p
        "zs_k_spec_chunk": float(B * 4 * V * (2 * SPEC_K + 1)),
    }
    # the row sums read every unmasked row's logits once per pass and a masked
    # row's gathered allowed values (x~ and y)
    nb = bits.cpu().numpy().view(np.uint32)
    allowed = [int(np.unpackbits(nb[i].view(np.uint8)).sum()) if W["masked"][i] else 0 for i in range(B)]
    sum_bytes = float(sum(4 * V if not W["masked"][i] else 8 * allowed[i] for i in range(B)))
    for k in ("zs_k_sapx2", "zs_k_sround2", "zs_k_sround3"):   # every row's terms (sapx1, sround1: big rows only)
        per_kernel_bytes[k] = sum_bytes
    dom_bytes = per_kernel_bytes.get(dom, step_bytes)
    achieved = dom_bytes / (dom_ms * 1e-3) / 1e9
    # the sampler chain alone (one stream): every sampler kernel's time, against
    # the bytes every row must read once
    samp_ms = sum(v for k, v in acc.items() if not k.startswith("zs_k_spec") and not k.startswith("zs_k_dfa"))
    samp_bytes = float(sum(row_bytes))
    samp_gbs = samp_bytes / (samp_ms * 1e-3) / 1e9
    ambig = int(((status.view("uint32") & 8) != 0).sum())
    cores = min(16, len(os.sched_getaffinity(0)))
    configs = {}
    for name in ("c1", "c2", "c3", "c4"):
        Cf = build_config(ctx, name, args.seed)
        configs[name] = config_measure(ctx, Cf)
        if not args.no_cpu:
            configs[name]["cpu"] = config_cpu(Cf, args.cpu_seconds / 4, cores)
        del Cf
    cpu = None
    if not args.no_cpu:
        cores = min(16, len(os.sched_getaffinity(0)))
        rps, nrows = cpu_baseline(W, args.cpu_seconds, cores)
        cpu = {"value": round(rps, 2), "unit": "rows/s", "cores": cores, "kind": "port",
               "sample": f"{nrows} rows of the same C5 batch through the C oracle "
                         f"(mask + adjust + sample + logprobs + entropy), one row per thread"}
    res = {
        "metric": "sampler rows/s @B=256,V=151936 fp32; % HBM peak; DFA-mask us/step",
        "value": round(B / (ms_step * 1e-3), 1),
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (seeded power-law logits, synthetic vocab, 512-state JSON-schema DFA, spec-decode logits)",
        "config": {"workload": "C5 full continuous-batching sampler step", "B": B, "V": V,
                   "masked_rows": int(W["masked"].sum()), "dfa_states": args.dfa_states, "top_logprobs": 5,
                   "entropy": True, "spec_k": SPEC_K},
        "step_hbm_frac": round(step_bytes / (ms_step * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
        "dfa_mask_us": round(us_mask, 2),
        "dfa_mask_us_configs": {"c5_json512": round(us_mask, 2),
                                **{k: round(v[0], 2) for k, v in dfa_cfg.items() if v is not None}},
        "dfa_mask_warm_us_configs": {"c5_json512": round(us_mask_warm, 2),
                                     **{k: round(v[1], 2) for k, v in dfa_cfg.items() if v is not None}},
        "spec_verify_us": round(us_spec, 2),
        "lane_step_us": lane_us,
        "kernel_ms": {k: round(v, 4) for k, v in acc.items()},
        "roofline": {"bound": "hbm", "kernel": dom, "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": TRAFFIC.get(dom),
                     "algorithmic_bytes": dom_bytes, "ms": round(dom_ms, 4)},
        "roofline_kernels": {k: {"ms": round(acc[k], 4), "algorithmic_bytes": per_kernel_bytes[k],
                                 "achieved": round(per_kernel_bytes[k] / (acc[k] * 1e-3) / 1e9, 1),
                                 "frac": round(per_kernel_bytes[k] / (acc[k] * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                                 "traffic": TRAFFIC.get(k)}
                             for k in ("zs_k_row", "zs_k_sapx2", "zs_k_sround2", "zs_k_sround3", "zs_k_pv")
                             if k in acc and k in per_kernel_bytes},
        "roofline_sampler": {"bound": "hbm", "kernels": "zs_sample (all its kernels, one stream)",
                             "achieved": round(samp_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                             "frac": round(samp_gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": samp_bytes,
                             "ms": round(samp_ms, 4)},
        "toplp_ambig_rows": ambig,
        "configs": configs,
        "cpu_model": cpu_model(),
        "cpu_baseline": cpu,
    }
    print(json.dumps(res), flush=True)
    # release the device objects before the interpreter shuts down
    torch.cuda.synchronize()
    ctx.close()


if __name__ == "__main__":
    main()
