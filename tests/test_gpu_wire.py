"""GPU: the OpenAI wire objects fed from zs_sample's outputs over a short
generation equal the same objects fed from the oracle's per-step results
(tokens and top ids exact; logprobs / entropy within the sampler's 1e-5
relative bar)."""
import json

import numpy as np
import pytest

from tests.gpu_util import close, oracle_row, run_gpu
from zllm_amd import openai as W

pytestmark = pytest.mark.gpu


class _Texts:
    def __init__(self, V):
        b = [("t%d" % i).encode() for i in range(V)]
        self.ntab = V
        self.text_offsets = np.array([0] + list(np.cumsum([len(x) for x in b])), np.uint32)
        self.text = np.frombuffer(b"".join(b), np.uint8).copy()


def test_wire_objects_from_sampler_outputs():
    print("[case] wire objects over 6 steps", flush=True)
    V, steps = 4096, 6
    rng = np.random.default_rng(11)
    p = dict(temperature=0.8, top_k=40, top_p=0.9, top_logprobs=5, seed=77)
    gl, gd = W.LogprobsCollector(5), W.Detector()
    ol, od = W.LogprobsCollector(5), W.Detector()
    for s in range(steps):
        x = (rng.standard_normal((1, V)) * 3).astype(np.float32)
        q = dict(p, counter=s)
        out = run_gpu(x, [q])
        gl.observe_output(out, 0)
        gd.observe_output(out, 0, V)
        ref = oracle_row(x[0], q)
        tok = ref["token"]
        assert int(out["token"][0]) == tok
        ol.entries.append(W.TokenLogprobs(tok, float(ref["logprob"]),
                                          [(int(i), float(v)) for i, v in zip(ref["top_ids"], ref["top_lps"])]))
        od.entropy.append(float(ref["entropy"]))
        od.max_prob.append(float(ref["max_prob"]))
        od.vocab = V
    t = _Texts(V)
    for kind in (W.ZS_LOGPROBS_CHAT, W.ZS_LOGPROBS_LEGACY):
        g, o = json.loads(gl.to_json(t, kind)), json.loads(ol.to_json(t, kind))
        if kind == W.ZS_LOGPROBS_CHAT:
            for a, b in zip(g["content"], o["content"]):
                assert a["token"] == b["token"] and a["bytes"] == b["bytes"]
                assert close(a["logprob"], b["logprob"])
                assert [x["token"] for x in a["top_logprobs"]] == [x["token"] for x in b["top_logprobs"]]
                assert all(close(x["logprob"], y["logprob"]) for x, y in zip(a["top_logprobs"], b["top_logprobs"]))
        else:
            assert g["tokens"] == o["tokens"]
            assert all(close(a, b) for a, b in zip(g["token_logprobs"], o["token_logprobs"]))
            assert [list(m) for m in g["top_logprobs"]] == [list(m) for m in o["top_logprobs"]]
    rg, ro = json.loads(gd.report().to_json()), json.loads(od.report().to_json())
    assert rg["n_tokens"] == ro["n_tokens"] == steps and rg["flagged"] == ro["flagged"]
    for k in ("risk_score", "mean_entropy", "normalized_entropy", "risky_fraction"):
        assert close(rg[k], ro[k]), k
