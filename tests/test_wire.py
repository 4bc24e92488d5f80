"""OpenAI wire output (CPU): the hallucination report against the oracle's
restatement of Detector::report (hallucination.rs:101-125), and the JSON text
of hallucination_json / chat_logprobs_json / legacy_logprobs_json
(rest.rs:1494-1503, 1710-1744) against serde_json's layout, restated here in
Python: compact separators, insertion-ordered maps, f32 widened to f64 and
printed in ryu's shortest layout, non-finite as null."""
import json
import math

import numpy as np
import pytest

from oracle import oracle as O
from zllm_amd import openai as W


def ryu_f64(x: float) -> str:
    """serde_json's f64 text: shortest round-trip digits (Python's repr uses
    the same shortest digits) in ryu's layout."""
    if x == 0.0:
        return "-0.0" if math.copysign(1.0, x) < 0 else "0.0"
    sign = "-" if x < 0 else ""
    mant, _, e = ("%r" % abs(x)).partition("e")
    ip, _, fp = mant.partition(".")
    allds = ip + fp
    point = len(ip) + (int(e) if e else 0)   # decimal point position within allds
    lead = len(allds) - len(allds.lstrip("0"))
    digits = allds.strip("0")
    kk = point - lead                          # 10^(kk-1) <= v < 10^kk
    n = len(digits)
    if n <= kk <= 16:
        return sign + digits + "0" * (kk - n) + ".0"
    if 0 < kk <= 16:
        return sign + digits[:kk] + "." + digits[kk:]
    if -5 < kk <= 0:
        return sign + "0." + "0" * (-kk) + digits
    if n == 1:
        return sign + digits + "e" + str(kk - 1)
    return sign + digits[0] + "." + digits[1:] + "e" + str(kk - 1)


@pytest.mark.parametrize("x,text", [(0.5, "0.5"), (1.0, "1.0"), (100.0, "100.0"), (1e16, "1e16"),
                                    (1e15, "1000000000000000.0"), (1e-5, "0.00001"), (1e-6, "1e-6"),
                                    (-2.5e-7, "-2.5e-7"), (123.456, "123.456"), (float(np.float32(0.1)),
                                                                                "0.10000000149011612")])
def test_ryu_layout_helper(x, text):
    # the test's own restatement, pinned on values whose serde_json text is known
    assert ryu_f64(x) == text


def f32_json(v) -> str:
    v = float(np.float32(v))
    return "null" if not math.isfinite(v) else ryu_f64(v)


def serde(v) -> str:
    """serde_json::to_string of a json! value (dict insertion order)."""
    if v is None:
        return "null"
    if isinstance(v, bool):
        return "true" if v else "false"
    if isinstance(v, int):
        return str(v)
    if isinstance(v, float):
        return f32_json(v)
    if isinstance(v, str):
        out = '"'
        for ch in v:
            o = ord(ch)
            out += {'"': '\\"', "\\": "\\\\", "\b": "\\b", "\f": "\\f", "\n": "\\n", "\r": "\\r",
                    "\t": "\\t"}.get(ch, "\\u%04x" % o if o < 0x20 else ch)
        return out + '"'
    if isinstance(v, list):
        return "[" + ",".join(serde(x) for x in v) + "]"
    return "{" + ",".join(serde(k) + ":" + serde(x) for k, x in v.items()) + "}"


# ------------------------------------------------------------ report
def _report(ent, mp, vocab):
    d = W.Detector()
    d.entropy, d.max_prob, d.vocab = [float(x) for x in ent], [float(x) for x in mp], vocab
    return d.report()


@pytest.mark.parametrize("seed", range(6))
def test_report_matches_oracle(seed):
    rng = np.random.default_rng(seed)
    n = int(rng.integers(1, 300))
    ent = rng.uniform(0, 4, n).astype(np.float32)
    mp = rng.uniform(0, 1, n).astype(np.float32)
    if seed % 2:
        ent[rng.integers(0, n, 3)] = ent.max()  # ties for the peak: the last one wins
    if seed == 5:
        ent[0] = np.nan
    vocab = int(rng.integers(1, 200000))
    r = _report(ent, mp, vocab)
    want, peak = O.report(ent, mp, vocab)
    got = np.array([r.risk_score, r.mean_entropy, r.normalized_entropy, r.risky_fraction], np.float32)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)) or \
        np.array_equal(np.isnan(got), np.isnan(want))
    assert r.peak_token == peak and r.n_tokens == n


def test_empty_report_and_json():
    r = _report([], [], 0)
    assert (r.risk_score, r.n_tokens, r.peak_token) == (0.0, 0, None)
    assert r.to_json() == ('{"risk_score":0.0,"mean_entropy":0.0,"normalized_entropy":0.0,"risky_fraction":0.0,'
                           '"n_tokens":0,"peak_token_index":null,"flagged":false}')


def test_report_json_layout():
    r = _report([0.1, 3.0, 2.5], [0.95, 0.2, 0.45], 32000)
    want = serde({"risk_score": r.risk_score, "mean_entropy": r.mean_entropy,
                  "normalized_entropy": r.normalized_entropy, "risky_fraction": r.risky_fraction,
                  "n_tokens": r.n_tokens, "peak_token_index": r.peak_token, "flagged": r.flagged(0.5)})
    assert r.to_json() == want
    assert json.loads(r.to_json())["peak_token_index"] == 1
    assert r.to_json(risk_threshold=0.1).endswith('"flagged":true}')


# ------------------------------------------------------------ logprobs
class _Table:
    """Decode texts of a tiny vocabulary (what zs_token_table_text holds)."""

    def __init__(self, texts):
        b = [t.encode("utf-8") for t in texts]
        self.ntab = len(b)
        self.text_offsets = np.array([0] + list(np.cumsum([len(x) for x in b])), np.uint32)
        self.text = np.frombuffer(b"".join(b) or b"\0", np.uint8).copy()

    def decode_text(self, i):
        return "" if i >= self.ntab else bytes(self.text[self.text_offsets[i]:self.text_offsets[i + 1]]).decode()


TEXTS = ["Hello", " world", "\n", "\"q\"", "é", "�", "", "\t\x01", " world"]


def _collector():
    c = W.LogprobsCollector(5)
    c.entries = [W.TokenLogprobs(0, float(np.float32(-0.1)), [(0, float(np.float32(-0.1))), (1, -2.5), (4, -3.75)]),
                 W.TokenLogprobs(3, float(np.float32(-1e-7)), [(3, float(np.float32(-1e-7)))]),
                 W.TokenLogprobs(7, float("-inf"), [(1, -0.5), (8, -0.25), (5, -9.0), (99, -20.0)]),
                 W.TokenLogprobs(2, -1.0, [])]
    return c


def test_chat_logprobs_json():
    t = _Table(TEXTS)
    c = _collector()
    dec = t.decode_text
    want = serde({"content": [
        {"token": dec(e.token_id), "logprob": e.logprob, "bytes": list(dec(e.token_id).encode()),
         "top_logprobs": [{"token": dec(i), "logprob": lp, "bytes": list(dec(i).encode())} for i, lp in e.top]}
        for e in c.entries]})
    got = c.to_json(t, W.ZS_LOGPROBS_CHAT)
    assert got == want
    assert json.loads(got)["content"][2]["logprob"] is None  # -inf -> null


def test_legacy_logprobs_json_with_repeated_texts():
    t = _Table(TEXTS)
    c = _collector()
    dec = t.decode_text
    tops = []
    for e in c.entries:
        m = {}
        for i, lp in e.top:
            m[dec(i)] = lp  # dict: first position, last value -- serde_json's preserve_order Map
        tops.append(m)
    want = serde({"tokens": [dec(e.token_id) for e in c.entries],
                  "token_logprobs": [e.logprob for e in c.entries], "top_logprobs": tops})
    got = c.to_json(t, W.ZS_LOGPROBS_LEGACY)
    assert got == want
    assert list(json.loads(got)["top_logprobs"][2].items())[0] == (" world", -0.25)


def test_collector_from_sampler_outputs():
    # zs_sample's output layout (token, logprob, top_* with a stride, top_n)
    out = dict(token=np.array([4, 1], np.int32), logprob=np.array([-0.5, -1.5], np.float32),
               top_ids=np.array([[4, 2, 0], [1, 3, 0]], np.int32),
               top_lps=np.array([[-0.5, -1.0, 0], [-1.5, -2.0, 0]], np.float32), top_n=np.array([2, 1], np.int32))
    c = W.LogprobsCollector(3)
    c.observe_output(out, 0)
    c.observe_output(out, 1)
    assert [(e.token_id, e.logprob, e.top) for e in c.entries] == [(4, -0.5, [(4, -0.5), (2, -1.0)]),
                                                                   (1, -1.5, [(1, -1.5)])]
