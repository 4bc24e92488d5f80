"""OpenAI wire output fed from the sampler's per-token outputs (host side):
LogprobsCollector (logprobs.rs:20-31) and Detector (hallucination.rs:77-125)
accumulate zs_sample's per-row outputs step by step; the JSON views are
produced by libzs (chat_logprobs_json / legacy_logprobs_json,
rest.rs:1710-1744; hallucination_json, rest.rs:1494-1503) with serde_json's
text layout."""
import ctypes as C
from dataclasses import dataclass, field
from typing import List, Optional, Tuple

import numpy as np

from ._lib import ZS_ELIMIT, HallucReport, lib

ZS_LOGPROBS_CHAT = 0
ZS_LOGPROBS_LEGACY = 1


def _string_call(fn, *args):
    need = C.c_size_t(0)
    cap = 1 << 14
    while True:
        buf = C.create_string_buffer(cap)
        rc = fn(*args, buf, cap, C.byref(need))
        if rc == ZS_ELIMIT and need.value > cap:
            cap = need.value
            continue
        if rc != 0:
            raise ValueError(f"libzs error {rc}")
        return buf.value.decode("utf-8")


@dataclass
class TokenLogprobs:  # logprobs.rs:10-17
    token_id: int
    logprob: float
    top: List[Tuple[int, float]] = field(default_factory=list)


class LogprobsCollector:
    """logprobs.rs:20-31; fed with zs_sample outputs instead of full logits."""

    def __init__(self, top_n: int):
        self.top_n = min(int(top_n), 20)
        self.entries: List[TokenLogprobs] = []

    def observe_output(self, out: dict, row: int):
        """Append row `row` of a zs_sample output dict (host arrays or tensors)."""
        g = {k: (v.cpu().numpy() if hasattr(v, "cpu") else np.asarray(v)) for k, v in out.items()
             if k in ("token", "logprob", "top_ids", "top_lps", "top_n")}
        n = min(int(g["top_n"][row]), self.top_n)
        top = [(int(np.uint32(g["top_ids"][row, k])), float(np.float32(g["top_lps"][row, k]))) for k in range(n)]
        self.entries.append(TokenLogprobs(int(np.uint32(g["token"][row])), float(np.float32(g["logprob"][row])),
                                          top))

    def _arrays(self):
        n = len(self.entries)
        stride = max([len(e.top) for e in self.entries] + [1])
        ids = np.array([e.token_id for e in self.entries] or [0], np.uint32)
        lps = np.array([e.logprob for e in self.entries] or [0], np.float32)
        cnt = np.array([len(e.top) for e in self.entries] or [0], np.uint32)
        tids = np.zeros((max(n, 1), stride), np.uint32)
        tlps = np.zeros((max(n, 1), stride), np.float32)
        for i, e in enumerate(self.entries):
            for k, (t, lp) in enumerate(e.top):
                tids[i, k], tlps[i, k] = t, lp
        return n, ids, lps, cnt, stride, tids, tlps

    def to_json(self, table, kind: int = ZS_LOGPROBS_CHAT) -> str:
        """chat (ZS_LOGPROBS_CHAT) or legacy completions logprobs object;
        `table` is a zllm_amd.vocab.HostTokenTable (its decode texts)."""
        n, ids, lps, cnt, stride, tids, tlps = self._arrays()
        return _string_call(lib().zs_logprobs_json, kind, n, ids.ctypes.data, lps.ctypes.data, cnt.ctypes.data,
                            stride, tids.ctypes.data, tlps.ctypes.data, table.text_offsets.ctypes.data,
                            table.text.ctypes.data if table.text.size else None, table.ntab)


@dataclass
class HallucinationReport:  # hallucination.rs:54-67 (summary fields)
    risk_score: float
    mean_entropy: float
    normalized_entropy: float
    risky_fraction: float
    peak_token: Optional[int]
    n_tokens: int
    _c: HallucReport = None

    def flagged(self, risk_threshold: float) -> bool:
        return self.risk_score >= risk_threshold

    def to_json(self, risk_threshold: float = 0.5) -> str:
        """hallucination_json (rest.rs:1494-1503)."""
        return _string_call(lib().zs_hallucination_json, C.byref(self._c), risk_threshold)


class Detector:
    """hallucination.rs:77-125 over zs_sample's per-token entropy / max_prob."""

    def __init__(self, entropy_threshold: float = 2.0, max_prob_threshold: float = 0.4):
        self.entropy_threshold = entropy_threshold
        self.max_prob_threshold = max_prob_threshold
        self.vocab = 0
        self.entropy: List[float] = []
        self.max_prob: List[float] = []

    def observe_output(self, out: dict, row: int, vocab: int):
        e = out["entropy"][row]
        m = out["max_prob"][row]
        self.entropy.append(float(e.item() if hasattr(e, "item") else e))
        self.max_prob.append(float(m.item() if hasattr(m, "item") else m))
        self.vocab = int(vocab)

    def is_empty(self) -> bool:
        return not self.entropy

    def report(self) -> HallucinationReport:
        e = np.array(self.entropy or [0], np.float32)
        m = np.array(self.max_prob or [0], np.float32)
        r = HallucReport()
        rc = lib().zs_hallucination_report(e.ctypes.data, m.ctypes.data, len(self.entropy), self.vocab,
                                           self.entropy_threshold, self.max_prob_threshold, C.byref(r))
        if rc != 0:
            raise ValueError(f"zs_hallucination_report: {rc}")
        return HallucinationReport(r.risk_score, r.mean_entropy, r.normalized_entropy, r.risky_fraction,
                                   None if r.peak_token < 0 else int(r.peak_token), int(r.n_tokens), r)
