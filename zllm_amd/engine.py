"""Host-side mirror of the reference engine interface over libzs.

Names follow src/engine/: SamplerConfig (sampler.rs:3-22), PenaltyConfig and
DecodeControl (decode_ctrl.rs:21-153), TokenByteTable / LogitFSM
(logit_fsm.rs:33-323). The batched entry point `sample_batch` replaces the
per-request `apply_mask -> sample_token -> observe` sequence of
rest.rs:2594-2624 for B rows at once on the GPU.

torch is used only for device memory and the stream; every computation runs
in libzs's HIP kernels.
"""
import ctypes as C
import sys
import weakref
import secrets
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Sequence, Tuple

import numpy as np
import torch

from ._lib import (Batch, LaneStream, RowParams, SpecBatch, ZS_OK, ZS_ROW_LOGPROBS, ZS_ROW_MASKED, ZS_ROW_UNCERTAINTY,
                   ZS_SPEC_BACKGROUND, ZsError, lib)

OPENAI_TOP_LOGPROBS_CAP = 20  # logprobs.rs:27-29


def _check(ctx_handle, rc, what):
    if rc != ZS_OK:
        msg = lib().zs_last_error(ctx_handle)
        raise ZsError(f"{what} failed ({rc}): {msg.decode() if msg else ''}")


def _finalizing() -> bool:
    """True during interpreter shutdown: destructors then leave device
    objects to the process exit instead of calling into the HIP runtime,
    which torch may already have begun to tear down."""
    return sys is None or sys.is_finalizing()


class Context:
    """One libzs context (device scratch sized for max_rows x max_vocab).

    close() releases the vocabularies and DFAs created on it, then the
    context; callers that own a context call it when done (the destructor
    does the same outside interpreter shutdown)."""

    def __init__(self, device: int = 0, max_rows: int = 256, max_vocab: int = 151936):
        self.device = device
        self.max_rows = max_rows
        self.max_vocab = max_vocab
        self._children = weakref.WeakSet()
        h = C.c_void_p()
        rc = lib().zs_ctx_create(device, max_rows, max_vocab, C.byref(h))
        if rc != ZS_OK:
            raise ZsError(f"zs_ctx_create failed ({rc})")
        self.h = h

    def _adopt(self, obj) -> None:
        self._children.add(obj)

    def close(self):
        if self.h:
            for child in list(self._children):
                child.close()
            lib().zs_ctx_destroy(self.h)
            self.h = None

    def set_profiling(self, on: bool):
        _check(self.h, lib().zs_set_profiling(self.h, 1 if on else 0), "zs_set_profiling")

    def last_timings(self) -> Dict[str, float]:
        """Per-kernel durations (ms) of the last zs_sample and zs_spec_verify
        calls (profiling on)."""
        names = (C.c_char_p * 32)()
        ms = (C.c_float * 32)()
        n = lib().zs_last_timings(self.h, names, ms, 32)
        if n < 0:
            _check(self.h, n, "zs_last_timings")
        return {names[i].decode(): float(ms[i]) for i in range(n)}

    def __del__(self):
        if _finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


@dataclass
class SamplerConfig:
    """sampler.rs:3-22 (defaults as there)."""
    temperature: float = 1.0
    top_k: int = 50
    top_p: float = 0.9
    min_p: float = 0.0


@dataclass
class PenaltyConfig:
    """decode_ctrl.rs:21-43."""
    repeat: float = 1.0
    presence: float = 0.0
    frequency: float = 0.0

    def is_active(self) -> bool:
        return self.repeat != 1.0 or self.presence != 0.0 or self.frequency != 0.0


class DecodeControl:
    """decode_ctrl.rs:45-153: penalties, logit_bias, the per-request RNG and the
    count map. The RNG is Philox4x32-10 keyed by `seed` with a per-step counter
    (the reference uses StdRng). Without a seed the reference draws from the
    thread RNG (sampler.rs:26-29, decode_ctrl.rs:73); here an unseeded request
    gets a fresh 64-bit key from the OS entropy source, so unseeded requests
    (and rows) draw independently of each other."""

    def __init__(self, penalties: Optional[PenaltyConfig] = None, logit_bias: Sequence[Tuple[int, float]] = (),
                 seed: Optional[int] = None):
        self.penalties = penalties or PenaltyConfig()
        self.logit_bias = [(int(t), float(b)) for t, b in logit_bias]
        self.counts: Dict[int, int] = {}
        self.seeded = seed is not None
        self.seed = secrets.randbits(64) if seed is None else int(seed) & (2**64 - 1)
        self.counter = 0

    def observe_prompt_tail(self, prompt: Sequence[int], last_n: int):  # decode_ctrl.rs:90-97
        if not self.penalties.is_active():
            return
        for t in list(prompt)[::-1][:last_n]:
            self.counts[int(t)] = self.counts.get(int(t), 0) + 1

    def modifies_logits(self) -> bool:  # decode_ctrl.rs:102-104
        return self.penalties.is_active() or bool(self.logit_bias)

    def observe(self, token: int):  # decode_ctrl.rs:149-153
        if self.penalties.is_active():
            self.counts[int(token)] = self.counts.get(int(token), 0) + 1


class TokenByteTable:
    """logit_fsm.rs:43-46: per-token surface bytes (None = never allowed under a
    grammar) and the EOS id, uploaded once per model."""

    def __init__(self, ctx: Context, tokens: Sequence[Optional[bytes]], eos: int):
        self.ctx = ctx
        self.ntab = len(tokens)
        self.eos = int(eos)
        offs = np.zeros(self.ntab + 1, np.uint32)
        valid = np.zeros(max(self.ntab, 1), np.uint8)
        buf = bytearray()
        for i, t in enumerate(tokens):
            if t is not None:
                valid[i] = 1
                buf += t
            offs[i + 1] = len(buf)
        data = np.frombuffer(bytes(buf) or b"\0", np.uint8).copy()
        h = C.c_void_p()
        rc = lib().zs_vocab_create(ctx.h, offs.ctypes.data, data.ctypes.data, valid.ctypes.data, self.ntab,
                                   self.eos, C.byref(h))
        _check(ctx.h, rc, "zs_vocab_create")
        self.h = h
        ctx._adopt(self)

    @classmethod
    def from_host_table(cls, ctx, host, eos=None):
        """Upload a zllm_amd.vocab.HostTokenTable (tokenizer.json / GGUF vocab);
        eos defaults to its eos_token_id (rest.rs:1331 refuses a grammar
        without one)."""
        eos = host.eos if eos is None else eos
        if eos is None:
            raise ValueError("tokenizer has no EOS token; regex grammar unavailable")
        return cls.from_csr(ctx, host.offsets, host.data if host.data.size else np.zeros(1, np.uint8), host.valid,
                            eos)

    @classmethod
    def from_csr(cls, ctx, offsets, data, valid, eos):
        obj = cls.__new__(cls)
        obj.ctx = ctx
        obj.ntab = len(offsets) - 1
        obj.eos = int(eos)
        offs = np.ascontiguousarray(offsets, np.uint32)
        data = np.ascontiguousarray(data, np.uint8)
        if data.size == 0:
            data = np.zeros(1, np.uint8)
        valid = np.ascontiguousarray(valid, np.uint8)
        h = C.c_void_p()
        rc = lib().zs_vocab_create(ctx.h, offs.ctypes.data, data.ctypes.data, valid.ctypes.data, obj.ntab,
                                   obj.eos, C.byref(h))
        _check(ctx.h, rc, "zs_vocab_create")
        obj.h = h
        ctx._adopt(obj)
        return obj

    def close(self):
        if getattr(self, "h", None):
            lib().zs_vocab_destroy(self.h)
            self.h = None

    def __del__(self):
        if _finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


class ByteDfa:
    """A built anchored byte DFA (the table regex-automata would produce):
    trans[S,256], dead/quit flags, accept = is_match(next_eoi_state(s))."""

    def __init__(self, ctx: Context, trans, dead, accept):
        self.ctx = ctx
        trans = np.ascontiguousarray(trans, np.uint32).reshape(-1)
        self.nstates = trans.size // 256
        dead = np.ascontiguousarray(dead, np.uint8)
        accept = np.ascontiguousarray(accept, np.uint8)
        h = C.c_void_p()
        rc = lib().zs_dfa_create(ctx.h, trans.ctypes.data, self.nstates, dead.ctypes.data, accept.ctypes.data,
                                 C.byref(h))
        _check(ctx.h, rc, "zs_dfa_create")
        self.h = h
        ctx._adopt(self)

    def close(self):
        if getattr(self, "h", None):
            lib().zs_dfa_destroy(self.h)
            self.h = None

    @property
    def table_form(self) -> str:
        """The table form the mask walk uses: "packed", "sparse", "displaced"
        (staged in LDS) or "l2" (past the LDS budget)."""
        return ("packed", "sparse", "displaced", "l2")[lib().zs_dfa_table_form(self.h)]

    def is_live(self, s: int) -> bool:
        return bool(lib().zs_dfa_is_live(self.h, s))

    def is_accept(self, s: int) -> bool:
        return bool(lib().zs_dfa_is_accept(self.h, s))

    def advance(self, table: TokenByteTable, state: int, token: int) -> Tuple[int, bool]:
        out = C.c_uint32()
        viable = C.c_int()
        rc = lib().zs_dfa_advance(self.h, table.h, state, token, C.byref(out), C.byref(viable))
        _check(self.ctx.h, rc, "zs_dfa_advance")
        return int(out.value), bool(viable.value)

    def mask(self, table: TokenByteTable, states: torch.Tensor, V: int, out: Optional[torch.Tensor] = None,
             any_out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Allow bitsets for rows at `states` (int32 device tensor, -1 = free)."""
        B = states.numel()
        words = (V + 31) // 32
        if out is None:
            out = torch.empty((B, words), dtype=torch.int32, device=states.device)
        stream = torch.cuda.current_stream(states.device).cuda_stream
        rc = lib().zs_dfa_mask(self.ctx.h, self.h, table.h, states.data_ptr(), B, V, out.data_ptr(),
                               any_out.data_ptr() if any_out is not None else None, stream)
        _check(self.ctx.h, rc, "zs_dfa_mask")
        return out

    def memo_clear(self) -> None:
        """Drop the memoised per-state bitsets: the next mask() walks every row."""
        lib().zs_dfa_memo_clear(self.h)

    def __del__(self):
        if _finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


class LogitFSM:
    """logit_fsm.rs:33-37: either a `ban:` list or a byte-DFA constraint with
    its current state. `compile` builds the DFA of `regex:`, `json_schema:`
    and `json:` grammars with the native compiler (zllm_amd.grammar) and
    uploads it to the table's context."""

    def __init__(self, banned: Sequence[int] = (), dfa: Optional[ByteDfa] = None,
                 table: Optional[TokenByteTable] = None, state: int = 0):
        self.banned = [int(b) for b in banned]
        self.dfa = dfa
        self.table = table
        self.state = state

    @classmethod
    def compile(cls, grammar: str, table: Optional[TokenByteTable] = None):  # logit_fsm.rs:190-228
        g = grammar.strip()
        if g.startswith("ban:"):
            banned = []
            for piece in g[4:].split(","):
                piece = piece.strip()
                if piece.isdigit() and int(piece) < 2**32:
                    banned.append(int(piece))
            return cls(banned=banned)
        if g == "":
            return cls()
        from . import grammar as G
        if g.startswith("regex:"):
            if table is None:
                raise G.GrammarError("regex grammar needs a tokenizer byte table")
            pattern = g[len("regex:"):]
        elif g.startswith("json_schema:"):
            if table is None:
                raise G.GrammarError("json_schema grammar needs a tokenizer byte table")
            pattern = G.schema_to_regex(g[len("json_schema:"):].strip())
        elif g.startswith("json:"):
            if table is None:
                raise G.GrammarError("json grammar needs a tokenizer byte table")
            pattern = G.any_json_regex_default()
        else:
            mode = next((m for m in ("regex", "json_schema", "json", "bnf") if g.startswith(m + ":")), "unknown")
            raise G.GrammarError(f'grammar mode "{mode}" is not implemented yet; supported: "ban:<id>,<id>,...", '
                                 '"regex:<pattern>", "json_schema:<schema>", "json:"')
        host = G.HostDfa(pattern)
        dfa = ByteDfa(table.ctx, host.trans, host.dead, host.accept)
        return cls(dfa=dfa, table=table, state=host.start)

    def is_active(self) -> bool:  # logit_fsm.rs:299-301
        return bool(self.banned) or self.dfa is not None

    def advance(self, token: int):  # logit_fsm.rs:275-290
        if self.dfa is not None:
            self.state, _ = self.dfa.advance(self.table, self.state, token)


@dataclass
class RowRequest:
    """One row of a batched step: sampler knobs + per-request state."""
    config: SamplerConfig = field(default_factory=SamplerConfig)
    ctrl: DecodeControl = field(default_factory=DecodeControl)
    fsm: Optional[LogitFSM] = None
    top_logprobs: int = 0
    masked: bool = False  # apply the row's allow bitset (set automatically for a DFA constraint)
    logprobs: bool = False              # OpenAI `logprobs` (LogprobsCollector, logprobs.rs)
    detect_hallucination: bool = False  # token_uncertainty (hallucination.rs)


class StepOutput:
    def __init__(self, **kw):
        self.__dict__.update(kw)


class BatchSampler:
    """Packs B requests into the zs_batch layout and runs zs_sample."""

    def __init__(self, ctx: Context, device="cuda"):
        self.ctx = ctx
        self.device = torch.device(device)

    @staticmethod
    def _csr(lists, dtype):
        off = np.zeros(len(lists) + 1, np.uint32)
        for i, l in enumerate(lists):
            off[i + 1] = off[i] + len(l)
        flat = np.concatenate([np.asarray(l, dtype) for l in lists]) if off[-1] else np.zeros(1, dtype)
        return off, flat

    def pack(self, logits: torch.Tensor, rows: List[RowRequest], allow_bits: Optional[torch.Tensor] = None):
        B, V = logits.shape
        dev = logits.device
        params = (RowParams * B)()
        cnt_ids, cnt_vals, bias_ids, bias_vals, bans = [], [], [], [], []
        seeds = np.zeros(B, np.uint64)
        counters = np.zeros(B, np.uint64)
        for i, rq in enumerate(rows):
            c, p = rq.config, rq.ctrl.penalties
            masked = rq.masked or (rq.fsm is not None and rq.fsm.dfa is not None)
            flags = (ZS_ROW_MASKED if masked else 0) | (ZS_ROW_LOGPROBS if (rq.logprobs or rq.top_logprobs) else 0) \
                | (ZS_ROW_UNCERTAINTY if rq.detect_hallucination else 0)
            params[i] = RowParams(c.temperature, c.top_k, c.top_p, c.min_p, p.repeat, p.presence, p.frequency,
                                  min(rq.top_logprobs, OPENAI_TOP_LOGPROBS_CAP), flags, 0)
            items = list(rq.ctrl.counts.items()) if p.is_active() else []
            cnt_ids.append([t for t, _ in items])
            cnt_vals.append([n for _, n in items])
            bias_ids.append([t for t, _ in rq.ctrl.logit_bias])
            bias_vals.append([b for _, b in rq.ctrl.logit_bias])
            bans.append(rq.fsm.banned if rq.fsm is not None else [])
            seeds[i] = rq.ctrl.seed
            counters[i] = rq.ctrl.counter
        t = lambda a, dt: torch.from_numpy(np.ascontiguousarray(a)).to(dev, dtype=dt) if a is not None else None
        co, ci = self._csr(cnt_ids, np.uint32)
        _, cv = self._csr(cnt_vals, np.uint32)
        bo, bi = self._csr(bias_ids, np.uint32)
        _, bv = self._csr(bias_vals, np.float32)
        no, ni = self._csr(bans, np.uint32)
        bufs = dict(
            params=torch.frombuffer(bytearray(params), dtype=torch.uint8).to(dev),
            cnt_off=t(co.view(np.int32), torch.int32), cnt_ids=t(ci.view(np.int32), torch.int32),
            cnt_vals=t(cv.view(np.int32), torch.int32),
            bias_off=t(bo.view(np.int32), torch.int32), bias_ids=t(bi.view(np.int32), torch.int32),
            bias_vals=t(bv, torch.float32),
            ban_off=t(no.view(np.int32), torch.int32), ban_ids=t(ni.view(np.int32), torch.int32),
            seed=t(seeds.view(np.int64), torch.int64), counter=t(counters.view(np.int64), torch.int64),
        )
        return bufs

    def run(self, logits: torch.Tensor, bufs: dict, allow_bits: Optional[torch.Tensor] = None,
            top_stride: int = OPENAI_TOP_LOGPROBS_CAP, out: Optional[dict] = None,
            pass_event: Optional[torch.cuda.Event] = None):
        """pass_event (optional, already recorded once so that it exists) is
        recorded where the sampler's kernels begin (zs_batch.pass_event)."""
        B, V = logits.shape
        dev = logits.device
        assert logits.dtype == torch.float32 and logits.stride(1) == 1
        if out is None:
            out = dict(
                token=torch.empty(B, dtype=torch.int32, device=dev),
                logprob=torch.empty(B, dtype=torch.float32, device=dev),
                top_ids=torch.zeros((B, top_stride), dtype=torch.int32, device=dev),
                top_lps=torch.zeros((B, top_stride), dtype=torch.float32, device=dev),
                top_n=torch.empty(B, dtype=torch.int32, device=dev),
                entropy=torch.empty(B, dtype=torch.float32, device=dev),
                max_prob=torch.empty(B, dtype=torch.float32, device=dev),
                margin=torch.empty(B, dtype=torch.float32, device=dev),
                chosen_lp=torch.empty(B, dtype=torch.float32, device=dev),
                status=torch.empty(B, dtype=torch.int32, device=dev),
            )
        b = Batch()
        b.B, b.V, b.ld = B, V, logits.stride(0)
        b.d_logits = logits.data_ptr()
        b.d_params = bufs["params"].data_ptr()
        b.d_cnt_off, b.d_cnt_ids, b.d_cnt_vals = bufs["cnt_off"].data_ptr(), bufs["cnt_ids"].data_ptr(), \
            bufs["cnt_vals"].data_ptr()
        b.d_bias_off, b.d_bias_ids, b.d_bias_vals = bufs["bias_off"].data_ptr(), bufs["bias_ids"].data_ptr(), \
            bufs["bias_vals"].data_ptr()
        b.d_ban_off, b.d_ban_ids = bufs["ban_off"].data_ptr(), bufs["ban_ids"].data_ptr()
        if allow_bits is not None:
            b.d_allow_bits = allow_bits.data_ptr()
            b.allow_words = allow_bits.shape[1]
        b.top_stride = top_stride
        b.d_seed, b.d_counter = bufs["seed"].data_ptr(), bufs["counter"].data_ptr()
        if pass_event is not None:
            b.pass_event = pass_event.cuda_event
        for k in ("token", "logprob", "top_ids", "top_lps", "top_n", "entropy", "max_prob", "margin", "chosen_lp",
                  "status"):
            setattr(b, "d_" + k, out[k].data_ptr())
        stream = torch.cuda.current_stream(dev).cuda_stream
        rc = lib().zs_sample(self.ctx.h, C.byref(b), stream)
        _check(self.ctx.h, rc, "zs_sample")
        return out

    def step(self, logits: torch.Tensor, rows: List[RowRequest], allow_bits: Optional[torch.Tensor] = None):
        """One decode step for every row; advances each row's RNG counter, count
        map and FSM state with the sampled token (rest.rs:2594-2624)."""
        bufs = self.pack(logits, rows, allow_bits)
        out = self.run(logits, bufs, allow_bits)
        torch.cuda.current_stream(logits.device).synchronize()
        toks = out["token"].cpu().numpy().view(np.uint32)
        for rq, tok in zip(rows, toks):
            rq.ctrl.counter += 1
            if rq.fsm is not None:
                rq.fsm.advance(int(tok))
            rq.ctrl.observe(int(tok))
        return out


# ---------------------------------------------------------------- spec decode
def verify_drafts(ctx: Context, target: torch.Tensor, draft_ids: torch.Tensor, temperature: torch.Tensor,
                  seed: torch.Tensor, counter: torch.Tensor, draft: Optional[torch.Tensor] = None,
                  background: bool = False):
    """Batched spec_decode::verify_drafts (spec_decode.rs:241-267) and, for
    temperature > 0 with draft logits, rejection sampling. target [B, k+1, V],
    draft [B, k, V], draft_ids [B, k] (int32). Returns (accepted, next).
    background: ZS_SPEC_BACKGROUND, for a call overlapped with other GPU work
    on another stream (same results)."""
    B, kp1, V = target.shape
    k = kp1 - 1
    dev = target.device
    if target.stride(1) % 4 or target.stride(2) != 1 or (draft is not None and draft.stride(1) != target.stride(1)):
        # the ABI reads rows with 16-byte loads: pad the row stride to a multiple of 4
        ld = (V + 3) // 4 * 4
        t2 = torch.zeros((B, kp1, ld), dtype=target.dtype, device=dev)
        t2[:, :, :V] = target
        target = t2[:, :, :V]
        if draft is not None:
            d2 = torch.zeros((B, k, ld), dtype=draft.dtype, device=dev)
            d2[:, :, :V] = draft
            draft = d2[:, :, :V]
    acc = torch.empty(B, dtype=torch.int32, device=dev)
    nxt = torch.empty(B, dtype=torch.int32, device=dev)
    sb = SpecBatch()
    sb.B, sb.V, sb.k, sb.ld = B, V, k, target.stride(1)
    sb.d_target = target.data_ptr()
    sb.d_draft = draft.data_ptr() if draft is not None else None
    sb.d_draft_ids = draft_ids.data_ptr()
    sb.d_temperature, sb.d_seed, sb.d_counter = temperature.data_ptr(), seed.data_ptr(), counter.data_ptr()
    sb.d_accepted, sb.d_next = acc.data_ptr(), nxt.data_ptr()
    sb.flags = ZS_SPEC_BACKGROUND if background else 0
    rc = lib().zs_spec_verify(ctx.h, C.byref(sb), torch.cuda.current_stream(dev).cuda_stream)
    _check(ctx.h, rc, "zs_spec_verify")
    return acc, nxt


# ---------------------------------------------------------------- batched lane
def lane_argmax(ctx: Context, logits: torch.Tensor) -> torch.Tensor:
    """BARGMAX_WGSL (shaders.rs:761-789) on [B, V] logits."""
    B, V = logits.shape
    out = torch.empty(B, dtype=torch.int32, device=logits.device)
    rc = lib().zs_lane_argmax(ctx.h, logits.data_ptr(), B, V, logits.stride(0), out.data_ptr(),
                              torch.cuda.current_stream(logits.device).cuda_stream)
    _check(ctx.h, rc, "zs_lane_argmax")
    return out


def lane_sample(ctx: Context, logits: torch.Tensor, temperature: torch.Tensor, seed: torch.Tensor) -> torch.Tensor:
    """BSAMPLE_WGSL Gumbel-max (shaders.rs:796-850); seed uint32 per row."""
    B, V = logits.shape
    out = torch.empty(B, dtype=torch.int32, device=logits.device)
    rc = lib().zs_lane_sample(ctx.h, logits.data_ptr(), B, V, logits.stride(0), temperature.data_ptr(),
                              seed.data_ptr(), out.data_ptr(), torch.cuda.current_stream(logits.device).cuda_stream)
    _check(ctx.h, rc, "zs_lane_sample")
    return out


def lane_topk(ctx: Context, logits: torch.Tensor, K: int = 64):
    """BTOPK_WGSL (shaders.rs:859-905): [B, K] values (desc) and ids."""
    B, V = logits.shape
    vals = torch.empty((B, K), dtype=torch.float32, device=logits.device)
    idxs = torch.empty((B, K), dtype=torch.int32, device=logits.device)
    rc = lib().zs_lane_topk(ctx.h, logits.data_ptr(), B, V, logits.stride(0), K, vals.data_ptr(), idxs.data_ptr(),
                            torch.cuda.current_stream(logits.device).cuda_stream)
    _check(ctx.h, rc, "zs_lane_topk")
    return vals, idxs


def lane_sample_topk(ctx: Context, vals: torch.Tensor, idxs: torch.Tensor, temperature: torch.Tensor,
                     top_k: torch.Tensor, top_p: torch.Tensor, seed: torch.Tensor) -> torch.Tensor:
    """gpu/sampling.rs:35-56 sample_topk per row over its top-K pool."""
    B, K = vals.shape
    out = torch.empty(B, dtype=torch.int32, device=vals.device)
    rc = lib().zs_lane_sample_topk(ctx.h, vals.data_ptr(), idxs.data_ptr(), B, K, temperature.data_ptr(),
                                   top_k.data_ptr(), top_p.data_ptr(), seed.data_ptr(), out.data_ptr(),
                                   torch.cuda.current_stream(vals.device).cuda_stream)
    _check(ctx.h, rc, "zs_lane_sample_topk")
    return out


def step_seed(base: int, gen_idx: int) -> int:
    """gpu/sampling.rs:9."""
    return int(lib().zs_step_seed(base & 0xFFFFFFFF, gen_idx & 0xFFFFFFFF))


# ---------------------------------------------------------------- continuous-batching lane
ZS_LANE_ARGMAX, ZS_LANE_SAMPLE, ZS_LANE_TOPK = 0, 1, 2


@dataclass
class SamplingParams:
    """gpu/sampling.rs:14-21: temp <= 0 greedy; top_k 0 = no cap; top_p >= 1
    (or 0) = no nucleus cut (both applied inside the top-64 pool)."""
    temp: float = 0.0
    top_k: int = 0
    top_p: float = 1.0

    @staticmethod
    def greedy():
        return SamplingParams(0.0, 0, 1.0)

    @staticmethod
    def temperature(temp: float):
        return SamplingParams(temp, 0, 1.0)

    def needs_topk(self) -> bool:  # gpu/sampling.rs:20
        return self.top_k > 0 or (0.0 < self.top_p < 1.0)


@dataclass
class LaneSeq:
    """The sampling state of CbSeq (gpu/batch.rs): tokens generated so far
    (the prefill's first token included), limits and seeding."""
    id: int
    params: SamplingParams
    base_seed: int
    eos: int
    max_tokens: int
    generated: List[int] = field(default_factory=list)

    def gen_index(self) -> int:
        return len(self.generated)


class LaneBatcher:
    """ContinuousBatcher::step's token selection (gpu/batch.rs:176-207) on
    libzs: the caller runs the model forward for the active streams (in
    `active` order) and hands the logits [m, V] to step(), which picks every
    stream's next token on the GPU with one zs_lane_step call (top-64 pool +
    nucleus / Gumbel sampling / argmax, seeds step_seed(base, gen_index)),
    reads back m ids and retires finished streams as the reference does."""

    def __init__(self, ctx: Context):
        self.ctx = ctx
        self.active: List[LaneSeq] = []
        self.last_path = None

    def add(self, seq: LaneSeq):
        self.active.append(seq)

    def select(self, logits: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Device ids for the active streams (no host sync)."""
        m, V = logits.shape
        assert m == len(self.active) and logits.dtype == torch.float32 and logits.stride(1) == 1
        if out is None:
            out = torch.empty(m, dtype=torch.int32, device=logits.device)
        st = (LaneStream * max(m, 1))()
        for i, s in enumerate(self.active):
            st[i].temp, st[i].top_k, st[i].top_p = s.params.temp, s.params.top_k, s.params.top_p
            st[i].base_seed, st[i].gen_index = s.base_seed & 0xFFFFFFFF, s.gen_index() & 0xFFFFFFFF
        path = C.c_int()
        stream = torch.cuda.current_stream(logits.device).cuda_stream
        rc = lib().zs_lane_step(self.ctx.h, logits.data_ptr(), m, V, logits.stride(0), st, out.data_ptr(),
                                C.byref(path), stream)
        _check(self.ctx.h, rc, "zs_lane_step")
        self.last_path = path.value
        return out

    def step(self, logits: torch.Tensor) -> List[Tuple[int, int, bool]]:
        """(id, token, done) per active stream; finished streams leave the batch."""
        ids = self.select(logits).cpu().numpy().view(np.uint32)
        res = []
        for s, t in zip(self.active, ids):
            s.generated.append(int(t))
            res.append((s.id, int(t), int(t) == s.eos or s.gen_index() >= s.max_tokens))
        self.active = [s for s in self.active if not (s.generated[-1] == s.eos or s.gen_index() >= s.max_tokens)]
        return res
