"""GPU parity: zs_dfa_mask allow bitsets against the oracle's apply_mask
(logit_fsm.rs:247-270) -- bit-exact."""
import numpy as np
import pytest
import torch

from oracle import oracle as O
from tests.tiny import TINY_EOS, TINY_TOKENS, dfa_ab_opt, dfa_ab_plus_c, dfa_ab_star_c, dfa_abc
from zllm_amd import synth

pytestmark = pytest.mark.gpu


def _gpu_bits(trans, dead, acc, tokens_csr, eos, states, V):
    from tests.gpu_util import ctx
    from zllm_amd.engine import ByteDfa, TokenByteTable
    c = ctx()
    offs, data, valid = tokens_csr
    table = TokenByteTable.from_csr(c, offs, data, valid, eos)
    dfa = ByteDfa(c, trans, dead, acc)
    st = torch.tensor(np.asarray(states, np.int32), device="cuda")
    anyv = torch.zeros(len(states), dtype=torch.int32, device="cuda")
    bits = dfa.mask(table, st, V, any_out=anyv)
    torch.cuda.synchronize()
    return bits.cpu().numpy().view(np.uint32), anyv.cpu().numpy(), dfa, table


def _csr(tokens):
    offs = [0]
    buf = bytearray()
    valid = []
    for t in tokens:
        valid.append(0 if t is None else 1)
        if t is not None:
            buf += t
        offs.append(len(buf))
    return np.array(offs, np.uint32), np.frombuffer(bytes(buf) or b"\0", np.uint8), np.array(valid, np.uint8)


@pytest.mark.parametrize("mk", [dfa_ab_star_c, dfa_abc, dfa_ab_opt, dfa_ab_plus_c])
def test_tiny_table_every_state(mk):
    trans, dead, acc = mk()
    S = trans.shape[0]
    V = 6
    print(f"[case] tiny {mk.__name__}", flush=True)
    bits, anyv, dfa, table = _gpu_bits(trans, dead, acc, _csr(TINY_TOKENS), TINY_EOS, list(range(S)) + [-1], V)
    od, ov = O.Dfa(trans, dead, acc), O.Vocab(TINY_TOKENS, TINY_EOS)
    for s in range(S):
        want = O.mask_bits(V, dfa=od, vocab=ov, state=s)
        assert bits[s].tolist() == want.tolist(), (s, bits[s], want)
        assert dfa.is_live(s) == bool(od.live[s])
    assert bits[S].tolist() == O.pack_bits(np.ones(V, bool)).tolist()


@pytest.mark.parametrize("S,V,ntab_delta", [(64, 5000, 0), (64, 128256, 0), (512, 20000, 0), (40, 3000, -100),
                                            (40, 3000, 37)])
def test_random_dfa_synthetic_vocab(S, V, ntab_delta):
    print(f"[case] S={S} V={V}", flush=True)
    ntab = V + ntab_delta
    offs, data = synth.synthetic_vocab(ntab, S + V)
    valid = np.ones(ntab, np.uint8)
    valid[::97] = 0
    eos = ntab - 3 if ntab_delta <= 0 else V + 5  # eos inside or beyond the table
    trans, dead, acc = synth.random_dfa(S, S * 7 + V, dead_rate=0.3)
    rng = np.random.default_rng(S + V)
    states = list(rng.integers(0, S, 24)) + [S - 1, -1]  # incl. the dead state and a free row
    bits, anyv, dfa, table = _gpu_bits(trans, dead, acc, (offs, data, valid), eos, states, V)
    tokens = [None if not valid[t] else bytes(data[offs[t]:offs[t + 1]]) for t in range(ntab)]
    od, ov = O.Dfa(trans, dead, acc), O.Vocab(tokens, eos)
    for i, s in enumerate(states):
        if s < 0:
            want = O.pack_bits(np.ones(V, bool))
        else:
            want = O.mask_bits(V, dfa=od, vocab=ov, state=int(s))
            allowed, a = O.dfa_allowed(od, ov, int(s))
            assert bool(anyv[i]) == a
        assert np.array_equal(bits[i], want), (i, s)


def test_advance_matches_oracle():
    from tests.gpu_util import ctx
    from zllm_amd.engine import ByteDfa, TokenByteTable
    trans, dead, acc = dfa_ab_star_c()
    c = ctx()
    table = TokenByteTable(c, TINY_TOKENS, TINY_EOS)
    dfa = ByteDfa(c, trans, dead, acc)
    od, ov = O.Dfa(trans, dead, acc), O.Vocab(TINY_TOKENS, TINY_EOS)
    for s in range(trans.shape[0]):
        for tok in range(7):
            assert dfa.advance(table, s, tok)[0] == O.advance(od, ov, s, tok)


@pytest.mark.parametrize("S,V,rows", [(512, 20000, 16), (2048, 30000, 12)])
def test_json_schema_dfa_grammar_vocab(S, V, rows):
    """Structured DFA (nested-object JSON schema, few byte classes) with a vocab
    of grammar fragments, so that walks survive many steps; the 2048-state
    automaton exercises the tightly packed LDS table at 12-bit entries."""
    print(f"[case] json S={S} V={V}", flush=True)
    trans, dead, acc = synth.json_dfa(S, S + 1)
    offs, data = synth.grammar_vocab(trans, dead, V, S + 2)
    valid = np.ones(V, np.uint8)
    valid[5::101] = 0
    eos = V - 1
    rng = np.random.default_rng(S + 3)
    good = np.nonzero(dead == 0)[0]
    states = list(rng.choice(good, rows)) + [0, -1]  # + the dead state and a free row
    bits, anyv, dfa, table = _gpu_bits(trans, dead, acc, (offs, data, valid), eos, states, V)
    tokens = [None if not valid[t] else bytes(data[offs[t]:offs[t + 1]]) for t in range(V)]
    od, ov = O.Dfa(trans, dead, acc), O.Vocab(tokens, eos)
    nonzero = 0
    for i, s in enumerate(states):
        if s < 0:
            want = O.pack_bits(np.ones(V, bool))
        else:
            want = O.mask_bits(V, dfa=od, vocab=ov, state=int(s))
            allowed, a = O.dfa_allowed(od, ov, int(s))
            assert bool(anyv[i]) == a
            nonzero += int(np.count_nonzero(want))
        assert np.array_equal(bits[i], want), (i, s)
    assert nonzero > 0


def test_large_random_dfa_through_l2():
    """A table beyond the LDS budget (3000 states x 256 classes) takes the
    L2-resident walk."""
    S, V = 3000, 8000
    print(f"[case] large S={S} V={V}", flush=True)
    offs, data = synth.synthetic_vocab(V, 77)
    valid = np.ones(V, np.uint8)
    trans, dead, acc = synth.random_dfa(S, 78, dead_rate=0.3)
    rng = np.random.default_rng(79)
    states = list(rng.integers(0, S - 1, 8)) + [-1]
    bits, anyv, dfa, table = _gpu_bits(trans, dead, acc, (offs, data, valid), V - 1, states, V)
    tokens = [bytes(data[offs[t]:offs[t + 1]]) for t in range(V)]
    od, ov = O.Dfa(trans, dead, acc), O.Vocab(tokens, V - 1)
    for i, s in enumerate(states):
        want = O.pack_bits(np.ones(V, bool)) if s < 0 else O.mask_bits(V, dfa=od, vocab=ov, state=int(s))
        assert np.array_equal(bits[i], want), (i, s)


def _class_dfa(S, ncls, per_state, seed):
    """S states over ncls byte classes (byte b in class b % ncls); every state
    has `per_state` classes into random states, the rest into the dead state
    S - 1; a third of the states accept."""
    rng = np.random.default_rng(seed)
    trans = np.full((S, 256), S - 1, np.uint32)
    for s in range(S - 1):
        for c in rng.choice(ncls, per_state, replace=False):
            trans[s, np.arange(c, 256, ncls)] = rng.integers(0, S - 1)
    dead = np.zeros(S, np.uint8)
    dead[S - 1] = 1
    acc = (rng.random(S) < 0.33).astype(np.uint8)
    acc[S - 1] = 0
    return trans, dead, acc


@pytest.mark.parametrize("S,ncls,per_state,form", [(3000, 40, 4, "displaced"), (3500, 60, 10, "sparse")])
def test_table_forms_past_the_packed_budget(S, ncls, per_state, form):
    """Tables too large for bit-packed rows in LDS: displaced rows (one read
    and a compare per step) and, where those do not fit either, sparse rows.
    Bitsets equal the oracle's for every row."""
    V = 8000
    print(f"[case] form={form} S={S} ncls={ncls} per_state={per_state}", flush=True)
    offs, data = synth.synthetic_vocab(V, 91)
    valid = np.ones(V, np.uint8)
    trans, dead, acc = _class_dfa(S, ncls, per_state, 92)
    rng = np.random.default_rng(93)
    states = list(rng.integers(0, S - 1, 12)) + [-1]
    bits, anyv, dfa, table = _gpu_bits(trans, dead, acc, (offs, data, valid), V - 1, states, V)
    assert dfa.table_form == form
    tokens = [bytes(data[offs[t]:offs[t + 1]]) for t in range(V)]
    od, ov = O.Dfa(trans, dead, acc), O.Vocab(tokens, V - 1)
    nonzero = 0
    for i, s in enumerate(states):
        want = O.pack_bits(np.ones(V, bool)) if s < 0 else O.mask_bits(V, dfa=od, vocab=ov, state=int(s))
        assert np.array_equal(bits[i], want), (form, i, s)
        nonzero += int(s >= 0 and want[: (V - 1) // 32].any())
    assert nonzero > 0


COMPILED = {
    "json": "json:",
    "tool_schema": 'json_schema:{"type":"object","properties":{"location":{"type":"string"},'
                   '"unit":{"enum":["celsius","fahrenheit"]},"days":{"type":"array","items":{"type":"integer"},'
                   '"maxItems":3}}}',
    "regex": r"regex:[A-Z][a-z]*( [a-z]+)*[.!?]( [A-Z][a-z]*( [a-z]+)*[.!?])*",
}


@pytest.mark.parametrize("name", list(COMPILED))
def test_compiled_grammar_masks(name):
    """Grammars compiled by the native regex / JSON-schema compiler
    (LogitFSM.compile): GPU masks along a constrained walk equal the oracle's,
    bit for bit."""
    from tests.gpu_util import ctx
    from zllm_amd import grammar as G
    from zllm_amd.engine import LogitFSM, TokenByteTable
    print(f"[case] compiled {name}", flush=True)
    g = COMPILED[name]
    pattern = (G.any_json_regex_default() if g == "json:" else
               G.schema_to_regex(g[len("json_schema:"):]) if g.startswith("json_schema:") else g[len("regex:"):])
    host = G.HostDfa(pattern)
    V = 8192
    offs, data = synth.grammar_vocab(host.trans, host.dead, V, 17)
    valid = np.ones(V, np.uint8)
    valid[::211] = 0
    eos = V - 1
    c = ctx()
    table = TokenByteTable.from_csr(c, offs, data, valid, eos)
    fsm = LogitFSM.compile(g, table)
    assert fsm.state == host.start and fsm.dfa.nstates == host.nstates
    if g == "json:":
        assert fsm.dfa.table_form == "displaced"
    tokens = [None if not valid[t] else bytes(data[offs[t]:offs[t + 1]]) for t in range(V)]
    od, ov = O.Dfa(host.trans, host.dead, host.accept), O.Vocab(tokens, eos)
    # states along a walk that always takes an allowed token
    rng = np.random.default_rng(5)
    states, s = [], host.start
    for _ in range(24):
        states.append(s)
        allowed, _ = O.dfa_allowed(od, ov, s)
        ids = np.nonzero(allowed)[0]
        if len(ids) == 0:
            break
        s = O.advance(od, ov, s, int(rng.choice(ids)))
    st = torch.tensor(np.asarray(states, np.int32), device="cuda")
    bits = fsm.dfa.mask(table, st, V)
    torch.cuda.synchronize()
    bits = bits.cpu().numpy().view(np.uint32)
    for i, s in enumerate(states):
        assert np.array_equal(bits[i], O.mask_bits(V, dfa=od, vocab=ov, state=int(s))), (name, i, s)


def test_real_vocab_table_and_json_grammar():
    """A byte-level BPE vocabulary (HF tokenizers) -> zs_token_table ->
    zs_vocab, with the `json:` grammar: GPU masks equal the oracle's."""
    tk = pytest.importorskip("tokenizers")
    from tests.gpu_util import ctx
    from tests.test_vocab import byte_level_bpe
    from zllm_amd.engine import LogitFSM, TokenByteTable
    from zllm_amd.vocab import HostTokenTable
    print("[case] real vocab json", flush=True)
    host = HostTokenTable.from_tokenizer_json(byte_level_bpe(seed=7, vocab_size=3000).to_str())
    c = ctx()
    table = TokenByteTable.from_host_table(c, host)
    fsm = LogitFSM.compile("json:", table)
    V = host.ntab + 5  # logits wider than the table: the extra ids are never allowed
    tokens = host.tokens()
    d = fsm.dfa
    from zllm_amd import grammar as G
    g = G.HostDfa(G.any_json_regex_default())
    od, ov = O.Dfa(g.trans, g.dead, g.accept), O.Vocab(tokens, host.eos)
    states = [g.start] + [int(s) for s in np.random.default_rng(3).integers(1, g.nstates, 15)]
    st = torch.tensor(np.asarray(states, np.int32), device="cuda")
    bits = d.mask(table, st, V)
    torch.cuda.synchronize()
    bits = bits.cpu().numpy().view(np.uint32)
    for i, s in enumerate(states):
        assert np.array_equal(bits[i], O.mask_bits(V, dfa=od, vocab=ov, state=s)), (i, s)


def test_viability_flags_across_kernel_paths():
    """A call on the L2-table path (more rows than the LDS walk takes) followed
    by one on the LDS path, on one context with the context's own viability
    flags: a flag left by the first call must not make a dead-end row's EOS
    disallowed in the second (logit_fsm.rs:258-262: EOS is allowed when no
    token is viable)."""
    from tests.tiny import build_dfa
    from zllm_amd.engine import ByteDfa, Context, TokenByteTable
    print("[case] fallback then packed DFA mask on one context", flush=True)
    # 0 -a-> 1 -z-> 2 (accepting); no token of the table starts with 'z', so
    # state 1 is live, not accepting, and has no viable token
    trans, dead, acc = build_dfa({0: {"a": 1}, 1: {"z": 2}}, [2], 3)
    V = 6
    c = Context(0, 1100, 64)
    offs, data, valid = _csr(TINY_TOKENS)
    table = TokenByteTable.from_csr(c, offs, data, valid, TINY_EOS)
    dfa = ByteDfa(c, trans, dead, acc)
    od, ov = O.Dfa(trans, dead, acc), O.Vocab(TINY_TOKENS, TINY_EOS)
    big = torch.zeros(1100, dtype=torch.int32, device="cuda")        # > ZS_DFA_MAXROWS rows: L2 path
    bits_big = dfa.mask(table, big, V)
    small = torch.tensor([1, 0], dtype=torch.int32, device="cuda")  # LDS path
    bits_small = dfa.mask(table, small, V)
    torch.cuda.synchronize()
    bb = bits_big.cpu().numpy().view(np.uint32)
    bs = bits_small.cpu().numpy().view(np.uint32)
    want0 = O.mask_bits(V, dfa=od, vocab=ov, state=0)
    want1 = O.mask_bits(V, dfa=od, vocab=ov, state=1)
    assert all(np.array_equal(bb[i], want0) for i in (0, 1, 1099))
    assert np.array_equal(bs[0], want1), (bs[0], want1)
    assert np.array_equal(bs[1], want0), (bs[1], want0)
    # and back on the L2 path after the LDS path
    bits_big2 = dfa.mask(table, torch.ones(1100, dtype=torch.int32, device="cuda"), V)
    torch.cuda.synchronize()
    assert np.array_equal(bits_big2.cpu().numpy().view(np.uint32)[7], want1)


def test_memo_hits_equal_fresh_walks():
    """The per-state memo (logit_fsm.rs:166-182's cache): masks served from it
    are bit-identical, with the same viability flags and EOS rule, to the
    masks of a DFA with an empty memo; rows that share a state in one call
    share one walk; another vocabulary or V invalidates the memo."""
    from tests.gpu_util import ctx
    from zllm_amd.engine import ByteDfa, TokenByteTable
    S, V = 512, 20000
    print(f"[case] memo json S={S} V={V}", flush=True)
    c = ctx()
    trans, dead, acc = synth.json_dfa(S, 41)
    offs, data = synth.grammar_vocab(trans, dead, V, 42)
    valid = np.ones(V, np.uint8)
    valid[3::89] = 0
    table = TokenByteTable.from_csr(c, offs, data, valid, V - 1)
    offs2, data2 = synth.grammar_vocab(trans, dead, V, 43)
    table2 = TokenByteTable.from_csr(c, offs2, data2, np.ones(V, np.uint8), V - 1)
    dfa = ByteDfa(c, trans, dead, acc)
    rng = np.random.default_rng(44)
    good = np.nonzero(dead == 0)[0]
    pool = rng.choice(good, 40, replace=False)

    def run(d, tab, states, v):
        st = torch.tensor(np.asarray(states, np.int32), device="cuda")
        anyv = torch.zeros(len(states), dtype=torch.int32, device="cuda")
        bits = d.mask(tab, st, v, any_out=anyv)
        torch.cuda.synchronize()
        return bits.cpu().numpy().view(np.uint32).copy(), anyv.cpu().numpy().copy()

    def fresh(tab, states, v):
        return run(ByteDfa(c, trans, dead, acc), tab, states, v)

    def same(got, want, what):
        assert np.array_equal(got[0], want[0]), what
        assert np.array_equal(got[1], want[1]), what

    # cold: repeated states in one call, the dead state, a free row
    s1 = [int(x) for x in pool[:20]] + [int(pool[0]), int(pool[3]), int(pool[3]), 0, -1]
    first = run(dfa, table, s1, V)
    tokens = [None if not valid[t] else bytes(data[offs[t]:offs[t + 1]]) for t in range(V)]
    od, ov = O.Dfa(trans, dead, acc), O.Vocab(tokens, V - 1)
    for i in (0, 3, 20, 21, 22, 23):
        assert np.array_equal(first[0][i], O.mask_bits(V, dfa=od, vocab=ov, state=s1[i])), i
    same(first, fresh(table, s1, V), "cold call")
    # all hits, twice; then a smaller call mixing hits and new states
    same(run(dfa, table, s1, V), first, "all hits")
    same(run(dfa, table, s1[::-1], V), (first[0][::-1], first[1][::-1]), "all hits, reversed")
    s2 = [int(x) for x in pool[15:35]] + [-1, int(pool[16])]
    same(run(dfa, table, s2, V), fresh(table, s2, V), "hits and misses")
    # another vocabulary, another V, then back: never a stale slot
    same(run(dfa, table2, s1, V), fresh(table2, s1, V), "other vocabulary")
    same(run(dfa, table, s1, V - 37), fresh(table, s1, V - 37), "other V")
    same(run(dfa, table, s1, V), first, "back to the first pair")
    # cleared memo: every row walked again
    dfa.memo_clear()
    same(run(dfa, table, s2, V), fresh(table, s2, V), "after memo_clear")


@pytest.mark.parametrize("mk", [dfa_ab_star_c, dfa_ab_plus_c])
def test_empty_token_and_direct_eos_rule(mk):
    """A valid token with no bytes is allowed from every live state (its walk
    ends where it starts, logit_fsm.rs:170-178), so every live state has a
    viable token and the EOS rule reduces to is_accept(s); the mask kernel
    then applies it without the separate EOS pass. Masks and viability flags
    equal the oracle's for every state, twice (the second call from the memo)."""
    trans, dead, acc = mk()
    S = trans.shape[0]
    tokens = [b"a", b"", b"b", b"ab", None, b"c", b"zz"]
    eos = 4
    V = 8
    print(f"[case] empty token {mk.__name__}", flush=True)
    od, ov = O.Dfa(trans, dead, acc), O.Vocab(tokens, eos)
    states = list(range(S)) + [-1, 1, 0]
    from tests.gpu_util import ctx
    from zllm_amd.engine import ByteDfa, TokenByteTable
    c = ctx()
    offs, data, valid = _csr(tokens)
    table = TokenByteTable.from_csr(c, offs, data, valid, eos)
    dfa = ByteDfa(c, trans, dead, acc)
    st = torch.tensor(np.asarray(states, np.int32), device="cuda")
    for _ in range(2):
        anyv = torch.full((len(states),), 7, dtype=torch.int32, device="cuda")
        bits = dfa.mask(table, st, V, any_out=anyv)
        torch.cuda.synchronize()
        b, a = bits.cpu().numpy().view(np.uint32), anyv.cpu().numpy()
        for i, s in enumerate(states):
            if s < 0:
                assert b[i].tolist() == O.pack_bits(np.ones(V, bool)).tolist()
                continue
            assert b[i].tolist() == O.mask_bits(V, dfa=od, vocab=ov, state=s).tolist(), (i, s)
            assert bool(a[i]) == O.dfa_allowed(od, ov, s)[1], (i, s)
