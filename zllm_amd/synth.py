"""Seeded synthetic workloads for the BASELINE.json configs.

There is no model on this path: logits, vocabularies and DFAs are generated
from a seed (numpy PCG64), the same on every machine with this image.
"""
import numpy as np

SPIKES = 16


def logits_normal(B, V, seed, sigma=2.0):
    rng = np.random.default_rng(seed)
    return (rng.standard_normal((B, V), dtype=np.float32) * np.float32(sigma)).astype(np.float32)


def logits_c1(seed=0):
    """Config 1: [1, 32000] N(0, 2.0), 8 random ids spiked by +12."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((1, 32000), dtype=np.float32) * np.float32(2.0)).astype(np.float32)
    ids = rng.choice(32000, 8, replace=False)
    x[0, ids] += np.float32(12.0)
    return x


def logits_powerlaw(B, V, seed, sigma=2.0, peak=15.0, nspikes=SPIKES):
    """N(0, sigma) plus a power-law peak: nspikes random ids spiked by peak*k^-1.2."""
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((B, V), dtype=np.float32) * np.float32(sigma)).astype(np.float32)
    ks = np.arange(1, nspikes + 1, dtype=np.float64)
    add = (peak * ks ** -1.2).astype(np.float32)
    for b in range(B):
        ids = rng.choice(V, nspikes, replace=False)
        x[b, ids] += add
    return x


def mixed_params(B, V, seed, hist=256):
    """Per-row knobs of configs 2 and 5: T in [0.5, 1.2], top_k in {0, 20, 50},
    top_p in [0.8, 1.0], frequency/presence in [0, 0.5] over `hist`-token
    histories. Returns a list of dicts + count maps."""
    rng = np.random.default_rng(seed + 7919)
    rows = []
    for b in range(B):
        h = rng.integers(0, V, size=hist)
        ids, cnt = np.unique(h, return_counts=True)
        rows.append(dict(
            temperature=float(np.float32(rng.uniform(0.5, 1.2))),
            top_k=int(rng.choice([0, 20, 50])),
            top_p=float(np.float32(rng.uniform(0.8, 1.0))),
            min_p=0.0,
            repeat=1.0,
            presence=float(np.float32(rng.uniform(0.0, 0.5))),
            frequency=float(np.float32(rng.uniform(0.0, 0.5))),
            counts=list(zip(ids.tolist(), cnt.tolist())),
        ))
    return rows


# ---------------------------------------------------------------- vocabulary
_ALNUM_PUNCT = np.frombuffer(b"abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789.,;:!?'\"-_()[]{}<>/\\@#$%&*+=",
                             np.uint8)
_LETTERS = np.frombuffer(b"abcdefghijklmnopqrstuvwxyz", np.uint8)


def synthetic_vocab(V, seed):
    """V token byte strings: lengths 1-16, geometric with mean 4; 70% ASCII
    letters/digits/punct, 20% space-prefixed words, 10% arbitrary UTF-8
    continuation bytes (0x80-0xBF). Returns (offsets u32[V+1], bytes u8[])."""
    rng = np.random.default_rng(seed + 104729)
    lens = np.minimum(rng.geometric(0.25, size=V), 16).astype(np.int64)
    kind = rng.random(V)
    out = np.zeros(int(lens.sum()), np.uint8)
    offs = np.zeros(V + 1, np.uint32)
    offs[1:] = np.cumsum(lens)
    pos = 0
    for t in range(V):
        n = int(lens[t])
        if kind[t] < 0.7:
            out[pos:pos + n] = rng.choice(_ALNUM_PUNCT, n)
        elif kind[t] < 0.9:
            out[pos] = 32
            if n > 1:
                out[pos + 1:pos + n] = rng.choice(_LETTERS, n - 1)
        else:
            out[pos:pos + n] = rng.integers(0x80, 0xC0, n)
        pos += n
    return offs, out


def random_dfa(S, seed, dead_rate=0.3, accept_rate=0.1):
    """Anchored byte DFA with S states x 256 bytes (state S-1 = dead), a
    `dead_rate` fraction of dead transitions and accepting states from seed."""
    rng = np.random.default_rng(seed + 15485863)
    dead_id = S - 1
    trans = rng.integers(0, S - 1, size=(S, 256)).astype(np.uint32)
    trans[rng.random((S, 256)) < dead_rate] = dead_id
    trans[dead_id, :] = dead_id
    dead = np.zeros(S, np.uint8)
    dead[dead_id] = 1
    accept = (rng.random(S) < accept_rate).astype(np.uint8)
    accept[dead_id] = 0
    return trans, dead, accept


# ---------------------------------------------------------------- JSON-schema DFA
_NAME_CHARS = b"abcdefghijklmnopqrstuvwxyz_"
_STR_CHARS = b"abcdefghijklmnopqrstuvwxyzABCDEFGHIJKLMNOPQRSTUVWXYZ0123456789 -_.,"


class _DfaBuilder:
    def __init__(self):
        self.rows = []
        self.accept = []
        self.dead = self.new()          # state 0: dead sink

    def new(self):
        self.rows.append(np.zeros(256, np.int64))   # default -> dead (0)
        self.accept.append(0)
        return len(self.rows) - 1

    def edge(self, s, byte, t):
        self.rows[s][byte] = t

    def literal(self, s, text):
        for b in text:
            t = self.new()
            self.edge(s, b, t)
            s = t
        return s


def json_dfa(target_states, seed, max_depth=2):
    """Anchored byte DFA for a synthetic JSON schema: nested objects of 6-12
    required properties in a fixed order (no whitespace), each property a
    string, number, bool, enum or (up to `max_depth`) nested object, names drawn
    from seed. Properties are added to the root object until the automaton has
    at least `target_states` states. Returns (trans u32[S,256], dead u8[S],
    accept u8[S]); state 0 is the dead state, state 1 the start."""
    rng = np.random.default_rng(seed + 7777)
    B = _DfaBuilder()
    start = B.new()

    def name():
        n = int(rng.integers(3, 11))
        return bytes(rng.choice(np.frombuffer(_NAME_CHARS, np.uint8), n).tolist())

    def value(s, depth):
        """Value from state s; returns the state after the value."""
        kind = rng.choice(["string", "number", "bool", "enum", "object"] if depth < max_depth
                          else ["string", "number", "bool", "enum"])
        if kind == "string":
            q = B.new()
            B.edge(s, ord('"'), q)
            for c in _STR_CHARS:
                B.edge(q, c, q)
            e = B.new()
            B.edge(q, ord('"'), e)
            return e
        if kind == "number":
            sign = B.new()
            B.edge(s, ord("-"), sign)
            ip = B.new()
            for c in b"0123456789":
                B.edge(s, c, ip)
                B.edge(sign, c, ip)
                B.edge(ip, c, ip)
            dot = B.new()
            B.edge(ip, ord("."), dot)
            fp = B.new()
            for c in b"0123456789":
                B.edge(dot, c, fp)
                B.edge(fp, c, fp)
            # the number ends at the next structural byte: the caller's edges
            # from the end state are copied onto ip and fp
            return ("number", ip, fp)
        if kind == "bool":
            t = B.literal(s, b"true")
            f_ = B.literal(s, b"fals")
            e = B.new()
            B.edge(f_, ord("e"), e)
            B.rows[t] = B.rows[e]   # share the continuation row (same object)
            return ("alias", e, t)
        if kind == "enum":
            e = B.new()
            words = {bytes(rng.choice(np.frombuffer(_NAME_CHARS, np.uint8), int(rng.integers(2, 8))).tolist())
                     for _ in range(int(rng.integers(2, 6)))}
            q = B.new()
            B.edge(s, ord('"'), q)
            for w in sorted(words):   # a trie of quoted words
                cur = q
                for c in w:
                    nxt = B.rows[cur][c]
                    if nxt == 0:
                        nxt = B.new()
                        B.edge(cur, c, nxt)
                    cur = nxt
                B.edge(cur, ord('"'), e)
            return e
        return obj(s, depth + 1, int(rng.integers(6, 13)))

    def close_value(v):
        """Normalises a value result to (end state, extra end states that share its row)."""
        if isinstance(v, tuple):
            if v[0] == "number":
                return v[1], [v[2]]
            return v[1], [v[2]]
        return v, []

    def obj(s, depth, nprops, grow=False):
        o = B.new()
        B.edge(s, ord("{"), o)
        cur, extra = o, []
        i = 0
        while True:
            if i > 0:
                c = B.new()
                B.edge(cur, ord(","), c)
                for x in extra:
                    B.edge(x, ord(","), c)
                cur, extra = c, []
            k = B.literal(cur, b'"' + name() + b'":')
            cur, extra = close_value(value(k, depth))
            i += 1
            if i >= nprops and (not grow or len(B.rows) >= target_states - 2):
                break
        end = B.new()
        B.edge(cur, ord("}"), end)
        for x in extra:
            B.edge(x, ord("}"), end)
        return end

    root_end = obj(start, 0, 6, grow=True)
    B.accept[root_end] = 1
    S = len(B.rows)
    trans = np.stack(B.rows).astype(np.uint32)
    dead = np.zeros(S, np.uint8)
    dead[0] = 1
    accept = np.array(B.accept, np.uint8)
    # anchored: renumber so that state 0 is the start (the reference walks
    # from the caller's current state; the start is what a fresh request uses)
    return trans, dead, accept


def grammar_vocab(trans, dead, V, seed, frac=0.5):
    """V tokens: a `frac` share are byte strings of random walks through the
    DFA (lengths geometric with mean 4, capped at 16, from random non-dead
    states along non-dead transitions), the rest as synthetic_vocab. Gives a
    vocabulary whose tokens survive long walks. Returns (offsets, bytes)."""
    rng = np.random.default_rng(seed + 3331)
    offs0, data0 = synthetic_vocab(V, seed)
    S = trans.shape[0]
    good = np.nonzero(dead == 0)[0]
    toks = []
    for t in range(V):
        if rng.random() < frac:
            s = int(rng.choice(good))
            n = int(min(rng.geometric(0.25), 16))
            out = bytearray()
            for _ in range(n):
                nxt = np.nonzero(dead[trans[s]] == 0)[0]
                if len(nxt) == 0:
                    break
                b = int(rng.choice(nxt))
                out.append(b)
                s = int(trans[s, b])
            if not out:
                out = bytearray(b"a")
            toks.append(bytes(out))
        else:
            toks.append(bytes(data0[offs0[t]:offs0[t + 1]]))
    offs = np.zeros(V + 1, np.uint32)
    offs[1:] = np.cumsum([len(x) for x in toks])
    return offs, np.frombuffer(b"".join(toks), np.uint8).copy()
