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
