"""Hand-built fixtures shared by the CPU and GPU tests.

`tiny_table` is the 6-entry vocab of logit_fsm.rs:331-342. The DFAs below are
hand-built dense tables for the anchored patterns the reference tests compile
with regex-automata (`ab*c`, `abc`, `ab?`, `ab+c`). They mimic the quirk the
reference documents at logit_fsm.rs:115-117: after a complete match, further
bytes lead to a non-dead state from which no match is reachable, so the mask
depends on liveness, not on the dead state alone. State numbering is this
file's own; the masks the reference tests assert do not depend on it.
"""
import numpy as np

TINY_TOKENS = [b"a", b"b", b"ab", b"c", None]
TINY_EOS = 5


def build_dfa(edges, accept, nstates):
    """edges: {state: {byte_or_'*': next}}; missing bytes go to the dead state
    (id nstates). Returns (trans[S,256], dead[S], accept[S]) with S = nstates+1."""
    S = nstates + 1
    dead_id = nstates
    trans = np.full((S, 256), dead_id, np.uint32)
    for s, m in edges.items():
        if "*" in m:
            trans[s, :] = m["*"]
        for b, t in m.items():
            if b == "*":
                continue
            trans[s, ord(b) if isinstance(b, str) else b] = t
    dead = np.zeros(S, np.uint8)
    dead[dead_id] = 1
    acc = np.zeros(S, np.uint8)
    for s in accept:
        acc[s] = 1
    return trans, dead, acc


def dfa_ab_star_c():
    # 0 -a-> 1, 1 -b-> 1, 1 -c-> 2 (match), 2 -*-> 3 (non-live), 3 -*-> 3
    return build_dfa({0: {"a": 1}, 1: {"b": 1, "c": 2}, 2: {"*": 3}, 3: {"*": 3}}, [2], 4)


def dfa_abc():
    return build_dfa({0: {"a": 1}, 1: {"b": 2}, 2: {"c": 3}, 3: {"*": 4}, 4: {"*": 4}}, [3], 5)


def dfa_ab_opt():
    # ab? : 1 and 2 are matches
    return build_dfa({0: {"a": 1}, 1: {"b": 2, "*": 3}, 2: {"*": 3}, 3: {"*": 3}}, [1, 2], 4)


def dfa_ab_plus_c():
    return build_dfa({0: {"a": 1}, 1: {"b": 2}, 2: {"b": 2, "c": 3}, 3: {"*": 4}, 4: {"*": 4}}, [3], 5)


def masked(x):
    x = np.asarray(x)
    return [bool(np.isneginf(v)) for v in x]
