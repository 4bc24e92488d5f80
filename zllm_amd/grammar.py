"""Grammar compilers over the C ABI (host only, no GPU): regex -> anchored
byte DFA (replacing regex-automata in logit_fsm.rs:62-91) and the JSON-schema
-> regex compiler of json_schema.rs (schema_to_regex :78, any_json_regex :84,
any_json_regex_default :89, tool_call_envelope_regex :99)."""
import ctypes as C
import json
from typing import Any, List, Sequence, Tuple, Union

import numpy as np

from ._lib import ZS_ELIMIT, lib

ANY_JSON_DEFAULT_DEPTH = 5  # json_schema.rs:41


class GrammarError(ValueError):
    """A user-facing compile error (the reference's Err(String))."""


def _string_call(fn, *args, err=True):
    need = C.c_size_t(0)
    cap = 1 << 16
    while True:
        buf = C.create_string_buffer(cap)
        ebuf = C.create_string_buffer(1024)
        extra = (ebuf, 1024) if err else ()
        rc = fn(*args, buf, cap, C.byref(need), *extra)
        if rc == ZS_ELIMIT and need.value > cap:
            cap = need.value
            continue
        if rc != 0:
            raise GrammarError(ebuf.value.decode("utf-8", "replace") if err else f"error {rc}")
        return buf.value.decode("utf-8")


def schema_to_regex(schema: Union[str, Any]) -> str:
    """json_schema.rs:78-80 (a schema given as JSON text or a Python value)."""
    text = schema if isinstance(schema, str) else json.dumps(schema, ensure_ascii=False)
    b = text.encode("utf-8")
    return _string_call(lib().zs_json_schema_regex, b, len(b))


def any_json_regex(depth: int) -> str:
    """json_schema.rs:84-86."""
    return _string_call(lib().zs_any_json_regex, int(depth), err=False)


def any_json_regex_default() -> str:
    """json_schema.rs:89-91."""
    return any_json_regex(ANY_JSON_DEFAULT_DEPTH)


def tool_call_envelope_regex(tools: Sequence[Tuple[str, Union[str, Any]]]) -> str:
    """json_schema.rs:99-112: (name, parameters schema) pairs."""
    n = len(tools)
    names = (C.c_char_p * max(n, 1))(*[t[0].encode("utf-8") for t in tools])
    schemas = (C.c_char_p * max(n, 1))(*[(t[1] if isinstance(t[1], str) else json.dumps(t[1], ensure_ascii=False))
                                         .encode("utf-8") for t in tools])
    return _string_call(lib().zs_tool_call_envelope_regex, names, schemas, n)


class HostDfa:
    """Anchored byte DFA of "the whole text matches `pattern`": trans[S, 256],
    dead (state 0), accept, start. Build the device copy with
    engine.ByteDfa(ctx, dfa.trans, dfa.dead, dfa.accept)."""

    def __init__(self, pattern: str):
        b = pattern.encode("utf-8")
        h = C.c_void_p()
        ebuf = C.create_string_buffer(1024)
        rc = lib().zs_regex_compile(b, len(b), C.byref(h), ebuf, 1024)
        if rc != 0:
            raise GrammarError(ebuf.value.decode("utf-8", "replace"))
        try:
            n, st = C.c_uint32(), C.c_uint32()
            lib().zs_grammar_info(h, C.byref(n), C.byref(st))
            S = n.value
            self.nstates, self.start = S, st.value
            self.trans = np.ctypeslib.as_array(C.cast(lib().zs_grammar_trans(h), C.POINTER(C.c_uint32)),
                                               (S, 256)).copy()
            self.accept = np.ctypeslib.as_array(C.cast(lib().zs_grammar_accept(h), C.POINTER(C.c_uint8)), (S,)).copy()
            self.dead = np.ctypeslib.as_array(C.cast(lib().zs_grammar_dead(h), C.POINTER(C.c_uint8)), (S,)).copy()
        finally:
            lib().zs_grammar_destroy(h)
        self.pattern = pattern

    def walk(self, state: int, data: bytes):
        """logit_fsm.rs:97-106: the state after `data`, or None at the dead state."""
        s = state
        for byte in data:
            s = int(self.trans[s, byte])
            if self.dead[s]:
                return None
        return s

    def full_match(self, text: Union[str, bytes]) -> bool:
        """Anchored whole-text match (json_schema.rs:279-304 full_match)."""
        data = text.encode("utf-8") if isinstance(text, str) else text
        s = self.walk(self.start, data)
        return s is not None and bool(self.accept[s])


def compile_regex(pattern: str) -> HostDfa:
    return HostDfa(pattern)
