"""Host-side grammar compilers (CPU): regex -> anchored byte DFA and JSON
schema -> regex.

The cases of json_schema.rs:312-489 and logit_fsm.rs:330-536 are restated
with the same inputs and expectations (the reference checks them on
regex-automata's DFA; here they run on the native one, the masks through the
oracle's apply_mask). The DFA's language is further pinned against an
independent engine (Python's `re.fullmatch`) on many strings, and the regex
text of a few schemas against the reference's format strings
(json_schema.rs:44-53, 114-268) expanded by hand."""
import json
import random
import re
import unicodedata

import numpy as np
import pytest

from oracle import oracle as O
from zllm_amd import grammar as G


def accepts(schema, text):
    return G.HostDfa(G.schema_to_regex(schema)).full_match(text)


def rejects(schema, text):
    return not accepts(schema, text)


# ------------------------------------------------------------ json_schema.rs tests
def test_primitives():  # json_schema.rs:312-323
    assert accepts({"type": "boolean"}, "true")
    assert accepts({"type": "boolean"}, "false")
    assert rejects({"type": "boolean"}, "True")
    assert accepts({"type": "integer"}, "-42")
    assert rejects({"type": "integer"}, "4.5")
    assert accepts({"type": "number"}, "3.14")
    assert accepts({"type": "number"}, "-1.2e10")
    assert accepts({"type": "null"}, "null")
    assert accepts({"type": "string"}, '"hi"')
    assert rejects({"type": "string"}, "hi")


def test_string_with_escapes():  # :325-330
    assert accepts({"type": "string"}, r'"a\"b"')
    assert accepts({"type": "string"}, r'"tab\tend"')
    assert accepts({"type": "string"}, '"é"')


def test_enums():  # :332-340
    s = {"enum": ["red", "green", "blue"]}
    assert accepts(s, '"green"')
    assert rejects(s, '"yellow"')
    n = {"enum": [1, 2, 3]}
    assert accepts(n, "2")
    assert rejects(n, "4")


def test_const_literal():  # :342-347
    assert accepts({"const": "yes"}, '"yes"')
    assert rejects({"const": "yes"}, '"no"')


def test_simple_object():  # :349-362
    s = {"type": "object", "properties": {"name": {"type": "string"}, "age": {"type": "integer"}}}
    assert accepts(s, '{"name":"Ada","age":36}')
    assert accepts(s, '{"name": "Ada", "age": 36}')
    assert rejects(s, '{"age":36,"name":"Ada"}')
    assert rejects(s, '{"name":"Ada"}')
    assert rejects(s, '{"name":"Ada","age":"36"}')


def test_nested_object_and_array():  # :364-379
    s = {"type": "object", "properties": {
        "tags": {"type": "array", "items": {"type": "string"}},
        "meta": {"type": "object", "properties": {"ok": {"type": "boolean"}}}}}
    assert accepts(s, '{"tags":["a","b"],"meta":{"ok":true}}')
    assert accepts(s, '{"tags":[],"meta":{"ok":false}}')
    assert rejects(s, '{"tags":[1],"meta":{"ok":true}}')


def test_array_bounds():  # :381-388
    s = {"type": "array", "items": {"type": "integer"}, "minItems": 2, "maxItems": 3}
    assert rejects(s, "[1]")
    assert accepts(s, "[1,2]")
    assert accepts(s, "[1,2,3]")
    assert rejects(s, "[1,2,3,4]")


def test_enum_with_regex_meta_in_value():  # :390-397
    s = {"enum": ["a.b", "c+d"]}
    assert accepts(s, '"a.b"')
    assert rejects(s, '"axb"')
    assert accepts(s, '"c+d"')


def test_key_with_special_chars():  # :399-404
    s = {"type": "object", "properties": {"a.b": {"type": "integer"}}}
    assert accepts(s, '{"a.b":1}')
    assert rejects(s, '{"axb":1}')


def test_unsupported_constructs_error():  # :406-412
    for bad in ({"$ref": "#/x"}, {"anyOf": [{"type": "string"}]}, {"type": "object", "properties": {"x": {}}}, 42):
        with pytest.raises(G.GrammarError):
            G.schema_to_regex(bad)


def test_bare_object_type_is_object_only():  # :414-426
    s = {"type": "object"}
    assert accepts(s, "{}")
    assert accepts(s, '{"a":1}')
    assert accepts(s, '{"a":1,"b":[true,null,"x"]}')
    assert rejects(s, '"just a string"')
    assert rejects(s, "42")
    assert rejects(s, "[1,2]")


def test_pathologically_deep_schema_is_rejected_fast():  # :428-437
    s = {"type": "boolean"}
    for _ in range(32 + 8):
        s = {"type": "object", "properties": {"x": s}}
    with pytest.raises(G.GrammarError, match="nesting exceeds 32"):
        G.schema_to_regex(s)


def test_any_json_value():  # :439-449
    d = G.HostDfa(G.any_json_regex_default())
    for ok in ["true", "-3.5", '"hi"', '{"a":1,"b":[1,2,{"c":true}]}', "[]", "{}"]:
        assert d.full_match(ok), ok
    assert not d.full_match("{not json")


def test_tool_call_envelope_selects_and_constrains():  # :451-471
    tools = [("get_weather", {"type": "object", "properties": {"city": {"type": "string"}}}),
             ("get_time", {"type": "object", "properties": {}})]
    d = G.HostDfa(G.tool_call_envelope_regex(tools))
    assert d.full_match('{"name":"get_weather","arguments":{"city":"Paris"}}')
    assert d.full_match('{"name":"get_time","arguments":{}}')
    assert not d.full_match('{"name":"get_weather","arguments":{}}')
    assert not d.full_match('{"name":"nope","arguments":{}}')
    assert not d.full_match('{"arguments":{},"name":"get_time"}')
    with pytest.raises(G.GrammarError):
        G.tool_call_envelope_regex([])


def test_tool_call_shape_compiles():  # :473-488
    s = {"type": "object", "properties": {"location": {"type": "string"},
                                          "unit": {"enum": ["celsius", "fahrenheit"]}}}
    assert accepts(s, '{"location":"Paris","unit":"celsius"}')
    assert rejects(s, '{"location":"Paris","unit":"kelvin"}')


# ------------------------------------------------------------ regex text of the compiler
SP = " ?"
STRING = r'"([^"\\]|\\(["\\/bfnrt]|u[0-9a-fA-F]{4}))*"'
INTEGER = r"-?(0|[1-9][0-9]*)"


def test_schema_regex_text():
    """The reference's format strings (json_schema.rs:44-53, 177-268) expanded
    by hand for a few schemas."""
    assert G.schema_to_regex({"type": "string"}) == STRING
    assert G.schema_to_regex({"type": "integer"}) == INTEGER
    assert G.schema_to_regex({"type": "number"}) == r"-?(0|[1-9][0-9]*)(\.[0-9]+)?([eE][+-]?[0-9]+)?"
    assert G.schema_to_regex({"type": "boolean"}) == "(true|false)"
    assert G.schema_to_regex({"type": "null"}) == "null"
    assert G.schema_to_regex({"type": "string", "pattern": "[a-z]+"}) == '"[a-z]+"'
    obj = {"type": "object", "properties": {"name": {"type": "string"}, "age": {"type": "integer"}}}
    assert G.schema_to_regex(obj) == (r"\{" + SP + '"name"' + SP + ":" + SP + STRING + SP + "," + SP + '"age"' + SP
                                      + ":" + SP + INTEGER + SP + r"\}")
    assert G.schema_to_regex({"type": "object", "properties": {}}) == r"\{" + SP + r"\}"
    sep = SP + "," + SP
    arr = {"type": "array", "items": {"type": "integer"}, "minItems": 2, "maxItems": 3}
    two, three = INTEGER + sep + INTEGER, INTEGER + sep + INTEGER + sep + INTEGER
    assert G.schema_to_regex(arr) == r"\[" + SP + "(" + two + "|" + three + ")" + SP + r"\]"
    assert G.schema_to_regex({"type": "array", "items": {"type": "integer"}}) == \
        r"\[" + SP + "(" + INTEGER + "(" + sep + INTEGER + ")*)?" + SP + r"\]"
    assert G.schema_to_regex({"type": "array", "items": {"type": "integer"}, "minItems": 2}) == \
        r"\[" + SP + two + "(" + sep + INTEGER + ")*" + SP + r"\]"
    assert G.schema_to_regex({"type": "array", "items": {"type": "integer"}, "maxItems": 2}) == \
        r"\[" + SP + "((" + INTEGER + "|" + two + "))?" + SP + r"\]"
    assert G.schema_to_regex({"type": "array", "items": {"type": "integer"}, "maxItems": 0}) == \
        r"\[" + SP + r"\]"
    with pytest.raises(G.GrammarError, match="maxItems < minItems"):
        G.schema_to_regex({"type": "array", "items": {"type": "integer"}, "minItems": 3, "maxItems": 2})
    with pytest.raises(G.GrammarError, match="needs \"items\""):
        G.schema_to_regex({"type": "array"})
    # any_value(0): the four primitive shapes
    assert G.any_json_regex(0) == "(" + "|".join([STRING, r"-?(0|[1-9][0-9]*)(\.[0-9]+)?([eE][+-]?[0-9]+)?",
                                                  "(true|false)", "null"]) + ")"


def test_schema_declaration_order_and_duplicate_keys():
    """preserve_order (Cargo.toml:34): declaration order; a repeated key keeps
    its first position with the last value."""
    text = '{"type":"object","properties":{"b":{"type":"integer"},"a":{"type":"null"},"b":{"type":"boolean"}}}'
    d = G.HostDfa(G.schema_to_regex(text))
    assert d.full_match('{"b":true,"a":null}')
    assert not d.full_match('{"b":1,"a":null}')
    assert not d.full_match('{"a":null,"b":true}')


@pytest.mark.parametrize("value,text", [
    (100, "100"), (100.0, "100.0"), (1.5, "1.5"), (1e20, "1e20"), (1e16, "1e16"), (1e15, "1000000000000000.0"),
    (0.0001, "0.0001"), (1e-5, "0.00001"), (1e-6, "1e-6"), (1.25e-7, "1.25e-7"), (-2.5, "-2.5"), (123456.789, "123456.789"),
    ("a\nb", '"a\\nb"'), ("q\"x", '"q\\"x"'), ("\x01", '"\\u0001"'), ("é", '"é"'), (True, "true"), (None, "null"),
    ([1, "x"], '[1,"x"]'), ({"k": [None]}, '{"k":[null]}'),
])
def test_literal_serialisation(value, text):
    """const / enum literals are serde_json's compact output, regex-escaped
    (json_schema.rs:70-73): float layout of ryu, string escapes of serde_json."""
    d = G.HostDfa(G.schema_to_regex({"const": value}))
    assert d.full_match(text), G.schema_to_regex({"const": value})


def test_negative_zero_literal():
    # serde_json reads "-0" as the float -0.0 and writes it back as "-0.0"
    d = G.HostDfa(G.schema_to_regex('{"const": -0}'))
    assert d.full_match("-0.0") and not d.full_match("0") and not d.full_match("-0")


def test_invalid_schema_json_is_an_error():
    for bad in ["{not json}", '{"type": "string",}', '{"type": "string"} x', '"\\ud800"']:
        with pytest.raises(G.GrammarError):
            G.schema_to_regex(bad)


# ------------------------------------------------------------ regex compiler
def test_bad_patterns_are_errors():  # logit_fsm.rs:418-421 and the parser's own cases
    for bad in ["a(", "a)", "*a", "a{2,1}", "[a", "(?z)", "\\b", "\\1", "a{", "[z-a]"]:
        with pytest.raises(G.GrammarError):
            G.HostDfa(bad)


def test_size_limit_is_an_error():
    # (a|b)*a(a|b){n}: the DFA needs 2^(n+1) states
    with pytest.raises(G.GrammarError, match="size limit"):
        G.HostDfa("(a|b)*a(a|b){20}")


def test_dfa_is_minimal_and_dead_is_the_only_non_live_state():
    d = G.HostDfa("(ab|cd)*e(f|g)?")
    dfa = O.Dfa(d.trans, d.dead, d.accept)
    assert d.dead[0] == 1 and d.dead[1:].sum() == 0
    assert all(dfa.live[s] for s in range(1, d.nstates))
    # Moore equivalence over the final table: no two states merge
    blk = d.accept.astype(np.int64) + 1
    blk[0] = 0
    for _ in range(d.nstates):
        sig = {}
        nb = np.array([sig.setdefault((blk[s],) + tuple(blk[d.trans[s]]), len(sig)) for s in range(d.nstates)])
        if len(sig) == len(set(blk.tolist())):
            break
        blk = nb
    assert len(set(blk.tolist())) == d.nstates


_WHITE_SPACE = set(range(0x09, 0x0E)) | {0x20, 0x85, 0xA0, 0x1680, 0x2028, 0x2029, 0x202F, 0x205F, 0x3000} | \
    set(range(0x2000, 0x200B))   # PropList.txt White_Space

PATTERNS = [
    r"ab*c", r"ab?", r"(a|bc)*d", r"[a-c]{2,4}x?", r"(?:foo|bar)+baz", r"[^\"\\]*", r"\.\+\*\?\(\)\|\[\]\{\}\^\$",
    r"(?i)hello", r"a.c", r"(?s)a.c", r"[0-9]+(\.[0-9]+)?", r"x{3}", r"x{2,}", r"(ab){0,2}c",
    r"é+[à-ÿ]", r"[^a-z]", r"\x41é\U0001F600\u00e9", r"(a|)b", r"", r"a|b|", r"(?x) a b # comment",
    r"[\d_]+", r"\D\S\W", r"[a-]+", r"[]a]+", r"[^]a]", r"^ab$", r"a^b", r"a$b", r"(a$|b)c?",
]
ALPHABET = ["a", "b", "c", "d", "x", "f", "o", "r", "z", "A", "H", "e", "l", "L", "O", ".", "\n", "é", "à", "ÿ",
            "😀", "0", "5", "_", " ", '"', "\\", "]", "-", "^", "$", "+"]


def _strings(rng, n):
    out = [""]
    for _ in range(n):
        L = rng.randint(1, 7)
        out.append("".join(rng.choice(ALPHABET) for _ in range(L)))
    return out


_WORD_CATS = {"Lu", "Ll", "Lt", "Lm", "Lo", "Nl", "Mn", "Mc", "Me", "Nd", "Pc"}


def _uts_word(ch):
    c = ord(ch)
    return unicodedata.category(ch) in _WORD_CATS or c in (0x200C, 0x200D) or 0x24B6 <= c <= 0x24E9 or \
        0x1F130 <= c <= 0x1F149 or 0x1F150 <= c <= 0x1F169 or 0x1F170 <= c <= 0x1F189


def _py_agrees(ch):
    return (bool(re.fullmatch(r"\s", ch)) == (ord(ch) in _WHITE_SPACE)) and \
        (bool(re.fullmatch(r"\w", ch)) == _uts_word(ch))


@pytest.mark.parametrize("pat", PATTERNS)
def test_language_matches_python_re(pat):
    """Whole-text match of the DFA agrees with re.fullmatch (an independent
    engine) on random strings and on strings the DFA generates."""
    d = G.HostDfa(pat)
    py = re.compile(pat)   # Unicode classes: on ALPHABET Python's \d \s \w agree with UTS #18
    rng = random.Random(hash(pat) & 0xffff)
    cases = _strings(rng, 400)
    # strings accepted by the DFA, from random walks that end in an accepting state
    for _ in range(200):
        s, buf = d.start, bytearray()
        for _ in range(rng.randint(0, 12)):
            nxt = [b for b in range(256) if not d.dead[d.trans[s, b]]]
            if not nxt:
                break
            b = rng.choice(nxt)
            buf.append(b)
            s = int(d.trans[s, b])
        if d.accept[s]:
            cases.append(bytes(buf).decode("utf-8"))  # accepted text is valid UTF-8
    if "$" in pat or "^" in pat:
        cases = [c for c in cases if "\n" not in c]  # Python's $ also matches before a final newline
    # Python's \s and \w differ from UTS #18 on a few scalars (U+001C..U+001F
    # are Python spaces, No digits are Python word characters): those are
    # pinned by the Unicode-class tests below instead
    cases = [c for c in cases if all(_py_agrees(ch) for ch in c)]
    for text in cases:
        assert d.full_match(text) == bool(py.fullmatch(text)), (pat, text)


def test_posix_classes():
    d = G.HostDfa(r"[[:digit:]]+[[:^alpha:]]")
    assert d.full_match("12-") and d.full_match("07") and not d.full_match("12a") and not d.full_match("a1")


def test_invalid_utf8_is_rejected():
    d = G.HostDfa(r"[^a]*")
    assert d.full_match("é".encode("utf-8"))
    for bad in [b"\xc3", b"\xff", b"\xed\xa0\x80", b"\xc0\xaf", b"\xf4\x90\x80\x80"]:
        assert not d.full_match(bad)


# ------------------------------------------------------------ logit_fsm.rs tests (masks by the oracle)
TINY = [b"a", b"b", b"ab", b"c", None]
EOS = 5


def _fsm(pattern):
    d = G.HostDfa(pattern)
    return d, O.Dfa(d.trans, d.dead, d.accept), O.Vocab(TINY, EOS)


def _masked(dfa, voc, state):
    x = O.apply_mask(np.zeros(6, np.float32), dfa=dfa, vocab=voc, state=state)
    return [bool(np.isneginf(v)) for v in x]


def test_regex_masks_to_viable_prefixes():  # logit_fsm.rs:370-379
    d, dfa, voc = _fsm("ab*c")
    assert _masked(dfa, voc, d.start) == [False, True, False, True, True, True]


def test_regex_advance_transitions_and_accepts():  # :381-396
    d, dfa, voc = _fsm("ab*c")
    s = O.advance(dfa, voc, d.start, 0)
    assert _masked(dfa, voc, s) == [True, False, True, False, True, True]
    s = O.advance(dfa, voc, s, 1)
    s = O.advance(dfa, voc, s, 3)
    assert _masked(dfa, voc, s) == [True, True, True, True, True, False]


def test_regex_multibyte_token_walks_whole_surface():  # :398-406
    d, dfa, voc = _fsm("abc")
    s = O.advance(dfa, voc, d.start, 2)
    assert _masked(dfa, voc, s) == [True, True, True, False, True, True]


def test_regex_optional_suffix_allows_eos_and_continuation():  # :408-416
    d, dfa, voc = _fsm("ab?")
    s = O.advance(dfa, voc, d.start, 0)
    assert _masked(dfa, voc, s) == [True, False, True, True, True, False]


def test_regex_constrains_a_greedy_loop_end_to_end():  # :492-536
    d, dfa, voc = _fsm("ab+c")
    prefs = [[3, 1, 0, 2, 4, 5], [0, 2, 1, 3, 4, 5], [3, 1, 0, 2, 4, 5], [0, 1, 2, 3, 4, 5]]
    out, s = [], d.start
    for pref in prefs:
        x = np.zeros(6, np.float32)
        for rank, i in enumerate(pref):
            x[i] = 10.0 - rank
        x = O.apply_mask(x, dfa=dfa, vocab=voc, state=s)
        pick = int(max(range(6), key=lambda i: (x[i], i)))
        if pick == 5:
            break
        out.append(pick)
        s = O.advance(dfa, voc, s, pick)
    assert out == [0, 1, 3]


def test_json_modes_compile_on_the_tiny_table():  # :430-451 (the compile step; masks need a GPU context)
    for pattern in [G.any_json_regex_default(), G.schema_to_regex('{"type":"boolean"}')]:
        d = G.HostDfa(pattern)
        dfa, voc = O.Dfa(d.trans, d.dead, d.accept), O.Vocab(TINY, EOS)
        # nothing of the tiny table starts JSON except nothing: only EOS stays open (forced stop)
        assert _masked(dfa, voc, d.start)[:5] == [True] * 5


def test_braced_escapes():
    assert G.HostDfa(r"\u{1F600}\x{41}\x42").full_match("😀AB")


# ------------------------------------------------------------ Unicode classes
# regex-syntax's Unicode mode (logit_fsm.rs:73-86 builds with the defaults):
# \d = \p{Nd}, \s = White_Space, \w = UTS #18 Annex C word characters,
# \p{..} general categories, simple case folding. Expected sets come from
# unicodedata's categories directly (an engine-independent restatement) and
# from Python's re where its semantics coincide.


def _bmp():
    return [c for c in range(0x10000) if not 0xD800 <= c <= 0xDFFF]


def _single_char_language(pat):
    """The BMP scalars c for which the DFA of `pat` fully matches chr(c)."""
    d = G.HostDfa(pat)
    out = set()
    for c in _bmp():
        s = d.start
        for b in chr(c).encode("utf-8"):
            s = int(d.trans[s, b])
        if not d.dead[s] and d.accept[s]:
            out.add(c)
    return out


def test_unicode_digit_class_is_nd():
    want = {c for c in _bmp() if unicodedata.category(chr(c)) == "Nd"}
    assert _single_char_language(r"\d") == want
    assert _single_char_language(r"\p{Nd}") == want
    d = G.HostDfa(r"\d+")
    assert d.full_match("٣١٤") and d.full_match("१२") and not d.full_match("²") and not d.full_match("Ⅳ")


def test_unicode_space_class_is_white_space():
    assert _single_char_language(r"\s") == {c for c in _WHITE_SPACE if c < 0x10000}
    d = G.HostDfa(r"a\sb")
    assert d.full_match("a\u3000b") and d.full_match("a\u00a0b") and not d.full_match("a\u001cb")


def test_unicode_word_class():
    L = {"Lu", "Ll", "Lt", "Lm", "Lo", "Nl", "Mn", "Mc", "Me", "Nd", "Pc"}
    want = {c for c in _bmp() if unicodedata.category(chr(c)) in L} | {0x200C, 0x200D} | set(range(0x24B6, 0x24EA))
    got = _single_char_language(r"\w")
    assert got == want
    assert 0x00B2 not in got          # superscript two (No): not a word character
    assert ord("‿") in got and ord("é") in got and ord("中") in got


def test_unicode_general_categories():
    for pat, cats in [(r"\p{L}", {"Lu", "Ll", "Lt", "Lm", "Lo"}), (r"\pN", {"Nd", "Nl", "No"}),
                      (r"\p{Lu}", {"Lu"}), (r"\p{Uppercase_Letter}", {"Lu"}), (r"\p{gc=Sc}", {"Sc"}),
                      (r"[\p{Zs}\p{Pd}]", {"Zs", "Pd"})]:
        want = {c for c in _bmp() if unicodedata.category(chr(c)) in cats}
        assert _single_char_language(pat) == want, pat
    notn = _single_char_language(r"\P{N}")
    assert ord("a") in notn and ord("٣") not in notn and ord("²") not in notn
    for bad in [r"\p{Greek}", r"\p{Alphabetic}", r"\p{", r"\bword\b"]:
        with pytest.raises(G.GrammarError):
            G.HostDfa(bad)


def test_unicode_case_folding():
    d = G.HostDfa(r"(?i)k")
    assert d.full_match("k") and d.full_match("K") and d.full_match("\u212a")   # Kelvin sign folds to k
    d = G.HostDfa(r"(?i)s")
    assert d.full_match("S") and d.full_match("\u017f")                       # long s
    d = G.HostDfa(r"(?i)σ+")
    assert d.full_match("Σσς")
    d = G.HostDfa(r"(?i)µ")
    assert d.full_match("μ") and d.full_match("Μ")
    d = G.HostDfa(r"(?i)ß")
    assert d.full_match("ẞ")
    d = G.HostDfa(r"(?i)i")
    assert d.full_match("I") and not d.full_match("ı") and not d.full_match("İ")  # no Turkic folds
    # letters of Latin-1, Greek and Cyrillic: case-insensitive single-letter
    # languages agree with Python's re.IGNORECASE
    block = list(range(0x41, 0x5B)) + list(range(0x61, 0x7B)) + list(range(0xC0, 0xFF)) + \
        list(range(0x391, 0x3AA)) + list(range(0x3B1, 0x3CA)) + list(range(0x410, 0x450))
    block = [c for c in block if c not in (0xD7, 0xF7)]
    for c in block[::3]:
        pat = "(?i)" + re.escape(chr(c))
        d = G.HostDfa(pat)
        py = re.compile(pat)
        for o in block:
            assert d.full_match(chr(o)) == bool(py.fullmatch(chr(o))), (hex(c), hex(o))


# ------------------------------------------------------------ look-around and (?-u)
# regex-automata's dense DFA (logit_fsm.rs:73-86) supports the line anchors of
# (?m) / (?mR) and ASCII word boundaries, and refuses Unicode ones at build
# time. Languages are pinned by brute force: every string of up to 5 symbols
# over a small alphabet, whole-text match against Python's re on bytes (its
# \b \w \s on bytes are the ASCII ones, its (?m) ^ $ are regex-syntax's
# StartLF / EndLF); the forms Python lacks are written with its look-around.
_LOOK_ALPHABET = [b"a", b"Z", b"1", b"_", b" ", b"\n", b"\r", "é".encode("utf-8"), b"-"]

_PY_CRLF_START = rb"(?:(?<![\s\S])|(?<=\n)|(?<=\r)(?!\n))"
_PY_CRLF_END = rb"(?:(?![\s\S])|(?=\r)|(?<!\r)(?=\n))"

LOOK_PATTERNS = [
    (r"(?-u)(?:\b\w+\b|\s|-)*", rb"(?:\b\w+\b|\s|-)*"),
    (r"(?-u)(?:a|\B|_| |\n|\b1)*", rb"(?:a|\B|_| |\n|\b1)*"),
    (r"(?-u)\<\w+\>(?: \<\w+\>)*", rb"(?<!\w)(?=\w)\w+(?<=\w)(?!\w)(?: (?<!\w)(?=\w)\w+(?<=\w)(?!\w))*"),
    (r"(?-u)(?:\b{start}a|\b{end}-|\s)*", rb"(?:(?<!\w)(?=\w)a|(?<=\w)(?!\w)-|\s)*"),
    (r"(?-u)\b{start-half}[a_ ]*\b{end-half}", rb"(?<!\w)[a_ ]*(?!\w)"),
    (r"(?-u)(?:a\>|\<1|_| )*", rb"(?:a(?<=\w)(?!\w)|(?<!\w)(?=\w)1|_| )*"),
    (r"(?-u)(?:a\b{end}|\b{start}1|_| )*", rb"(?:a(?<=\w)(?!\w)|(?<!\w)(?=\w)1|_| )*"),
    (r"(?-u)(?:a\b{end-half}|\b{start-half}1| |_)*", rb"(?:a(?!\w)|(?<!\w)1| |_)*"),
    (r"(?-u:\b)(?:é|a|1)+", rb"\b(?:\xc3\xa9|a|1)+"),
    (r"(?m)^a*$(?:\n^a*$)*", rb"(?m)^a*$(?:\n^a*$)*"),
    (r"(?m)(?:^|a|\n|\r|$|_$)*", rb"(?m)(?:^|a|\n|\r|$|_$)*"),
    (r"(?m)(?:^_|a$|\n|\r|é)*", rb"(?m)(?:^_|a$|\n|\r|\xc3\xa9)*"),
    (r"(?mR)(?:^a|_$|\n|\r)*", rb"(?:" + _PY_CRLF_START + rb"a|_" + _PY_CRLF_END + rb"|\n|\r)*"),
    (r"(?mR)(?:^|$|\r|\n|a)*", rb"(?:" + _PY_CRLF_START + rb"|" + _PY_CRLF_END + rb"|\r|\n|a)*"),
    (r"(?m:^a)\n(?-m:^a)", rb"(?m:^a)\n(?<![\s\S])a"),
    (r"\Aa\z|(?m)^b$", rb"(?m)(?<![\s\S])a(?![\s\S])|^b$"),
    (r"(?i-u)[k-m]+\w", rb"(?i)[k-m]+\w"),
    (r"(?-u)[\w--\d]+ \s", rb"[A-Za-z_]+ \s"),
]


def _all_strings(alphabet, n):
    out, layer = [b""], [b""]
    for _ in range(n):
        layer = [s + a for s in layer for a in alphabet]
        out += layer
    return out


@pytest.mark.parametrize("pat,py", LOOK_PATTERNS)
def test_look_around_matches_python_re(pat, py):
    d = G.HostDfa(pat)
    rx = re.compile(py)
    texts = _all_strings(_LOOK_ALPHABET, 4) + [b"ab 1_\n", b"a\r\na", b"a\n\r_", b"Za -a\r"]
    for t in texts:
        assert d.full_match(t) == bool(rx.fullmatch(t)), (pat, t)


def test_look_around_known_answers():
    # (?mR): '\r' and '\n' both end lines, and ^ / $ never match between "\r\n"
    d = G.HostDfa(r"(?mR)a$\r\n^b")
    assert d.full_match("a\r\nb")
    assert not G.HostDfa(r"(?mR)a\r^\nb").full_match("a\r\nb")
    assert not G.HostDfa(r"(?mR)a\r$\nb").full_match("a\r\nb")
    assert G.HostDfa(r"(?mR)a\r^b").full_match("a\rb")
    assert G.HostDfa(r"(?m)a\r^\nb").full_match("a\r\nb") is False      # (?m) alone: only '\n' starts a line
    assert G.HostDfa(r"(?m)a\n^\nb").full_match("a\n\nb")
    # without (?m), ^ $ are \A \z
    assert not G.HostDfa(r"a\n^b").full_match("a\nb")
    assert not G.HostDfa(r"a$\nb").full_match("a\nb")
    # ASCII word boundaries: bytes above 0x7F are not word bytes
    assert G.HostDfa(r"(?-u:\b)é").full_match("é") is False
    assert G.HostDfa(r"a(?-u:\b)é").full_match("aé")
    assert G.HostDfa(r"(?-u:\B)").full_match("") and not G.HostDfa(r"(?-u:\b)").full_match("")
    # the masks see the assertions: after "a", "b" may not follow a \b
    d = G.HostDfa(r"(?-u)a\b[a-z ]*")
    s = d.walk(d.start, b"a")
    assert d.walk(s, b"b") is None and d.walk(s, b" ") is not None


def test_unicode_mode_off():
    d = G.HostDfa(r"(?-u)\w+")
    assert d.full_match("ab_9") and not d.full_match("é")
    assert G.HostDfa(r"(?-u)\d").full_match("5") and not G.HostDfa(r"(?-u)\d").full_match("٣")
    assert G.HostDfa(r"(?-u)\s").full_match("\x0b") and not G.HostDfa(r"(?-u)\s").full_match("\u3000")
    d = G.HostDfa(r"(?i-u)k")
    assert d.full_match("k") and d.full_match("K") and not d.full_match("\u212a")
    d = G.HostDfa(r"(?i)k(?-u:k)")
    assert d.full_match("\u212ak") and not d.full_match("k\u212a")
    assert G.HostDfa(r"(?-u)é\x{e9}\u00e9").full_match("ééé")   # literals outside classes stay scalars
    assert G.HostDfa(r"(?-u)(?u:.)").full_match("é")
    assert G.HostDfa(r"(?-u:[[:^alpha:]&&[0-9]])").full_match("5")


@pytest.mark.parametrize("bad", [
    r"\b", r"\B", r"\<", r"\>", r"\b{start}", r"(?-u:\b{foo})", r"(?-u:\b{start)",   # Unicode boundaries, bad names
    r"(?-u).", r"(?s-u).", r"(?-u)\W", r"(?-u)\D", r"(?-u)[^a]", r"(?-u)[\S]", r"(?-u)\xFF", r"(?-u)[\x80]",
    r"(?-u)[é]", r"(?-u)\pL", r"(?-u:[[:^alpha:]])", r"(?-u)[[^a]&&b]", r"[\b]",
])
def test_look_and_byte_mode_errors(bad):
    with pytest.raises(G.GrammarError):
        G.HostDfa(bad)


# ------------------------------------------------------------ class set operations
# [A&&B] [A--B] [A~~B]: equal precedence, left to right, looser than union;
# negation applies to the result. Expected sets come from Python set
# arithmetic over the single-scalar languages of the operands.
_SET_UNIVERSE = [chr(c) for c in list(range(0x20, 0x250)) + [0x391, 0x3B1, 0x3C3, 0x3C2, 0x410, 0x430, 0x212A,
                                                              0x17F, 0x660, 0x966, 0x3000]]


def _lang(pat):
    d = G.HostDfa(pat)
    return {c for c in _SET_UNIVERSE if d.full_match(c)}


@pytest.mark.parametrize("a,op,b", [
    (r"\w", "&&", r"\d"), (r"\p{L}", "--", r"[a-z]"), (r"[a-g]", "~~", r"[c-z]"), (r"\pL", "&&", r"\p{Lu}"),
    (r"[\x20-\x7e]", "--", r"\w"), (r"\s", "~~", r"[\t-\r]"), (r"[^a-z]", "&&", r"[\x20-\x7a]"),
])
def test_class_set_operations(a, op, b):
    A, B = _lang(a), _lang(b)
    want = {"&&": A & B, "--": A - B, "~~": A ^ B}[op]
    assert _lang("[" + a + op + b + "]") == want
    assert _lang("[^" + a + op + b + "]") == set(_SET_UNIVERSE) - want


def test_class_set_operation_precedence():
    # union binds tighter: [ab&&bc] == [[ab]&&[bc]]; operators go left to right
    assert _lang(r"[ab&&bc]") == {"b"}
    assert _lang(r"[a-z--b&&c-e]") == {"c", "d", "e"}
    assert _lang(r"[a-z&&c-e--d]") == {"c", "e"}
    assert _lang(r"[a-c~~b-d~~c]") == {"a", "c", "d"}
    assert _lang(r"[[a-c]--[b]]") == {"a", "c"}
    assert _lang(r"[a-]") == {"a", "-"}
    # case folding applies to each operand before the operation
    assert _lang(r"(?i)[a-z--k]") == _lang(r"(?i)[a-jl-z]")
    assert "\u212a" not in _lang(r"(?i)[a-z--k]") and "\u017f" in _lang(r"(?i)[a-z--k]")
