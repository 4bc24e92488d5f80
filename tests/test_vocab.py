"""Grammar byte table of a real vocabulary (CPU): zs_token_table_from_json /
_from_gguf against HF tokenizers' own decode.

The reference builds the table as decode([id], skip_special_tokens=true) per
id (tokenizer.rs:108-117) with the Rust `tokenizers` crate (0.21.4). The
Python `tokenizers` package here wraps the same crate (0.22.2), so the
expected tables come from its decode on tokenizers built in the test (no
model files exist offline): byte-level BPE with special and plain added
tokens, SentencePiece-style byte fallback, Metaspace, WordPiece, Unigram and
decoder-less vocabularies. The GGUF path is checked against the construction
of gguf_vocab.rs:75-171 (BPE over the embedded tokens, ByteLevel decoder,
type-3 tokens special, type-4 tokens added) done with the same package over a
GGUF file written here."""
import json
import random
import struct

import numpy as np
import pytest

tokenizers = pytest.importorskip("tokenizers")
from tokenizers import Tokenizer, decoders, models, pre_tokenizers, trainers  # noqa: E402

from zllm_amd.vocab import HostTokenTable, TokenTableError  # noqa: E402


def _corpus(seed, n=3000):
    rng = random.Random(seed)
    words = ["the", "grammar", "token", "json", "schema", "décodé", "naïve", "数据", "模型", "🙂", "😀x", "über",
             "Straße", "{\"a\":", "1.5e-3", "\n", "\t", "  ", "can't", "it's", "ÿ", " ", "ending."]
    return [" ".join(rng.choice(words) for _ in range(rng.randint(1, 12))) for _ in range(n)]


def expected_table(tok):
    out = []
    for i in range(tok.get_vocab_size(with_added_tokens=True)):
        s = tok.decode([i], skip_special_tokens=True)
        out.append(s.encode("utf-8") if s and "�" not in s else None)
    return out


def eos_of(tok):
    for t in ("</s>", "<|end_of_text|>", "<|eot_id|>"):
        i = tok.token_to_id(t)
        if i is not None:
            return i
    return None


def check(tok):
    got = HostTokenTable.from_tokenizer_json(tok.to_str())
    want = expected_table(tok)
    assert got.ntab == len(want)
    toks = got.tokens()
    bad = [(i, toks[i], want[i]) for i in range(len(want)) if toks[i] != want[i]]
    assert not bad, bad[:10]
    assert got.eos == eos_of(tok)
    return got


def byte_level_bpe(seed=1, vocab_size=1500):
    tok = Tokenizer(models.BPE())
    tok.pre_tokenizer = pre_tokenizers.ByteLevel(add_prefix_space=False)
    tok.decoder = decoders.ByteLevel()
    trainer = trainers.BpeTrainer(vocab_size=vocab_size, special_tokens=["<|end_of_text|>", "<|eot_id|>"],
                                  initial_alphabet=pre_tokenizers.ByteLevel.alphabet(), show_progress=False)
    tok.train_from_iterator(_corpus(seed), trainer)
    tok.add_tokens(["<tool_call>", " spaced tok", "añadido"])
    tok.add_special_tokens(["<|im_end|>"])
    return tok


def test_byte_level_bpe():
    got = check(byte_level_bpe())
    # partial UTF-8 pieces are None, whole characters are kept
    assert any(v == 0 for v in got.valid) and any(v == 1 for v in got.valid)


def _sp_vocab():
    pieces = ["<unk>", "<s>", "</s>"] + [f"<0x{b:02X}>" for b in range(256)]
    pieces += ["▁", "▁the", "▁a", "ing", "é", "▁é", "▁▁", "x▁y", "数", "▁数据", "▁naïve", "s", "t", "▁to", "ken"]
    return {p: i for i, p in enumerate(pieces)}


def test_sentencepiece_byte_fallback():
    tok = Tokenizer(models.BPE(vocab=_sp_vocab(), merges=[], byte_fallback=True, unk_token="<unk>"))
    tok.pre_tokenizer = pre_tokenizers.Metaspace()
    tok.decoder = decoders.Sequence([decoders.Replace("▁", " "), decoders.ByteFallback(), decoders.Fuse(),
                                     decoders.Strip(" ", 1, 0)])
    tok.add_special_tokens(["<s>", "</s>", "<unk>"])
    got = check(tok)
    assert got.tokens()[3 + 0x41] == b"A"       # <0x41>
    assert got.tokens()[3 + 0xE2] is None       # a lone lead byte
    assert got.eos == 2


@pytest.mark.parametrize("scheme", ["always", "first", "never"])
def test_metaspace(scheme):
    tok = Tokenizer(models.BPE(vocab=_sp_vocab(), merges=[], unk_token="<unk>"))
    tok.decoder = decoders.Metaspace(replacement="▁", prepend_scheme=scheme)
    check(tok)


def test_wordpiece():
    vocab = {w: i for i, w in enumerate(["[UNK]", "[CLS]", "hello", "##ing", "##s", "world", ".", "do", "n't", "'",
                                         "##.", "a ."])}
    tok = Tokenizer(models.WordPiece(vocab=vocab, unk_token="[UNK]"))
    tok.decoder = decoders.WordPiece(prefix="##")
    tok.add_special_tokens(["[CLS]"])
    check(tok)


def test_unigram_and_no_decoder():
    tok = Tokenizer(models.Unigram([("<unk>", 0.0), ("▁hi", -1.0), ("there", -2.0), ("▁é", -2.5), ("x", -3.0)],
                                   unk_id=0))
    tok.decoder = decoders.Metaspace()
    check(tok)
    plain = Tokenizer(models.Unigram([("<unk>", 0.0), ("a b", -1.0), ("c", -2.0)], unk_id=0))
    check(plain)


def test_bpe_suffix_decoder():
    tok = Tokenizer(models.BPE(vocab={"<unk>": 0, "lo</w>": 1, "w": 2, "</w>": 3}, merges=[], unk_token="<unk>"))
    tok.decoder = decoders.BPEDecoder(suffix="</w>")
    check(tok)


def test_errors():
    with pytest.raises(TokenTableError):
        HostTokenTable.from_tokenizer_json("{not json")
    with pytest.raises(TokenTableError, match="not supported"):
        HostTokenTable.from_tokenizer_json(json.dumps({"model": {"type": "BPE", "vocab": {"a": 0}},
                                                       "decoder": {"type": "CTC"}}))


# ------------------------------------------------------------ GGUF
def _gguf_str(s):
    b = s.encode("utf-8")
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, kvs):
    """GGUF v3 header with metadata only (no tensors)."""
    out = b"GGUF" + struct.pack("<IQQ", 3, 0, len(kvs))
    for key, (typ, val) in kvs.items():
        out += _gguf_str(key) + struct.pack("<I", typ)
        if typ == 8:
            out += _gguf_str(val)
        elif typ == 9:
            et, items = val
            out += struct.pack("<IQ", et, len(items))
            for it in items:
                out += _gguf_str(it) if et == 8 else struct.pack({4: "<I", 5: "<i", 6: "<f", 7: "<?"}[et], it)
        else:
            out += struct.pack({4: "<I", 5: "<i", 6: "<f", 7: "<?", 10: "<Q", 11: "<q", 12: "<d"}[typ], val)
    with open(path, "wb") as f:
        f.write(out)


def test_gguf_byte_level(tmp_path):
    src = byte_level_bpe(seed=3, vocab_size=800)
    vocab = src.get_vocab(with_added_tokens=True)
    tokens = [None] * len(vocab)
    for t, i in vocab.items():
        tokens[i] = t
    types = [1] * len(tokens)
    for i, t in enumerate(tokens):
        if t in ("<|end_of_text|>", "<|eot_id|>", "<|im_end|>"):
            types[i] = 3
        elif t in ("<tool_call>", " spaced tok"):
            types[i] = 4
    path = str(tmp_path / "v.gguf")
    write_gguf(path, {
        "general.architecture": (8, "llama"),
        "llama.context_length": (4, 8192),
        "llama.rope.freq_base": (6, 500000.0),
        "tokenizer.ggml.model": (8, "gpt2"),
        "tokenizer.ggml.pre": (8, "llama-bpe"),
        "tokenizer.ggml.tokens": (9, (8, tokens)),
        "tokenizer.ggml.token_type": (9, (5, types)),
        "tokenizer.ggml.merges": (9, (8, ["a b", "c d"])),
        "tokenizer.ggml.add_bos_token": (7, True),
        "tokenizer.ggml.bos_token_id": (4, 0),
        "general.size": (10, 12345),
    })
    got = HostTokenTable.from_gguf(path)
    # gguf_vocab.rs:75-171 with the same crate: BPE over the tokens, ByteLevel
    # decoder, control tokens special, user-defined tokens added
    ref = Tokenizer(models.BPE(vocab={t: i for i, t in enumerate(tokens)}, merges=[]))
    ref.decoder = decoders.ByteLevel()
    ref.add_special_tokens([t for t, ty in zip(tokens, types) if ty == 3])
    ref.add_tokens([t for t, ty in zip(tokens, types) if ty == 4])
    want = expected_table(ref)
    assert got.tokens() == want
    assert got.eos == eos_of(ref)


def test_gguf_spm_vocab_is_refused(tmp_path):
    path = str(tmp_path / "spm.gguf")
    write_gguf(path, {"tokenizer.ggml.model": (8, "llama"), "tokenizer.ggml.tokens": (9, (8, ["a", "b"]))})
    with pytest.raises(TokenTableError, match="only byte-level BPE"):
        HostTokenTable.from_gguf(path)
    with pytest.raises(TokenTableError):
        HostTokenTable.from_gguf(str(tmp_path / "missing.gguf"))
