// zs_tokens.cpp -- the grammar byte table of a real vocabulary, on the host.
//
// Restates LlamaTokenizer::token_bytes_table (tokenizer.rs:108-117): for every
// id below get_vocab_size(true), decode([id]) with special tokens skipped;
// the surface bytes, or None when the text is empty or holds U+FFFD (special
// tokens, partial byte-level pieces). The decode is HF tokenizers' (0.21, the
// reference's dependency): the id's token string (added tokens first, then
// the model's vocab), dropped when its content is a special added token, then
// the tokenizer.json decoder chain. Supported decoders: ByteLevel, Metaspace,
// ByteFallback, Fuse, Strip, Replace (string patterns), WordPiece, BPEDecoder
// and Sequence; no decoder joins with " ".
//
// Sources: a tokenizer.json document, or the vocab embedded in a GGUF file
// (gguf_vocab.rs:75-171: byte-level BPE "gpt2" vocabs only; control tokens
// (type 3) are special added tokens, user-defined ones (4) plain added
// tokens; the decoder is ByteLevel). The EOS id is eos_token_id
// (tokenizer.rs:52-57): the first of "</s>", "<|end_of_text|>", "<|eot_id|>".
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <new>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>
#include "../../include/zs.h"
#include "zs_json.h"

using zsj::JV;

struct zs_token_table {
    std::vector<uint32_t> offsets;
    std::vector<uint8_t> bytes;
    std::vector<uint8_t> valid;
    int64_t eos = -1;
    // decode([id]) text of every id, U+FFFD pieces and "" of specials
    // included (what the logprobs JSON shows, rest.rs:1714)
    std::vector<uint32_t> text_offsets;
    std::vector<uint8_t> text;
};

namespace {

struct TokError {
    std::string msg;
};

// ---------------------------------------------------------------- UTF-8
void put_utf8(std::string& o, uint32_t cp) {
    if (cp < 0x80) o += (char)cp;
    else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 0x3f)); }
    else if (cp < 0x10000) {
        o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 0x3f)); o += (char)(0x80 | (cp & 0x3f));
    } else {
        o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 0x3f));
        o += (char)(0x80 | ((cp >> 6) & 0x3f)); o += (char)(0x80 | (cp & 0x3f));
    }
}
// scalars of a valid UTF-8 string
std::vector<uint32_t> chars_of(const std::string& s) {
    std::vector<uint32_t> o;
    for (size_t i = 0; i < s.size();) {
        const unsigned char c = (unsigned char)s[i];
        int n = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : 4;
        uint32_t cp = n == 1 ? c : n == 2 ? (c & 0x1f) : n == 3 ? (c & 0x0f) : (c & 0x07);
        for (int k = 1; k < n && i + k < s.size(); k++) cp = (cp << 6) | ((unsigned char)s[i + k] & 0x3f);
        o.push_back(cp);
        i += n;
    }
    return o;
}
std::string from_chars(const std::vector<uint32_t>& v, size_t a, size_t b) {
    std::string o;
    for (size_t i = a; i < b; i++) put_utf8(o, v[i]);
    return o;
}
// String::from_utf8_lossy: each maximal invalid subpart becomes U+FFFD
std::string utf8_lossy(const std::string& b) {
    std::string o;
    const size_t n = b.size();
    size_t i = 0;
    while (i < n) {
        const unsigned char c = (unsigned char)b[i];
        if (c < 0x80) { o += (char)c; i++; continue; }
        int need;
        unsigned char lo = 0x80, hi = 0xBF;
        if (c >= 0xC2 && c <= 0xDF) need = 1;
        else if (c == 0xE0) { need = 2; lo = 0xA0; }
        else if (c >= 0xE1 && c <= 0xEC) need = 2;
        else if (c == 0xED) { need = 2; hi = 0x9F; }
        else if (c >= 0xEE && c <= 0xEF) need = 2;
        else if (c == 0xF0) { need = 3; lo = 0x90; }
        else if (c >= 0xF1 && c <= 0xF3) need = 3;
        else if (c == 0xF4) { need = 3; hi = 0x8F; }
        else { o += "\xEF\xBF\xBD"; i++; continue; }
        size_t j = i + 1;
        int got = 0;
        while (got < need && j < n) {
            const unsigned char d = (unsigned char)b[j];
            const unsigned char l = got == 0 ? lo : 0x80, h = got == 0 ? hi : 0xBF;
            if (d < l || d > h) break;
            j++;
            got++;
        }
        if (got == need) o.append(b, i, j - i);
        else o += "\xEF\xBF\xBD";
        i = j;
    }
    return o;
}

// GPT-2 byte <-> printable-character map (byte-level BPE)
struct ByteMap {
    std::unordered_map<uint32_t, uint8_t> char_to_byte;
    ByteMap() {
        int n = 0;
        for (int b = 0; b < 256; b++) {
            const bool keep = (b >= 33 && b <= 126) || (b >= 161 && b <= 172) || (b >= 174 && b <= 255);
            const uint32_t cp = keep ? (uint32_t)b : (uint32_t)(256 + n++);
            char_to_byte[cp] = (uint8_t)b;
        }
    }
};
const ByteMap& byte_map() {
    static ByteMap m;
    return m;
}

// ---------------------------------------------------------------- decoders
struct Decoder {
    std::string type;
    // Metaspace
    uint32_t replacement = 0x2581;
    bool prepend = true;
    // Strip
    uint32_t strip_ch = ' ';
    size_t strip_start = 0, strip_stop = 0;
    // Replace
    std::string pat, content;
    // WordPiece / BPEDecoder
    std::string prefix = "##", suffix = "</w>";
    bool cleanup = true;
    std::vector<Decoder> seq;
};

const JV* field(const JV& o, const char* k) { return o.get(k); }
std::string str_field(const JV& o, const char* k, const std::string& dflt) {
    const JV* v = o.get(k);
    return v && v->t == JV::STR ? v->s : dflt;
}
uint32_t first_char(const std::string& s, uint32_t dflt) {
    std::vector<uint32_t> c = chars_of(s);
    return c.empty() ? dflt : c[0];
}

Decoder parse_decoder(const JV& d) {
    Decoder o;
    if (d.t != JV::OBJ) throw TokError{"decoder must be an object"};
    o.type = str_field(d, "type", "");
    if (o.type == "Sequence") {
        const JV* ds = field(d, "decoders");
        if (!ds || ds->t != JV::ARR) throw TokError{"Sequence decoder without decoders"};
        for (auto& x : ds->a) o.seq.push_back(parse_decoder(x));
    } else if (o.type == "Metaspace") {
        o.replacement = first_char(str_field(d, "replacement", "\xE2\x96\x81"), 0x2581);
        const JV* ps = field(d, "prepend_scheme");
        if (ps && ps->t == JV::STR) o.prepend = ps->s != "never";
        else {
            const JV* aps = field(d, "add_prefix_space");
            o.prepend = !(aps && aps->t == JV::BOOL && !aps->b);
        }
    } else if (o.type == "Strip") {
        o.strip_ch = first_char(str_field(d, "content", " "), ' ');
        const JV* a = field(d, "start");
        const JV* b = field(d, "stop");
        o.strip_start = a && a->t == JV::POS ? (size_t)a->u : 0;
        o.strip_stop = b && b->t == JV::POS ? (size_t)b->u : 0;
    } else if (o.type == "Replace") {
        const JV* p = field(d, "pattern");
        const JV* s = p ? p->get("String") : nullptr;
        if (!s || s->t != JV::STR) throw TokError{"Replace decoder with a regex pattern is not supported"};
        o.pat = s->s;
        o.content = str_field(d, "content", "");
    } else if (o.type == "WordPiece") {
        o.prefix = str_field(d, "prefix", "##");
        const JV* c = field(d, "cleanup");
        o.cleanup = !(c && c->t == JV::BOOL && !c->b);
    } else if (o.type == "BPEDecoder") {
        o.suffix = str_field(d, "suffix", "</w>");
    } else if (o.type != "ByteLevel" && o.type != "ByteFallback" && o.type != "Fuse") {
        throw TokError{"decoder type \"" + o.type + "\" is not supported"};
    }
    return o;
}

std::string replace_all(const std::string& s, const std::string& a, const std::string& b) {
    if (a.empty()) return s;
    std::string o;
    size_t i = 0;
    for (;;) {
        size_t j = s.find(a, i);
        if (j == std::string::npos) { o.append(s, i, std::string::npos); return o; }
        o.append(s, i, j - i);
        o += b;
        i = j + a.size();
    }
}

std::string wordpiece_cleanup(std::string s) {
    static const char* const pairs[][2] = {{" .", "."}, {" ?", "?"}, {" !", "!"}, {" ,", ","}, {" ' ", "'"},
                                           {" n't", "n't"}, {" 'm", "'m"}, {" do not", " don't"}, {" 's", "'s"},
                                           {" 've", "'ve"}, {" 're", "'re"}};
    for (auto& p : pairs) s = replace_all(s, p[0], p[1]);
    return s;
}

// one decoder's decode_chain over the token strings
std::vector<std::string> decode_chain(const Decoder& d, std::vector<std::string> toks) {
    if (d.type == "Sequence") {
        for (auto& x : d.seq) toks = decode_chain(x, toks);
        return toks;
    }
    if (d.type == "ByteLevel") {
        const ByteMap& m = byte_map();
        std::string raw;
        for (auto& t : toks) {
            std::string b;
            bool ok = true;
            for (uint32_t c : chars_of(t)) {
                auto it = m.char_to_byte.find(c);
                if (it == m.char_to_byte.end()) { ok = false; break; }
                b += (char)it->second;
            }
            raw += ok ? b : t;
        }
        return {utf8_lossy(raw)};
    }
    if (d.type == "Metaspace") {
        std::vector<std::string> o;
        for (size_t i = 0; i < toks.size(); i++) {
            std::string s;
            for (uint32_t c : chars_of(toks[i])) {
                if (c == d.replacement) {
                    if (!(i == 0 && d.prepend)) s += ' ';
                } else {
                    put_utf8(s, c);
                }
            }
            o.push_back(s);
        }
        return o;
    }
    if (d.type == "ByteFallback") {
        std::vector<std::string> o;
        std::string pending;
        auto flush = [&]() {
            if (pending.empty()) return;
            if (utf8_lossy(pending) == pending) o.push_back(pending);
            else for (size_t k = 0; k < pending.size(); k++) o.push_back("\xEF\xBF\xBD");
            pending.clear();
        };
        for (auto& t : toks) {
            int byte = -1;
            if (t.size() == 6 && t.compare(0, 3, "<0x") == 0 && t[5] == '>') {
                // u8::from_str_radix(&t[3..5], 16): optional '+', then hex digits
                const char* p = t.c_str() + 3;
                int v = 0, nd = 0;
                int k = 0;
                if (p[0] == '+') k = 1;
                for (; k < 2; k++) {
                    const char c = p[k];
                    int x = (c >= '0' && c <= '9') ? c - '0' : (c >= 'a' && c <= 'f') ? c - 'a' + 10
                            : (c >= 'A' && c <= 'F') ? c - 'A' + 10 : -1;
                    if (x < 0) { nd = -1; break; }
                    v = v * 16 + x;
                    nd++;
                }
                if (nd > 0) byte = v;
            }
            if (byte >= 0) { pending += (char)byte; continue; }
            flush();
            o.push_back(t);
        }
        flush();
        return o;
    }
    if (d.type == "Fuse") {
        std::string s;
        for (auto& t : toks) s += t;
        return {s};
    }
    if (d.type == "Strip") {
        std::vector<std::string> o;
        for (auto& t : toks) {
            std::vector<uint32_t> c = chars_of(t);
            size_t a = 0, b = c.size();
            for (size_t i = 0; i < c.size() && i < d.strip_start; i++) {
                if (c[i] != d.strip_ch) break;
                a = i + 1;
            }
            for (size_t i = 0; i < c.size() && i < d.strip_stop; i++) {
                if (c[c.size() - 1 - i] != d.strip_ch) break;
                b = c.size() - 1 - i;
            }
            o.push_back(a < b ? from_chars(c, a, b) : std::string());
        }
        return o;
    }
    if (d.type == "Replace") {
        for (auto& t : toks) t = replace_all(t, d.pat, d.content);
        return toks;
    }
    if (d.type == "WordPiece") {
        for (size_t i = 0; i < toks.size(); i++) {
            std::string t = toks[i];
            if (i != 0) {
                if (t.compare(0, d.prefix.size(), d.prefix) == 0) t = t.substr(d.prefix.size());
                else t = " " + t;
            }
            if (d.cleanup) t = wordpiece_cleanup(t);
            toks[i] = t;
        }
        return toks;
    }
    if (d.type == "BPEDecoder") {
        for (size_t i = 0; i < toks.size(); i++)
            toks[i] = replace_all(toks[i], d.suffix, i + 1 == toks.size() ? "" : " ");
        return toks;
    }
    return toks;
}

// ---------------------------------------------------------------- vocabulary model
struct Vocab {
    std::unordered_map<uint32_t, std::string> model_id_to_tok;
    std::unordered_map<std::string, uint32_t> model_tok_to_id;
    std::unordered_map<uint32_t, std::string> added_id_to_tok;
    std::unordered_map<std::string, uint32_t> added_tok_to_id;
    std::unordered_set<std::string> special;
    bool has_decoder = false;
    Decoder dec;

    int64_t token_to_id(const std::string& t) const {
        auto a = added_tok_to_id.find(t);
        if (a != added_tok_to_id.end()) return a->second;
        auto m = model_tok_to_id.find(t);
        return m != model_tok_to_id.end() ? (int64_t)m->second : -1;
    }
    void add_token(const std::string& content, uint32_t id, bool is_special) {
        added_id_to_tok[id] = content;
        added_tok_to_id[content] = id;
        if (is_special) special.insert(content);
    }
    // decode([id], skip_special_tokens = true)
    bool decode(uint32_t id, std::string& out) const {
        const std::string* t = nullptr;
        auto a = added_id_to_tok.find(id);
        if (a != added_id_to_tok.end()) t = &a->second;
        else {
            auto m = model_id_to_tok.find(id);
            if (m != model_id_to_tok.end()) t = &m->second;
        }
        std::vector<std::string> toks;
        if (t && !special.count(*t)) toks.push_back(*t);
        if (has_decoder) toks = decode_chain(dec, toks);
        out.clear();
        for (size_t i = 0; i < toks.size(); i++) {
            if (!has_decoder && i) out += ' ';
            out += toks[i];
        }
        return true;
    }
    void table(zs_token_table& tt) const {
        // get_vocab_size(true): distinct token strings of the model and the added tokens
        size_t n = model_tok_to_id.size();
        for (auto& kv : added_tok_to_id)
            if (!model_tok_to_id.count(kv.first)) n++;
        tt.offsets.assign(1, 0);
        tt.text_offsets.assign(1, 0);
        tt.valid.assign(n, 0);
        std::string s;
        for (size_t id = 0; id < n; id++) {
            decode((uint32_t)id, s);
            tt.text.insert(tt.text.end(), s.begin(), s.end());
            tt.text_offsets.push_back((uint32_t)tt.text.size());
            if (!s.empty() && s.find("\xEF\xBF\xBD") == std::string::npos) {
                tt.valid[id] = 1;
                tt.bytes.insert(tt.bytes.end(), s.begin(), s.end());
            }
            tt.offsets.push_back((uint32_t)tt.bytes.size());
        }
        for (const char* e : {"</s>", "<|end_of_text|>", "<|eot_id|>"}) {
            int64_t id = token_to_id(e);
            if (id >= 0) { tt.eos = id; break; }
        }
    }
};

void vocab_from_tokenizer_json(const JV& root, Vocab& v) {
    const JV* model = root.get("model");
    if (!model || model->t != JV::OBJ) throw TokError{"tokenizer.json has no model"};
    const JV* voc = model->get("vocab");
    const std::string mtype = str_field(*model, "type", "");
    if (voc && voc->t == JV::OBJ) {
        for (auto& m : voc->o) {
            if (m.second.t != JV::POS || m.second.u > 0xffffffffull) throw TokError{"vocab id out of range"};
            v.model_tok_to_id[m.first] = (uint32_t)m.second.u;
            v.model_id_to_tok[(uint32_t)m.second.u] = m.first;
        }
    } else if (voc && voc->t == JV::ARR) {  // Unigram: [piece, score] by id
        for (size_t i = 0; i < voc->a.size(); i++) {
            const JV& e = voc->a[i];
            if (e.t != JV::ARR || e.a.empty() || e.a[0].t != JV::STR) throw TokError{"bad Unigram vocab entry"};
            v.model_tok_to_id[e.a[0].s] = (uint32_t)i;
            v.model_id_to_tok[(uint32_t)i] = e.a[0].s;
        }
    } else {
        throw TokError{"tokenizer.json model \"" + mtype + "\" has no vocab"};
    }
    if (const JV* added = root.get("added_tokens"); added && added->t == JV::ARR) {
        for (auto& t : added->a) {
            const JV* id = t.get("id");
            const JV* c = t.get("content");
            const JV* sp = t.get("special");
            if (!id || id->t != JV::POS || !c || c->t != JV::STR) throw TokError{"bad added_tokens entry"};
            v.add_token(c->s, (uint32_t)id->u, sp && sp->t == JV::BOOL && sp->b);
        }
    }
    const JV* dec = root.get("decoder");
    if (dec && dec->t == JV::OBJ) {
        v.dec = parse_decoder(*dec);
        v.has_decoder = true;
    }
}

// ---------------------------------------------------------------- GGUF metadata
class GgufReader {
public:
    explicit GgufReader(FILE* f) : f_(f) {}
    void read_exact(void* p, size_t n) {
        if (fread(p, 1, n, f_) != n) throw TokError{"invalid GGUF: truncated metadata"};
    }
    template <class T>
    T get() {
        T v;
        read_exact(&v, sizeof v);
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (n > (1ull << 30)) throw TokError{"invalid GGUF: string too long"};
        std::string s((size_t)n, '\0');
        if (n) read_exact(&s[0], (size_t)n);
        return s;
    }
    // skip (or keep) one value of type t
    void value(uint32_t t, std::vector<std::string>* strs, std::vector<int64_t>* ints, std::string* one,
               int64_t* one_int) {
        static const int width[13] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
        if (t == 8) {
            std::string s = str();
            if (one) *one = s;
            if (strs) strs->push_back(std::move(s));
            return;
        }
        if (t == 9) {
            const uint32_t et = get<uint32_t>();
            const uint64_t n = get<uint64_t>();
            if (n > (1ull << 28)) throw TokError{"invalid GGUF: array too long"};
            for (uint64_t i = 0; i < n; i++) value(et, strs, ints, nullptr, nullptr);
            return;
        }
        if (t > 12) throw TokError{"invalid GGUF: unknown value type"};
        uint8_t b[8] = {0};
        read_exact(b, (size_t)width[t]);
        int64_t v = 0;
        switch (t) {
            case 0: v = b[0]; break;
            case 1: v = (int8_t)b[0]; break;
            case 2: { uint16_t x; memcpy(&x, b, 2); v = x; break; }
            case 3: { int16_t x; memcpy(&x, b, 2); v = x; break; }
            case 4: { uint32_t x; memcpy(&x, b, 4); v = x; break; }
            case 5: { int32_t x; memcpy(&x, b, 4); v = x; break; }
            case 7: v = b[0] != 0; break;
            case 10: { uint64_t x; memcpy(&x, b, 8); v = (int64_t)x; break; }
            case 11: { int64_t x; memcpy(&x, b, 8); v = x; break; }
            default: break;  // floats are not needed
        }
        if (ints) ints->push_back(v);
        if (one_int) *one_int = v;
    }

private:
    FILE* f_;
};

void vocab_from_gguf(FILE* f, Vocab& v) {
    GgufReader r(f);
    char magic[4];
    r.read_exact(magic, 4);
    if (memcmp(magic, "GGUF", 4) != 0) throw TokError{"invalid GGUF: bad magic"};
    const uint32_t version = r.get<uint32_t>();
    if (version < 2) throw TokError{"invalid GGUF: unsupported version"};
    (void)r.get<uint64_t>();  // tensor count
    const uint64_t nkv = r.get<uint64_t>();
    std::string model_kind;
    std::vector<std::string> tokens;
    std::vector<int64_t> types;
    for (uint64_t i = 0; i < nkv; i++) {
        const std::string key = r.str();
        const uint32_t t = r.get<uint32_t>();
        if (key == "tokenizer.ggml.model") r.value(t, nullptr, nullptr, &model_kind, nullptr);
        else if (key == "tokenizer.ggml.tokens") r.value(t, &tokens, nullptr, nullptr, nullptr);
        else if (key == "tokenizer.ggml.token_type") r.value(t, nullptr, &types, nullptr, nullptr);
        else r.value(t, nullptr, nullptr, nullptr, nullptr);
    }
    if (model_kind != "gpt2")
        throw TokError{"GGUF-embedded vocab kind \"" + model_kind +
                       "\" is not supported (only byte-level BPE \"gpt2\"); place the model's tokenizer.json next to "
                       "the GGUF"};
    if (tokens.empty()) throw TokError{"GGUF missing tokenizer.ggml.tokens"};
    for (size_t i = 0; i < tokens.size(); i++) {
        v.model_tok_to_id[tokens[i]] = (uint32_t)i;  // a repeated token keeps its last id
    }
    for (auto& kv : v.model_tok_to_id) v.model_id_to_tok[kv.second] = kv.first;
    for (size_t i = 0; i < types.size() && i < tokens.size(); i++) {
        if (types[i] == 3 || types[i] == 4) {
            const int64_t id = v.token_to_id(tokens[i]);
            v.add_token(tokens[i], (uint32_t)(id >= 0 ? id : (int64_t)i), types[i] == 3);
        }
    }
    v.dec.type = "ByteLevel";
    v.has_decoder = true;
}

void put_err(char* err, size_t cap, const std::string& m) {
    if (!err || !cap) return;
    size_t n = m.size() < cap - 1 ? m.size() : cap - 1;
    memcpy(err, m.data(), n);
    err[n] = '\0';
}

template <class F>
int build_table(zs_token_table** out, char* err, size_t errcap, F&& fill) {
    if (!out) {
        put_err(err, errcap, "null argument");
        return ZS_EINVAL;
    }
    *out = nullptr;
    zs_token_table* t = new (std::nothrow) zs_token_table;
    if (!t) {
        put_err(err, errcap, "out of host memory");
        return ZS_ENOMEM;
    }
    try {
        Vocab v;
        fill(v);
        v.table(*t);
    } catch (const TokError& e) {
        delete t;
        put_err(err, errcap, e.msg);
        return ZS_EINVAL;
    } catch (const zsj::JsonError& e) {
        delete t;
        put_err(err, errcap, "failed to load tokenizer: " + e.msg);
        return ZS_EINVAL;
    } catch (const std::bad_alloc&) {
        delete t;
        put_err(err, errcap, "out of host memory");
        return ZS_ENOMEM;
    }
    *out = t;
    return ZS_OK;
}

}  // namespace

extern "C" int zs_token_table_from_json(const char* json, size_t len, zs_token_table** out, char* err,
                                        size_t errcap) {
    if (!json && len) {
        put_err(err, errcap, "null argument");
        return ZS_EINVAL;
    }
    return build_table(out, err, errcap, [&](Vocab& v) {
        const std::string text(json ? json : "", len);
        JV root = zsj::Reader(text).parse();
        vocab_from_tokenizer_json(root, v);
    });
}

extern "C" int zs_token_table_from_gguf(const char* path, zs_token_table** out, char* err, size_t errcap) {
    if (!path) {
        put_err(err, errcap, "null argument");
        return ZS_EINVAL;
    }
    return build_table(out, err, errcap, [&](Vocab& v) {
        FILE* f = fopen(path, "rb");
        if (!f) throw TokError{std::string("cannot open ") + path};
        try {
            vocab_from_gguf(f, v);
        } catch (...) {
            fclose(f);
            throw;
        }
        fclose(f);
    });
}

extern "C" int zs_token_table_info(const zs_token_table* t, uint32_t* ntab, uint32_t* nbytes, int64_t* eos) {
    if (!t) return ZS_EINVAL;
    if (ntab) *ntab = (uint32_t)t->valid.size();
    if (nbytes) *nbytes = (uint32_t)t->bytes.size();
    if (eos) *eos = t->eos;
    return ZS_OK;
}
extern "C" const uint32_t* zs_token_table_offsets(const zs_token_table* t) { return t ? t->offsets.data() : nullptr; }
extern "C" const uint8_t* zs_token_table_bytes(const zs_token_table* t) { return t ? t->bytes.data() : nullptr; }
extern "C" const uint8_t* zs_token_table_valid(const zs_token_table* t) { return t ? t->valid.data() : nullptr; }
extern "C" int zs_token_table_text(const zs_token_table* t, const uint32_t** offsets, const uint8_t** bytes) {
    if (!t || !offsets || !bytes) return ZS_EINVAL;
    *offsets = t->text_offsets.data();
    *bytes = t->text.data();
    return ZS_OK;
}
extern "C" void zs_token_table_destroy(zs_token_table* t) { delete t; }
