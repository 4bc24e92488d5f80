// zs_json.h -- a small strict JSON reader (RFC 8259) and the pieces of a
// serde_json-compatible writer for the host-side code (zs_schema.cpp,
// zs_tokens.cpp, zs_wire.cpp). Object members stay in document
// order; a repeated key replaces the value in its first position (serde_json
// with `preserve_order`, the reference's build, Cargo.toml:34). Numbers are
// classified as serde_json does: non-negative / negative integers that fit 64
// bits, everything else (fraction, exponent, overflow, "-0") as f64.
#pragma once
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <charconv>
#include <cmath>
#include <string>
#include <utility>
#include <vector>

namespace zsj {

struct JV {
    enum T { NUL, BOOL, POS, NEG, F64, STR, ARR, OBJ } t = NUL;
    bool b = false;
    uint64_t u = 0;
    int64_t i = 0;
    double d = 0.0;
    std::string s;
    std::vector<JV> a;
    std::vector<std::pair<std::string, JV>> o;
    const JV* get(const char* k) const {
        if (t != OBJ) return nullptr;
        for (auto& m : o)
            if (m.first == k) return &m.second;
        return nullptr;
    }
};

struct JsonError {
    std::string msg;
};

class Reader {
public:
    explicit Reader(const std::string& s) : s_(s) {}
    JV parse() {
        JV v = value(0);
        ws();
        if (p_ < s_.size()) fail("trailing characters");
        return v;
    }

private:
    const std::string& s_;
    size_t p_ = 0;

    [[noreturn]] void fail(const std::string& m) {
        // line / column like serde_json's messages
        size_t line = 1, col = 0;
        for (size_t i = 0; i < p_ && i < s_.size(); i++) {
            if (s_[i] == '\n') { line++; col = 0; } else col++;
        }
        throw JsonError{m + " at line " + std::to_string(line) + " column " + std::to_string(col + 1)};
    }
    void ws() {
        while (p_ < s_.size() && (s_[p_] == ' ' || s_[p_] == '\t' || s_[p_] == '\n' || s_[p_] == '\r')) p_++;
    }
    void lit(const char* w) {
        size_t n = strlen(w);
        if (s_.compare(p_, n, w) != 0) fail("expected value");
        p_ += n;
    }
    JV value(int depth) {
        ws();
        if (p_ >= s_.size()) fail("EOF while parsing a value");
        JV v;
        const char c = s_[p_];
        if (c == 'n') { lit("null"); return v; }
        if (c == 't') { lit("true"); v.t = JV::BOOL; v.b = true; return v; }
        if (c == 'f') { lit("false"); v.t = JV::BOOL; return v; }
        if (c == '"') { v.t = JV::STR; v.s = str(); return v; }
        if (c == '-' || (c >= '0' && c <= '9')) return number();
        if (c == '[' || c == '{') {
            if (depth >= 128) fail("recursion limit exceeded");
            p_++;
            const char close = c == '[' ? ']' : '}';
            v.t = c == '[' ? JV::ARR : JV::OBJ;
            ws();
            if (p_ < s_.size() && s_[p_] == close) { p_++; return v; }
            for (;;) {
                if (v.t == JV::ARR) {
                    v.a.push_back(value(depth + 1));
                } else {
                    ws();
                    if (p_ >= s_.size() || s_[p_] != '"') fail("key must be a string");
                    std::string k = str();
                    ws();
                    if (p_ >= s_.size() || s_[p_] != ':') fail("expected `:`");
                    p_++;
                    JV m = value(depth + 1);
                    bool found = false;
                    for (auto& e : v.o)
                        if (e.first == k) { e.second = std::move(m); found = true; break; }
                    if (!found) v.o.emplace_back(std::move(k), std::move(m));
                }
                ws();
                if (p_ >= s_.size()) fail("EOF while parsing");
                if (s_[p_] == ',') { p_++; continue; }
                if (s_[p_] == close) { p_++; return v; }
                fail(v.t == JV::ARR ? "expected `,` or `]`" : "expected `,` or `}`");
            }
        }
        fail("expected value");
    }
    uint32_t hex4() {
        if (p_ + 4 > s_.size()) fail("EOF while parsing a string");
        uint32_t v = 0;
        for (int i = 0; i < 4; i++) {
            const char c = s_[p_++];
            int d = (c >= '0' && c <= '9') ? c - '0' : (c >= 'a' && c <= 'f') ? c - 'a' + 10
                    : (c >= 'A' && c <= 'F') ? c - 'A' + 10 : -1;
            if (d < 0) fail("invalid escape");
            v = v * 16 + (uint32_t)d;
        }
        return v;
    }
    static void put_utf8(std::string& o, uint32_t cp) {
        if (cp < 0x80) o += (char)cp;
        else if (cp < 0x800) { o += (char)(0xC0 | (cp >> 6)); o += (char)(0x80 | (cp & 0x3f)); }
        else if (cp < 0x10000) {
            o += (char)(0xE0 | (cp >> 12)); o += (char)(0x80 | ((cp >> 6) & 0x3f)); o += (char)(0x80 | (cp & 0x3f));
        } else {
            o += (char)(0xF0 | (cp >> 18)); o += (char)(0x80 | ((cp >> 12) & 0x3f));
            o += (char)(0x80 | ((cp >> 6) & 0x3f)); o += (char)(0x80 | (cp & 0x3f));
        }
    }
    std::string str() {
        p_++;  // opening quote
        std::string o;
        for (;;) {
            if (p_ >= s_.size()) fail("EOF while parsing a string");
            const unsigned char c = (unsigned char)s_[p_];
            if (c == '"') { p_++; return o; }
            if (c < 0x20) fail("control character (\\u0000-\\u001F) found while parsing a string");
            if (c != '\\') { o += (char)c; p_++; continue; }
            p_++;
            if (p_ >= s_.size()) fail("EOF while parsing a string");
            const char e = s_[p_++];
            switch (e) {
                case '"': o += '"'; break;
                case '\\': o += '\\'; break;
                case '/': o += '/'; break;
                case 'b': o += '\b'; break;
                case 'f': o += '\f'; break;
                case 'n': o += '\n'; break;
                case 'r': o += '\r'; break;
                case 't': o += '\t'; break;
                case 'u': {
                    uint32_t cp = hex4();
                    if (cp >= 0xDC00 && cp <= 0xDFFF) fail("lone leading surrogate in hex escape");
                    if (cp >= 0xD800 && cp <= 0xDBFF) {
                        if (p_ + 2 > s_.size() || s_[p_] != '\\' || s_[p_ + 1] != 'u')
                            fail("unexpected end of hex escape");
                        p_ += 2;
                        const uint32_t lo = hex4();
                        if (lo < 0xDC00 || lo > 0xDFFF) fail("lone leading surrogate in hex escape");
                        cp = 0x10000 + ((cp - 0xD800) << 10) + (lo - 0xDC00);
                    }
                    put_utf8(o, cp);
                    break;
                }
                default: fail("invalid escape");
            }
        }
    }
    JV number() {
        const size_t st = p_;
        const bool neg = s_[p_] == '-';
        if (neg) p_++;
        if (p_ >= s_.size() || !(s_[p_] >= '0' && s_[p_] <= '9')) fail("invalid number");
        if (s_[p_] == '0' && p_ + 1 < s_.size() && s_[p_ + 1] >= '0' && s_[p_ + 1] <= '9') fail("invalid number");
        while (p_ < s_.size() && s_[p_] >= '0' && s_[p_] <= '9') p_++;
        const size_t int_end = p_;
        bool is_float = false;
        if (p_ < s_.size() && s_[p_] == '.') {
            is_float = true;
            p_++;
            if (p_ >= s_.size() || !(s_[p_] >= '0' && s_[p_] <= '9')) fail("invalid number");
            while (p_ < s_.size() && s_[p_] >= '0' && s_[p_] <= '9') p_++;
        }
        if (p_ < s_.size() && (s_[p_] == 'e' || s_[p_] == 'E')) {
            is_float = true;
            p_++;
            if (p_ < s_.size() && (s_[p_] == '+' || s_[p_] == '-')) p_++;
            if (p_ >= s_.size() || !(s_[p_] >= '0' && s_[p_] <= '9')) fail("invalid number");
            while (p_ < s_.size() && s_[p_] >= '0' && s_[p_] <= '9') p_++;
        }
        JV v;
        if (!is_float) {
            // integer: fits 64 bits as serde_json keeps it?
            unsigned __int128 m = 0;
            bool big = false;
            for (size_t i = st + (neg ? 1 : 0); i < int_end; i++) {
                m = m * 10 + (unsigned)(s_[i] - '0');
                if (m > ((unsigned __int128)1 << 64)) { big = true; break; }
            }
            if (!big && !neg && m <= UINT64_MAX) { v.t = JV::POS; v.u = (uint64_t)m; return v; }
            if (!big && neg && m != 0 && m <= ((unsigned __int128)1 << 63)) {
                v.t = JV::NEG;
                v.i = (int64_t)(0 - (uint64_t)m);
                return v;
            }
        }
        const std::string txt = s_.substr(st, p_ - st);
        v.t = JV::F64;
        v.d = strtod(txt.c_str(), nullptr);
        if (std::isinf(v.d)) fail("number out of range");
        return v;
    }
};

// ---------------------------------------------------------------- writer
// ryu's layout of the shortest round-trip digits (serde_json's f64 output)
inline std::string f64_text(double d) {
    if (d == 0.0) return std::signbit(d) ? "-0.0" : "0.0";
    std::string out;
    if (d < 0) { out += '-'; d = -d; }
    char buf[64];
    auto r = std::to_chars(buf, buf + sizeof buf, d, std::chars_format::scientific);
    std::string sci(buf, r.ptr);
    const size_t e = sci.find('e');
    std::string digits;
    for (size_t i = 0; i < e; i++)
        if (sci[i] != '.') digits += sci[i];
    const int sexp = atoi(sci.c_str() + e + 1);
    const int length = (int)digits.size();
    const int kk = sexp + 1;          // 10^(kk-1) <= v < 10^kk
    const int k = kk - length;        // exponent of the last digit
    if (k >= 0 && kk <= 16) {
        out += digits;
        out.append((size_t)(kk - length), '0');
        out += ".0";
    } else if (kk > 0 && kk <= 16) {
        out += digits.substr(0, (size_t)kk);
        out += '.';
        out += digits.substr((size_t)kk);
    } else if (kk > -5 && kk <= 0) {
        out += "0.";
        out.append((size_t)(-kk), '0');
        out += digits;
    } else if (length == 1) {
        out += digits;
        out += 'e';
        out += std::to_string(kk - 1);
    } else {
        out += digits[0];
        out += '.';
        out += digits.substr(1);
        out += 'e';
        out += std::to_string(kk - 1);
    }
    return out;
}

inline void write_str(std::string& o, const std::string& s) {
    static const char hex[] = "0123456789abcdef";
    o += '"';
    for (unsigned char c : s) {
        switch (c) {
            case '"': o += "\\\""; break;
            case '\\': o += "\\\\"; break;
            case '\b': o += "\\b"; break;
            case '\f': o += "\\f"; break;
            case '\n': o += "\\n"; break;
            case '\r': o += "\\r"; break;
            case '\t': o += "\\t"; break;
            default:
                if (c < 0x20) { o += "\\u00"; o += hex[c >> 4]; o += hex[c & 15]; }
                else o += (char)c;
        }
    }
    o += '"';
}

}  // namespace zsj
