// zs_regex.cpp -- regex -> anchored byte DFA on the host.
//
// Replaces the dense DFA that logit_fsm.rs:62-88 builds with regex-automata
// (anchored start, MatchKind::All, minimised, 24 MB size limit). Only the
// language matters to the masks: a token is allowed iff its bytes keep the
// text a prefix of some full match (logit_fsm.rs:166-182 with is_live
// :121-161), and EOS needs the text itself to be a full match (:110-112), so
// any DFA of the same language gives the same masks. The DFA here recognises
// "the whole text matches the pattern": Thompson NFA over UTF-8 bytes, subset
// construction over byte equivalence classes, Moore minimisation (which also
// folds every state that cannot reach a match into the dead state 0).
//
// Syntax (the regex-syntax subset that patterns reach here): literals (UTF-8),
// escapes of punctuation, \t \n \r \f \v \a, \xHH \x{H..} \uHHHH \u{H..}
// \UHHHHHHHH, classes [..] with ranges, negation, nested classes, ASCII
// POSIX names and the set operations && -- ~~ (equal precedence, left to
// right, binding looser than union), '.', groups ( ), (?: ), (?P<n> ),
// (?<n> ), flags (?imsxuUR-imsxuUR) and (?flags: ), alternation, * + ? {n}
// {n,} {n,m} with lazy forms (same language), the anchors ^ $ \A \z, with
// (?m) the line anchors ^ $ (after / before '\n'; with (?mR) '\r' and '\n'
// both end lines and ^ $ never match between "\r\n"), and the ASCII word
// boundaries \b \B \< \> \b{start} \b{end} \b{start-half} \b{end-half}
// under (?-u). Unicode mode, as regex-syntax's default: \d is \p{Nd}, \s is
// White_Space, \w is [\p{Alphabetic}\p{M}\p{Nd}\p{Pc}\p{Join_Control}]
// (UTS #18 Annex C), \p{..} / \P{..} take general categories (short or long
// names, one-letter groups, gc= forms) and Any / ASCII / Assigned, and
// case-insensitive mode uses simple case folding. The tables (zs_unicode.h)
// are generated from Python's unicodedata (Unicode 13.0 in this image;
// regex-syntax 0.8.10 has 16.0: scalars assigned after 13.0 are outside \w
// \d \p{..} here). (?-u) makes \d \s \w ASCII and case folding ASCII-only,
// and, as regex-syntax does with UTF-8 mode on, refuses what could match
// bytes that are not UTF-8 ('.', negated byte classes, \x80-\xFF) and
// non-ASCII class members. Errors as in regex-automata's dense DFA builder:
// Unicode word boundaries (\b and friends without (?-u)). Refused with an
// error although regex-syntax accepts them: script and binary properties
// other than the above (\p{Greek}).
//
// Look-around (anchors, line anchors, word boundaries) is resolved during
// subset construction: a DFA state is a set of NFA states plus the class of
// the byte before the position (start of text, ASCII word byte, '\n', '\r',
// other). Assertions in a set stay pending until the next byte, or the end of
// the text, is known; then each holds or fails from (previous, next).
#include <stdint.h>
#include <string.h>
#include <algorithm>
#include <initializer_list>
#include <string>
#include <unordered_map>
#include <vector>
#include "zs_grammar.h"
#include "zs_unicode.h"

namespace {

const uint32_t CP_MAX = 0x10FFFF;
const uint32_t INF = 0xffffffffu;

// ------------------------------------------------------------ codepoint sets
struct CpSet {
    std::vector<std::pair<uint32_t, uint32_t>> r;  // inclusive ranges
    void add(uint32_t lo, uint32_t hi) { r.push_back({lo, hi}); }
    void add(const CpSet& o) { r.insert(r.end(), o.r.begin(), o.r.end()); }
    void canon() {
        std::sort(r.begin(), r.end());
        std::vector<std::pair<uint32_t, uint32_t>> o;
        for (auto& x : r) {
            if (!o.empty() && x.first <= o.back().second + 1) o.back().second = std::max(o.back().second, x.second);
            else o.push_back(x);
        }
        r.swap(o);
    }
    // complement over the Unicode scalar values
    void negate() {
        canon();
        std::vector<std::pair<uint32_t, uint32_t>> o;
        uint32_t next = 0;
        for (auto& x : r) {
            if (x.first > next) o.push_back({next, x.first - 1});
            next = x.second + 1;
        }
        if (next <= CP_MAX) o.push_back({next, CP_MAX});
        r.swap(o);
        remove_surrogates();
    }
    void remove_surrogates() {
        std::vector<std::pair<uint32_t, uint32_t>> o;
        for (auto& x : r) {
            if (x.second < 0xD800 || x.first > 0xDFFF) { o.push_back(x); continue; }
            if (x.first < 0xD800) o.push_back({x.first, 0xD7FF});
            if (x.second > 0xDFFF) o.push_back({0xE000, x.second});
        }
        r.swap(o);
    }
    bool contains(uint32_t c) const {   // canonical ranges
        size_t lo = 0, hi = r.size();
        while (lo < hi) {
            const size_t mid = (lo + hi) / 2;
            if (r[mid].second < c) lo = mid + 1;
            else hi = mid;
        }
        return lo < r.size() && r[lo].first <= c;
    }
    // simple case folding (case-insensitive flag): adds every scalar that
    // folds like a member (classes are cycles in zs_uc_fold)
    void fold() {
        canon();
        for (;;) {
            std::vector<std::pair<uint32_t, uint32_t>> extra;
            for (const auto& e : zs_uc_fold)
                if (contains(e[0]) && !contains(e[1])) extra.push_back({e[1], e[1]});
            if (extra.empty()) return;
            r.insert(r.end(), extra.begin(), extra.end());
            canon();
        }
    }
    // ASCII-only case folding (regex-syntax's byte classes)
    void fold_ascii() {
        canon();
        std::vector<std::pair<uint32_t, uint32_t>> extra;
        for (auto& x : r) {
            const uint32_t lo = x.first, hi = std::min(x.second, 0x7Fu);
            if (lo > hi) continue;
            const uint32_t a = std::max(lo, (uint32_t)'a'), b = std::min(hi, (uint32_t)'z');
            if (a <= b) extra.push_back({a - 32, b - 32});
            const uint32_t A = std::max(lo, (uint32_t)'A'), B = std::min(hi, (uint32_t)'Z');
            if (A <= B) extra.push_back({A + 32, B + 32});
        }
        r.insert(r.end(), extra.begin(), extra.end());
        canon();
    }
    bool is_ascii() const {
        for (auto& x : r) if (x.second > 0x7F) return false;
        return true;
    }
    // set operations of classes (canonical operands)
    static CpSet meet(const CpSet& a, const CpSet& b) {
        CpSet o;
        size_t i = 0, j = 0;
        while (i < a.r.size() && j < b.r.size()) {
            const uint32_t lo = std::max(a.r[i].first, b.r[j].first), hi = std::min(a.r[i].second, b.r[j].second);
            if (lo <= hi) o.add(lo, hi);
            if (a.r[i].second < b.r[j].second) i++;
            else j++;
        }
        return o;
    }
    static CpSet minus(const CpSet& a, const CpSet& b) {
        CpSet nb = b;
        nb.negate();
        return meet(a, nb);
    }
    static CpSet symdiff(const CpSet& a, const CpSet& b) {
        CpSet o = minus(a, b);
        o.add(minus(b, a));
        o.canon();
        return o;
    }
};

// ------------------------------------------------------------ syntax tree
enum Kind { K_EMPTY, K_CLASS, K_CAT, K_ALT, K_REP, K_LOOK };

// zero-width assertions (K_LOOK's mn, N_LOOK's lo)
enum Look : uint8_t {
    L_TEXT_START, L_TEXT_END, L_LF_START, L_LF_END, L_CRLF_START, L_CRLF_END,
    L_WORD, L_NOT_WORD, L_WORD_START, L_WORD_END, L_WORD_START_HALF, L_WORD_END_HALF
};
struct Node {
    Kind k;
    CpSet set;
    std::vector<int> kids;
    uint32_t mn = 0, mx = 0;
};

struct Flags {
    bool i = false, s = false, x = false, m = false, u = true, R = false;
};

struct ParseError {
    std::string msg;
};

class Parser {
public:
    Parser(const std::string& p, std::vector<Node>& ar) : p_(p), ar_(ar) {}
    int parse() {
        Flags f;
        int n = parse_alt(f, 0);
        if (pos_ < p_.size()) {
            if (p_[pos_] == ')') fail("unopened group");
            fail("unexpected character");
        }
        return n;
    }

private:
    const std::string& p_;
    std::vector<Node>& ar_;
    size_t pos_ = 0;

    [[noreturn]] void fail(const std::string& m) {
        throw ParseError{m + " at offset " + std::to_string(pos_)};
    }
    bool eof() const { return pos_ >= p_.size(); }
    char peek() const { return p_[pos_]; }
    int node(Kind k) {
        ar_.push_back(Node{});
        ar_.back().k = k;
        return (int)ar_.size() - 1;
    }
    // one UTF-8 encoded scalar of the pattern
    uint32_t next_cp() {
        const unsigned char c = (unsigned char)p_[pos_];
        int n = c < 0x80 ? 1 : (c >> 5) == 6 ? 2 : (c >> 4) == 14 ? 3 : (c >> 3) == 30 ? 4 : 0;
        if (!n || pos_ + n > p_.size()) fail("invalid UTF-8 in pattern");
        uint32_t cp = n == 1 ? c : n == 2 ? (c & 0x1f) : n == 3 ? (c & 0x0f) : (c & 0x07);
        for (int i = 1; i < n; i++) {
            const unsigned char d = (unsigned char)p_[pos_ + i];
            if ((d >> 6) != 2) fail("invalid UTF-8 in pattern");
            cp = (cp << 6) | (d & 0x3f);
        }
        pos_ += n;
        return cp;
    }
    void skip_verbose(const Flags& f) {
        if (!f.x) return;
        while (!eof()) {
            char c = peek();
            if (c == ' ' || c == '\t' || c == '\n' || c == '\r' || c == '\f' || c == '\v') { pos_++; continue; }
            if (c == '#') {
                while (!eof() && peek() != '\n') pos_++;
                continue;
            }
            break;
        }
    }

    int parse_alt(Flags& f, int depth) {
        if (depth > 250) fail("exceeds the nesting limit");
        std::vector<int> br;
        br.push_back(parse_concat(f, depth));
        while (!eof() && peek() == '|') {
            pos_++;
            br.push_back(parse_concat(f, depth));
        }
        if (br.size() == 1) return br[0];
        int n = node(K_ALT);
        ar_[n].kids = br;
        return n;
    }

    int parse_concat(Flags& f, int depth) {
        std::vector<int> items;
        for (;;) {
            skip_verbose(f);
            if (eof() || peek() == '|' || peek() == ')') break;
            const char c = peek();
            if (c == '*' || c == '+' || c == '?' || c == '{') {
                if (items.empty()) fail("repetition operator missing expression");
                items.back() = parse_rep(items.back(), f);
                continue;
            }
            int a = parse_atom(f, depth);
            if (a >= 0) items.push_back(a);
        }
        if (items.empty()) return node(K_EMPTY);
        if (items.size() == 1) return items[0];
        int n = node(K_CAT);
        ar_[n].kids = items;
        return n;
    }

    bool parse_dec(uint32_t* v) {
        size_t st = pos_;
        uint64_t x = 0;
        while (!eof() && peek() >= '0' && peek() <= '9') {
            x = x * 10 + (uint64_t)(peek() - '0');
            if (x > 100000) fail("repetition count too large");
            pos_++;
        }
        *v = (uint32_t)x;
        return pos_ > st;
    }

    int parse_rep(int atom, const Flags& f) {
        uint32_t mn, mx;
        const char c = peek();
        pos_++;
        if (c == '*') { mn = 0; mx = INF; }
        else if (c == '+') { mn = 1; mx = INF; }
        else if (c == '?') { mn = 0; mx = 1; }
        else {
            skip_verbose(f);
            if (!parse_dec(&mn)) fail("repetition quantifier expects a valid decimal");
            skip_verbose(f);
            mx = mn;
            if (!eof() && peek() == ',') {
                pos_++;
                skip_verbose(f);
                if (!parse_dec(&mx)) mx = INF;
                skip_verbose(f);
            }
            if (eof() || peek() != '}') fail("unclosed counted repetition");
            pos_++;
            if (mx != INF && mx < mn) fail("invalid repetition count range");
        }
        if (!eof() && peek() == '?') pos_++;  // lazy: same language
        int n = node(K_REP);
        ar_[n].kids = {atom};
        ar_[n].mn = mn;
        ar_[n].mx = mx;
        return n;
    }

    int class_node(CpSet s, const Flags& f) {
        if (f.i) {
            if (f.u) s.fold();
            else s.fold_ascii();
        }
        s.remove_surrogates();
        s.canon();
        int n = node(K_CLASS);
        ar_[n].set = s;
        return n;
    }

    // flags like "i-sx"; returns true when the group continues with ':'
    void parse_flags(Flags& f) {
        bool neg = false;
        for (;;) {
            if (eof()) fail("unclosed group");
            char c = peek();
            if (c == ')' || c == ':') return;
            pos_++;
            switch (c) {
                case '-': neg = true; break;
                case 'i': f.i = !neg; break;
                case 's': f.s = !neg; break;
                case 'x': f.x = !neg; break;
                case 'm': f.m = !neg; break;
                case 'U': break;  // swaps greediness: same language
                case 'u': f.u = !neg; break;
                case 'R': f.R = !neg; break;
                default: fail("unrecognized flag");
            }
        }
    }

    int parse_atom(Flags& f, int depth) {
        const char c = peek();
        if (c == '(') {
            pos_++;
            Flags inner = f;
            if (!eof() && peek() == '?') {
                pos_++;
                if (eof()) fail("unclosed group");
                if (peek() == ':') {
                    pos_++;
                } else if (peek() == 'P' || peek() == '<') {
                    if (peek() == 'P') pos_++;
                    if (eof() || peek() != '<') fail("invalid capture group name");
                    pos_++;
                    size_t st = pos_;
                    while (!eof() && peek() != '>') pos_++;
                    if (eof() || pos_ == st) fail("invalid capture group name");
                    pos_++;
                } else {
                    parse_flags(inner);
                    if (peek() == ')') {  // (?flags): applies to the rest of the group
                        pos_++;
                        f = inner;
                        return -1;
                    }
                    pos_++;  // ':'
                }
            }
            int n = parse_alt(inner, depth + 1);
            if (eof() || peek() != ')') fail("unclosed group");
            pos_++;
            return n;
        }
        if (c == ')') fail("unopened group");
        if (c == '[') return class_node(parse_class(f), Flags{});  // folded inside
        if (c == '.') {
            if (!f.u) fail("pattern can match invalid UTF-8");
            pos_++;
            CpSet s;
            if (f.s) s.add(0, CP_MAX);
            else { s.add(0, 9); s.add(11, CP_MAX); }
            return class_node(s, Flags{});
        }
        if (c == '^' || c == '$') {
            pos_++;
            const bool st = c == '^';
            if (!f.m) return look(st ? L_TEXT_START : L_TEXT_END);
            if (f.R) return look(st ? L_CRLF_START : L_CRLF_END);
            return look(st ? L_LF_START : L_LF_END);
        }
        if (c == '\\') {
            pos_++;
            if (eof()) fail("incomplete escape sequence");
            const char e = peek();
            if (e == 'A' || e == 'z') {
                pos_++;
                return look(e == 'A' ? L_TEXT_START : L_TEXT_END);
            }
            if (e == 'b' || e == 'B' || e == '<' || e == '>') return word_boundary(f);
            CpSet s;
            if (perl_class(s, f.u)) return class_node(s, f);
            const uint32_t cp = escape_cp(f.u);
            s.add(cp, cp);
            return class_node(s, f);
        }
        CpSet s;
        uint32_t cp = next_cp();
        s.add(cp, cp);
        return class_node(s, f);
    }

    int look(Look l) {
        const int n = node(K_LOOK);
        ar_[n].mn = l;
        return n;
    }

    // \b \B \< \> \b{start} \b{end} \b{start-half} \b{end-half}; pos_ at
    // the letter. "\b{" followed by a non-letter is \b and a repetition.
    int word_boundary(const Flags& f) {
        const char e = peek();
        pos_++;
        Look l = e == 'B' ? L_NOT_WORD : e == '<' ? L_WORD_START : e == '>' ? L_WORD_END : L_WORD;
        auto name_char = [](char c) { return (c >= 'a' && c <= 'z') || (c >= 'A' && c <= 'Z') || c == '-'; };
        if (e == 'b' && pos_ + 1 < p_.size() && p_[pos_] == '{' && name_char(p_[pos_ + 1])) {
            size_t q = pos_ + 1;
            while (q < p_.size() && name_char(p_[q])) q++;
            if (q >= p_.size() || p_[q] != '}') fail("unclosed special word boundary");
            const std::string name = p_.substr(pos_ + 1, q - pos_ - 1);
            if (name == "start") l = L_WORD_START;
            else if (name == "end") l = L_WORD_END;
            else if (name == "start-half") l = L_WORD_START_HALF;
            else if (name == "end-half") l = L_WORD_END_HALF;
            else fail("unrecognized special word boundary");
            pos_ = q + 1;
        }
        if (f.u)
            fail("Unicode word boundaries cannot be built into a DFA (use an ASCII one, such as (?-u:\\b))");
        return look(l);
    }

    uint32_t hex_digits(int n_fixed) {
        uint32_t v = 0;
        int n = 0;
        bool braced = !eof() && peek() == '{';
        if (braced) pos_++;
        while (!eof()) {
            char c = peek();
            int d = (c >= '0' && c <= '9') ? c - '0' : (c >= 'a' && c <= 'f') ? c - 'a' + 10
                    : (c >= 'A' && c <= 'F') ? c - 'A' + 10 : -1;
            if (d < 0) break;
            v = v * 16 + (uint32_t)d;
            if (v > CP_MAX) fail("invalid Unicode scalar value");
            pos_++;
            n++;
            if (!braced && n == n_fixed) break;
        }
        if (braced) {
            if (eof() || peek() != '}' || n == 0) fail("invalid hexadecimal escape");
            pos_++;
        } else if (n != n_fixed) {
            fail("invalid hexadecimal escape");
        }
        if (v >= 0xD800 && v <= 0xDFFF) fail("invalid Unicode scalar value");
        return v;
    }

    // the scalar denoted by an escape (pos_ at the character after '\')
    // (byte mode: \xHH above 0x7F is a byte, which regex-syntax refuses in
    // UTF-8 mode; \x{..}, \u and \U always denote scalars)
    uint32_t escape_cp(bool u) {
        const char e = peek();
        pos_++;
        if (e == 'x' && !u && (eof() || peek() != '{')) {
            const uint32_t v = hex_digits(2);
            if (v > 0x7F) fail("pattern can match invalid UTF-8");
            return v;
        }
        switch (e) {
            case 'n': return '\n';
            case 't': return '\t';
            case 'r': return '\r';
            case 'f': return 0x0C;
            case 'v': return 0x0B;
            case 'a': return 0x07;
            case 'x': return hex_digits(2);
            case 'u': return hex_digits(4);
            case 'U': return hex_digits(8);
            default: break;
        }
        const unsigned char ue = (unsigned char)e;
        if (ue < 0x80 && !((e >= '0' && e <= '9') || (e >= 'a' && e <= 'z') || (e >= 'A' && e <= 'Z')))
            return ue;  // escaped punctuation or space
        pos_--;
        if (e == 'b' || e == 'B' || e == '<' || e == '>') fail("word boundary assertions are not allowed in classes");
        if (e >= '0' && e <= '9') fail("backreferences are not supported");
        fail("unrecognized escape sequence");
    }

    // the scalars of general categories (bit k of mask: zs_uc_cat_names[k])
    static void add_cats(CpSet& s, uint32_t mask) {
        for (const auto& g : zs_uc_cats)
            if ((mask >> g.cat) & 1u) s.add(g.lo, g.hi);
    }
    static uint32_t cat_bit(const char* n) {
        for (int k = 0; k < ZS_UC_NCATS; k++)
            if (!strcmp(zs_uc_cat_names[k], n)) return 1u << k;
        return 0;
    }
    static uint32_t cats(std::initializer_list<const char*> ns) {
        uint32_t m = 0;
        for (const char* n : ns) m |= cat_bit(n);
        return m;
    }
    // PropList.txt White_Space
    static void add_white_space(CpSet& s) {
        s.add(0x09, 0x0D); s.add(0x20, 0x20); s.add(0x85, 0x85); s.add(0xA0, 0xA0); s.add(0x1680, 0x1680);
        s.add(0x2000, 0x200A); s.add(0x2028, 0x2029); s.add(0x202F, 0x202F); s.add(0x205F, 0x205F);
        s.add(0x3000, 0x3000);
    }
    // \w: Alphabetic (letters, Nl and Other_Alphabetic), marks, Nd, Pc and
    // Join_Control; the Other_Alphabetic scalars outside the marks are the
    // circled and squared Latin letters (category So)
    static void add_word(CpSet& s) {
        add_cats(s, cats({"Lu", "Ll", "Lt", "Lm", "Lo", "Nl", "Mn", "Mc", "Me", "Nd", "Pc"}));
        s.add(0x200C, 0x200D);
        s.add(0x24B6, 0x24E9);
        s.add(0x1F130, 0x1F149);
        s.add(0x1F150, 0x1F169);
        s.add(0x1F170, 0x1F189);
    }

    // \d \D \s \S \w \W \p{..} \P{..}; pos_ at the letter. Byte mode
    // (u false): ASCII \d \s \w, whose negations match bytes above 0x7F
    // and are refused; \p is refused.
    bool perl_class(CpSet& s, bool u) {
        const char e = peek();
        CpSet b;
        if (!u && (e == 'd' || e == 'D' || e == 's' || e == 'S' || e == 'w' || e == 'W')) {
            if (e == 'D' || e == 'S' || e == 'W') fail("pattern can match invalid UTF-8");
            if (e == 'd') b.add('0', '9');
            else if (e == 's') { b.add('\t', '\r'); b.add(' ', ' '); }
            else { b.add('0', '9'); b.add('A', 'Z'); b.add('_', '_'); b.add('a', 'z'); }
            pos_++;
            s.add(b);
            return true;
        }
        if (e == 'd' || e == 'D') add_cats(b, cats({"Nd"}));
        else if (e == 's' || e == 'S') add_white_space(b);
        else if (e == 'w' || e == 'W') add_word(b);
        else if (e == 'p' || e == 'P') {
            if (!u) fail("Unicode classes are not allowed when Unicode mode is disabled");
            pos_++;
            std::string name;
            if (!eof() && peek() == '{') {
                const size_t end = p_.find('}', pos_);
                if (end == std::string::npos) fail("unclosed Unicode class");
                name = p_.substr(pos_ + 1, end - pos_ - 1);
                pos_ = end + 1;
            } else {
                if (eof()) fail("incomplete escape sequence");
                name = std::string(1, peek());
                pos_++;
            }
            unicode_class(name, b);
            if (e == 'P') b.negate();
            s.add(b);
            return true;
        } else {
            return false;
        }
        pos_++;
        if (e == 'D' || e == 'S' || e == 'W') b.negate();
        s.add(b);
        return true;
    }

    // \p{name}: general categories, Any, ASCII, Assigned (UAX #44 loose
    // matching: case, spaces, '_' and '-' ignored; "gc=" prefixes allowed)
    void unicode_class(const std::string& raw, CpSet& b) {
        std::string n;
        bool neg = false;
        for (char c : raw) {
            if (c == ' ' || c == '_' || c == '-') continue;
            n += (char)((c >= 'A' && c <= 'Z') ? c - 'A' + 'a' : c);
        }
        if (!n.empty() && n[0] == '^') { neg = true; n = n.substr(1); }
        for (const char* pre : {"generalcategory=", "generalcategory:", "gc=", "gc:"}) {
            const size_t L = strlen(pre);
            if (n.compare(0, L, pre) == 0) { n = n.substr(L); break; }
        }
        static const struct { const char* name; const char* cats; } T[] = {
            {"l", "Lu Ll Lt Lm Lo"}, {"letter", "Lu Ll Lt Lm Lo"}, {"lc", "Lu Ll Lt"}, {"l&", "Lu Ll Lt"},
            {"casedletter", "Lu Ll Lt"}, {"lu", "Lu"}, {"uppercaseletter", "Lu"}, {"ll", "Ll"},
            {"lowercaseletter", "Ll"}, {"lt", "Lt"}, {"titlecaseletter", "Lt"}, {"lm", "Lm"},
            {"modifierletter", "Lm"}, {"lo", "Lo"}, {"otherletter", "Lo"}, {"m", "Mn Mc Me"},
            {"mark", "Mn Mc Me"}, {"combiningmark", "Mn Mc Me"}, {"mn", "Mn"}, {"nonspacingmark", "Mn"},
            {"mc", "Mc"}, {"spacingmark", "Mc"}, {"me", "Me"}, {"enclosingmark", "Me"}, {"n", "Nd Nl No"},
            {"number", "Nd Nl No"}, {"nd", "Nd"}, {"decimalnumber", "Nd"}, {"digit", "Nd"}, {"nl", "Nl"},
            {"letternumber", "Nl"}, {"no", "No"}, {"othernumber", "No"}, {"p", "Pc Pd Ps Pe Pi Pf Po"},
            {"punctuation", "Pc Pd Ps Pe Pi Pf Po"}, {"punct", "Pc Pd Ps Pe Pi Pf Po"}, {"pc", "Pc"},
            {"connectorpunctuation", "Pc"}, {"pd", "Pd"}, {"dashpunctuation", "Pd"}, {"ps", "Ps"},
            {"openpunctuation", "Ps"}, {"pe", "Pe"}, {"closepunctuation", "Pe"}, {"pi", "Pi"},
            {"initialpunctuation", "Pi"}, {"pf", "Pf"}, {"finalpunctuation", "Pf"}, {"po", "Po"},
            {"otherpunctuation", "Po"}, {"s", "Sm Sc Sk So"}, {"symbol", "Sm Sc Sk So"}, {"sm", "Sm"},
            {"mathsymbol", "Sm"}, {"sc", "Sc"}, {"currencysymbol", "Sc"}, {"sk", "Sk"},
            {"modifiersymbol", "Sk"}, {"so", "So"}, {"othersymbol", "So"}, {"z", "Zs Zl Zp"},
            {"separator", "Zs Zl Zp"}, {"zs", "Zs"}, {"spaceseparator", "Zs"}, {"zl", "Zl"},
            {"lineseparator", "Zl"}, {"zp", "Zp"}, {"paragraphseparator", "Zp"}, {"cc", "Cc"},
            {"control", "Cc"}, {"cntrl", "Cc"}, {"cf", "Cf"}, {"format", "Cf"}, {"co", "Co"},
            {"privateuse", "Co"}, {"cs", "Cs"}, {"surrogate", "Cs"},
        };
        bool found = false;
        for (const auto& t : T) {
            if (n != t.name) continue;
            uint32_t m = 0;
            std::string cs = t.cats;
            for (size_t i = 0; i < cs.size(); i += 3) m |= cat_bit(cs.substr(i, 2).c_str());
            add_cats(b, m);
            found = true;
            break;
        }
        if (!found) {
            if (n == "any") b.add(0, CP_MAX);
            else if (n == "ascii") b.add(0, 0x7F);
            else if (n == "assigned") add_cats(b, 0xffffffffu);
            else if (n == "cn" || n == "unassigned") { add_cats(b, 0xffffffffu); b.negate(); }
            else if (n == "c" || n == "other") {   // Cc Cf Cs Co and the unassigned
                CpSet a;
                add_cats(a, ~cats({"Cc", "Cf", "Cs", "Co"}));
                a.negate();
                b.add(a);
            } else {
                fail("Unicode property not supported (general categories, Any, ASCII and Assigned only)");
            }
        }
        if (neg) b.negate();
    }

    bool posix_class(CpSet& s) {
        // pos_ at "[:"
        size_t end = p_.find(":]", pos_ + 2);
        if (end == std::string::npos) return false;
        std::string name = p_.substr(pos_ + 2, end - pos_ - 2);
        bool neg = !name.empty() && name[0] == '^';
        if (neg) name = name.substr(1);
        CpSet b;
        if (name == "alnum") { b.add('0', '9'); b.add('A', 'Z'); b.add('a', 'z'); }
        else if (name == "alpha") { b.add('A', 'Z'); b.add('a', 'z'); }
        else if (name == "ascii") b.add(0, 0x7f);
        else if (name == "blank") { b.add('\t', '\t'); b.add(' ', ' '); }
        else if (name == "cntrl") { b.add(0, 0x1f); b.add(0x7f, 0x7f); }
        else if (name == "digit") b.add('0', '9');
        else if (name == "graph") b.add('!', '~');
        else if (name == "lower") b.add('a', 'z');
        else if (name == "print") b.add(' ', '~');
        else if (name == "punct") { b.add('!', '/'); b.add(':', '@'); b.add('[', '`'); b.add('{', '~'); }
        else if (name == "space") { b.add('\t', '\r'); b.add(' ', ' '); }
        else if (name == "upper") b.add('A', 'Z');
        else if (name == "word") { b.add('0', '9'); b.add('A', 'Z'); b.add('_', '_'); b.add('a', 'z'); }
        else if (name == "xdigit") { b.add('0', '9'); b.add('A', 'F'); b.add('a', 'f'); }
        else return false;
        if (neg) b.negate();
        s.add(b);
        pos_ = end + 2;
        return true;
    }

    // one class member that is a single scalar (for ranges); -1 if not
    int64_t class_char(CpSet& into, bool* was_set, bool u) {
        *was_set = false;
        uint32_t cp;
        if (peek() == '\\') {
            pos_++;
            if (eof()) fail("incomplete escape sequence");
            CpSet s;
            if (perl_class(s, u)) {
                into.add(s);
                *was_set = true;
                return -1;
            }
            cp = escape_cp(u);
        } else {
            cp = next_cp();
        }
        if (!u && cp > 0x7F) fail("Unicode not allowed here (a class with Unicode mode disabled)");
        return cp;
    }

    // fold the operands of a set operation, as regex-syntax does before it
    // applies the operation (and again to the result)
    static void fold_by(CpSet& s, const Flags& f) {
        if (!f.i) return;
        if (f.u) s.fold();
        else s.fold_ascii();
    }

    // [..]: unions of items, joined left to right by && -- ~~, then the
    // negation; byte mode refuses a class (nested ones included) that ends up
    // with members above 0x7F
    CpSet parse_class(const Flags& f) {
        const size_t open = pos_;
        pos_++;  // '['
        bool neg = false;
        if (!eof() && peek() == '^') { pos_++; neg = true; }
        CpSet acc, s;
        char op = 0;
        bool first = true;
        auto apply = [&]() {
            if (!op) { acc = s; return; }
            fold_by(acc, f);
            fold_by(s, f);
            acc.canon();
            s.canon();
            acc = op == '&' ? CpSet::meet(acc, s) : op == '-' ? CpSet::minus(acc, s) : CpSet::symdiff(acc, s);
        };
        for (;;) {
            if (eof()) { pos_ = open; fail("unclosed character class"); }
            const char c = peek();
            if (c == ']' && !first) { pos_++; break; }
            first = false;
            if (c == '[') {
                if (pos_ + 1 < p_.size() && p_[pos_ + 1] == ':' && posix_class(s)) continue;
                CpSet inner = parse_class(f);
                s.add(inner);
                continue;
            }
            if ((c == '&' || c == '-' || c == '~') && pos_ + 1 < p_.size() && p_[pos_ + 1] == c &&
                !(c == '-' && pos_ + 2 < p_.size() && p_[pos_ + 2] == ']')) {
                apply();
                op = c;
                s = CpSet{};
                pos_ += 2;
                continue;
            }
            bool was_set;
            int64_t lo = class_char(s, &was_set, f.u);
            if (was_set) continue;
            if (!eof() && peek() == '-' && pos_ + 1 < p_.size() && p_[pos_ + 1] != ']') {
                pos_++;
                bool ws2;
                CpSet dummy;
                int64_t hi = class_char(dummy, &ws2, f.u);
                if (ws2) fail("invalid character class range");
                if (hi < lo) fail("invalid character class range");
                s.add((uint32_t)lo, (uint32_t)hi);
            } else {
                s.add((uint32_t)lo, (uint32_t)lo);
            }
        }
        apply();
        fold_by(acc, f);
        if (neg) acc.negate();
        acc.canon();
        if (!f.u && (neg || !acc.is_ascii())) { pos_ = open; fail("pattern can match invalid UTF-8"); }
        return acc;
    }
};

// ------------------------------------------------------------ Thompson NFA
enum NKind : uint8_t { N_BYTE, N_SPLIT, N_EPS, N_MATCH, N_LOOK };  // N_LOOK: assertion lo, then a
struct NState {
    NKind k;
    uint8_t lo, hi;
    uint32_t a, b;
};

struct TooBig {};

class NfaBuilder {
public:
    std::vector<NState> st;
    explicit NfaBuilder(size_t limit) : limit_(limit) {}
    uint32_t add(NKind k, uint32_t a = 0, uint32_t b = 0, uint8_t lo = 0, uint8_t hi = 0) {
        if (st.size() >= limit_) throw TooBig{};
        st.push_back(NState{k, lo, hi, a, b});
        return (uint32_t)st.size() - 1;
    }
    uint32_t build(const std::vector<Node>& ar, int n, uint32_t next) {
        const Node& nd = ar[n];
        switch (nd.k) {
            case K_EMPTY: return next;
            case K_LOOK: return add(N_LOOK, next, 0, (uint8_t)nd.mn);
            case K_CLASS: return cls(nd.set, next);
            case K_CAT: {
                uint32_t s = next;
                for (size_t i = nd.kids.size(); i-- > 0;) s = build(ar, nd.kids[i], s);
                return s;
            }
            case K_ALT: {
                uint32_t s = build(ar, nd.kids.back(), next);
                for (size_t i = nd.kids.size() - 1; i-- > 0;) s = add(N_SPLIT, build(ar, nd.kids[i], next), s);
                return s;
            }
            case K_REP: {
                uint32_t s = next;
                if (nd.mx == INF) {
                    uint32_t loop = add(N_SPLIT, 0, next);
                    uint32_t body = build(ar, nd.kids[0], loop);
                    st[loop].a = body;
                    s = loop;
                } else {
                    for (uint32_t i = nd.mn; i < nd.mx; i++) s = add(N_SPLIT, build(ar, nd.kids[0], s), next);
                }
                for (uint32_t i = 0; i < nd.mn; i++) s = build(ar, nd.kids[0], s);
                return s;
            }
        }
        return next;
    }

private:
    size_t limit_;
    // byte sequence [lo_i, hi_i]... then next
    uint32_t seq(const std::vector<std::pair<uint8_t, uint8_t>>& bs, uint32_t next) {
        uint32_t s = next;
        for (size_t i = bs.size(); i-- > 0;) s = add(N_BYTE, s, 0, bs[i].first, bs[i].second);
        return s;
    }
    static int enc(uint32_t cp, uint8_t* b) {
        if (cp < 0x80) { b[0] = (uint8_t)cp; return 1; }
        if (cp < 0x800) { b[0] = (uint8_t)(0xC0 | (cp >> 6)); b[1] = (uint8_t)(0x80 | (cp & 0x3f)); return 2; }
        if (cp < 0x10000) {
            b[0] = (uint8_t)(0xE0 | (cp >> 12)); b[1] = (uint8_t)(0x80 | ((cp >> 6) & 0x3f));
            b[2] = (uint8_t)(0x80 | (cp & 0x3f));
            return 3;
        }
        b[0] = (uint8_t)(0xF0 | (cp >> 18)); b[1] = (uint8_t)(0x80 | ((cp >> 12) & 0x3f));
        b[2] = (uint8_t)(0x80 | ((cp >> 6) & 0x3f)); b[3] = (uint8_t)(0x80 | (cp & 0x3f));
        return 4;
    }
    // split a scalar range into ranges whose UTF-8 forms are products of byte
    // ranges (same length, differing only in a suffix of full continuation bytes)
    void utf8_split(uint32_t lo, uint32_t hi, std::vector<std::vector<std::pair<uint8_t, uint8_t>>>& out) {
        if (lo > hi) return;
        static const uint32_t bounds[3] = {0x7F, 0x7FF, 0xFFFF};
        for (uint32_t m : bounds)
            if (lo <= m && hi > m) { utf8_split(lo, m, out); utf8_split(m + 1, hi, out); return; }
        if (hi < 0x80) { out.push_back({{(uint8_t)lo, (uint8_t)hi}}); return; }
        const int n = hi < 0x800 ? 2 : hi < 0x10000 ? 3 : 4;
        for (int i = 1; i < n; i++) {
            const uint32_t m = (1u << (6 * i)) - 1;
            if ((lo & ~m) != (hi & ~m)) {
                if ((lo & m) != 0) { utf8_split(lo, lo | m, out); utf8_split((lo | m) + 1, hi, out); return; }
                if ((hi & m) != m) { utf8_split(lo, (hi & ~m) - 1, out); utf8_split(hi & ~m, hi, out); return; }
            }
        }
        uint8_t a[4], b[4];
        enc(lo, a);
        enc(hi, b);
        std::vector<std::pair<uint8_t, uint8_t>> v;
        for (int i = 0; i < n; i++) v.push_back({a[i], b[i]});
        out.push_back(v);
    }
    uint32_t cls(const CpSet& s, uint32_t next) {
        std::vector<std::vector<std::pair<uint8_t, uint8_t>>> seqs;
        for (auto& x : s.r) utf8_split(x.first, x.second, seqs);
        if (seqs.empty()) return add(N_BYTE, next, 0, 1, 0);  // matches nothing (lo > hi)
        uint32_t st0 = seq(seqs.back(), next);
        for (size_t i = seqs.size() - 1; i-- > 0;) st0 = add(N_SPLIT, seq(seqs[i], next), st0);
        return st0;
    }
};

// ------------------------------------------------------------ subset construction
struct VecHash {
    size_t operator()(const std::vector<uint32_t>& v) const {
        uint64_t h = 1469598103934665603ull;
        for (uint32_t x : v) { h ^= x; h *= 1099511628211ull; }
        return (size_t)h;
    }
};

// class of the byte before a position, as far as the assertions can tell
enum Ctx : uint32_t { C_START, C_WORD, C_LF, C_CR, C_OTHER };
inline bool word_byte(int b) {
    return (b >= '0' && b <= '9') || (b >= 'A' && b <= 'Z') || b == '_' || (b >= 'a' && b <= 'z');
}
inline uint32_t ctx_of(int b) { return word_byte(b) ? C_WORD : b == '\n' ? C_LF : b == '\r' ? C_CR : C_OTHER; }
// does assertion l hold between prev and next (a byte, or -1 at the end)?
// (regex-automata's Look semantics; CRLF lines never split "\r\n")
inline bool look_holds(uint8_t l, uint32_t prev, int next) {
    const bool wp = prev == C_WORD, wn = next >= 0 && word_byte(next);
    switch (l) {
        case L_TEXT_START: return prev == C_START;
        case L_TEXT_END: return next < 0;
        case L_LF_START: return prev == C_START || prev == C_LF;
        case L_LF_END: return next < 0 || next == '\n';
        case L_CRLF_START: return prev == C_START || prev == C_LF || (prev == C_CR && next != '\n');
        case L_CRLF_END: return next < 0 || next == '\r' || (next == '\n' && prev != C_CR);
        case L_WORD: return wp != wn;
        case L_NOT_WORD: return wp == wn;
        case L_WORD_START: return !wp && wn;
        case L_WORD_END: return wp && !wn;
        case L_WORD_START_HALF: return !wp;
        case L_WORD_END_HALF: return !wn;
        default: return false;
    }
}

class Determinizer {
public:
    Determinizer(const std::vector<NState>& n, uint32_t start, size_t limit_bytes)
        : n_(n), start_(start), limit_(limit_bytes), mark_(n.size(), 0) {}

    bool run(zs_host_dfa& out, std::string& err) {
        // byte equivalence classes from the NFA's byte ranges (and, with
        // assertions, the bytes they tell apart)
        std::vector<uint8_t> cut(257, 0);
        bool looks = false;
        for (auto& s : n_) {
            if (s.k == N_BYTE && s.lo <= s.hi) { cut[s.lo] = 1; cut[(size_t)s.hi + 1] = 1; }
            if (s.k == N_LOOK) looks = true;
        }
        if (looks)
            for (int b : {(int)'0', '9' + 1, (int)'A', 'Z' + 1, (int)'_', '_' + 1, (int)'a', 'z' + 1, (int)'\n', '\n' + 1, (int)'\r', '\r' + 1})
                cut[b] = 1;
        uint8_t cls_of[256];
        int nc = 0;
        for (int b = 0; b < 256; b++) {
            if (b > 0 && cut[b]) nc++;
            cls_of[b] = (uint8_t)nc;
        }
        nc++;
        std::vector<uint8_t> rep(nc);
        for (int b = 255; b >= 0; b--) rep[cls_of[b]] = (uint8_t)b;
        size_t stride = 1;
        while (stride < (size_t)nc + 1) stride <<= 1;
        const size_t max_states = limit_ / (stride * 4);

        // key: the sorted NFA set, then (when it holds pending assertions)
        // a marker word with the previous-byte context
        std::unordered_map<std::vector<uint32_t>, uint32_t, VecHash> ids;
        std::vector<std::vector<uint32_t>> sets;
        std::vector<uint32_t> ctxs;
        std::vector<uint8_t> acc;
        std::vector<uint32_t> tr;  // [state][class]
        auto intern = [&](std::vector<uint32_t>&& v, uint32_t ctx) -> int64_t {
            bool pend = false;
            for (uint32_t q : v) pend |= n_[q].k == N_LOOK;
            if (!pend) ctx = C_OTHER;
            std::vector<uint32_t> key = v;
            if (pend) key.push_back(0xFFFFFF00u | ctx);
            auto it = ids.find(key);
            if (it != ids.end()) return it->second;
            if (sets.size() >= max_states) return -1;
            uint32_t id = (uint32_t)sets.size();
            acc.push_back(accepting(v, ctx) ? 1 : 0);
            ids.emplace(std::move(key), id);
            sets.push_back(std::move(v));
            ctxs.push_back(ctx);
            return id;
        };
        intern(std::vector<uint32_t>{}, C_OTHER);  // 0: dead (empty set)
        std::vector<uint32_t> s0;
        closure({start_}, s0);
        intern(std::move(s0), C_START);  // 1: start (a non-empty set)
        for (size_t i = 0; i < sets.size(); i++) {
            tr.resize(sets.size() * nc, 0);
            for (int c = 0; c < nc; c++) {
                const uint8_t b = rep[c];
                std::vector<uint32_t> tgt;
                step(sets[i], ctxs[i], b, tgt);
                std::vector<uint32_t> cl;
                if (!tgt.empty()) closure(tgt, cl);
                int64_t id = intern(std::move(cl), ctx_of(b));
                if (id < 0) {
                    err = "DFA exceeded the size limit (" + std::to_string(limit_) + " bytes)";
                    return false;
                }
                tr.resize(sets.size() * nc, 0);
                tr[i * nc + c] = (uint32_t)id;
            }
        }
        minimize_and_emit(tr, acc, nc, cls_of, out);
        return true;
    }

private:
    const std::vector<NState>& n_;
    uint32_t start_;
    size_t limit_;
    std::vector<uint32_t> mark_;
    uint32_t epoch_ = 0;

    // states reachable by empty moves; keeps byte, match and (pending)
    // assertion states
    void closure(const std::vector<uint32_t>& from, std::vector<uint32_t>& out) {
        epoch_++;
        std::vector<uint32_t> stack(from.rbegin(), from.rend());
        while (!stack.empty()) {
            uint32_t q = stack.back();
            stack.pop_back();
            if (mark_[q] == epoch_) continue;
            mark_[q] = epoch_;
            const NState& s = n_[q];
            switch (s.k) {
                case N_BYTE: case N_MATCH: case N_LOOK: out.push_back(q); break;
                case N_EPS: stack.push_back(s.a); break;
                case N_SPLIT: stack.push_back(s.b); stack.push_back(s.a); break;
            }
        }
        std::sort(out.begin(), out.end());
    }
    // the NFA states after byte b from this set, whose previous byte was of
    // class prev: assertions are resolved with (prev, b) on the way
    void step(const std::vector<uint32_t>& set, uint32_t prev, uint8_t b, std::vector<uint32_t>& tgt) {
        epoch_++;
        std::vector<uint32_t> stack(set.rbegin(), set.rend());
        while (!stack.empty()) {
            uint32_t q = stack.back();
            stack.pop_back();
            if (mark_[q] == epoch_) continue;
            mark_[q] = epoch_;
            const NState& s = n_[q];
            switch (s.k) {
                case N_BYTE: if (s.lo <= b && b <= s.hi) tgt.push_back(s.a); break;
                case N_LOOK: if (look_holds(s.lo, prev, b)) stack.push_back(s.a); break;
                case N_EPS: stack.push_back(s.a); break;
                case N_SPLIT: stack.push_back(s.b); stack.push_back(s.a); break;
                default: break;
            }
        }
    }
    // a match is reached at the end of the text from this set
    bool accepting(const std::vector<uint32_t>& set, uint32_t prev) {
        epoch_++;
        std::vector<uint32_t> stack(set.begin(), set.end());
        while (!stack.empty()) {
            uint32_t q = stack.back();
            stack.pop_back();
            if (mark_[q] == epoch_) continue;
            mark_[q] = epoch_;
            const NState& s = n_[q];
            switch (s.k) {
                case N_MATCH: return true;
                case N_LOOK: if (look_holds(s.lo, prev, -1)) stack.push_back(s.a); break;
                case N_EPS: stack.push_back(s.a); break;
                case N_SPLIT: stack.push_back(s.b); stack.push_back(s.a); break;
                default: break;
            }
        }
        return false;
    }

    // Moore partition refinement; block of the empty set becomes state 0
    static void minimize_and_emit(const std::vector<uint32_t>& tr, const std::vector<uint8_t>& acc, int nc,
                                  const uint8_t* cls_of, zs_host_dfa& out) {
        const size_t n = acc.size();
        // states that reach an accepting state; all others share the dead block
        std::vector<std::vector<uint32_t>> rev(n);
        for (size_t s = 0; s < n; s++)
            for (int c = 0; c < nc; c++) rev[tr[s * nc + c]].push_back((uint32_t)s);
        std::vector<uint8_t> live(n, 0);
        std::vector<uint32_t> stack;
        for (size_t s = 0; s < n; s++) if (acc[s]) { live[s] = 1; stack.push_back((uint32_t)s); }
        while (!stack.empty()) {
            uint32_t s = stack.back();
            stack.pop_back();
            for (uint32_t p : rev[s]) if (!live[p]) { live[p] = 1; stack.push_back(p); }
        }
        std::vector<uint32_t> blk(n);
        for (size_t s = 0; s < n; s++) blk[s] = !live[s] ? 0u : acc[s] ? 2u : 1u;
        size_t nb = 0;
        for (;;) {
            std::unordered_map<std::vector<uint32_t>, uint32_t, VecHash> sig;
            std::vector<uint32_t> nbk(n);
            std::vector<uint32_t> key(nc + 1);
            // the dead block keeps id 0
            for (size_t s = 0; s < n; s++) {
                key[0] = blk[s];
                for (int c = 0; c < nc; c++) key[c + 1] = blk[tr[s * nc + c]];
                if (blk[s] == 0) { nbk[s] = 0; continue; }
                auto it = sig.find(key);
                if (it == sig.end()) it = sig.emplace(key, (uint32_t)sig.size() + 1).first;
                nbk[s] = it->second;
            }
            const size_t cnt = sig.size() + 1;
            blk.swap(nbk);
            if (cnt == nb) break;
            nb = cnt;
        }
        // renumber: dead 0, start 1, then in discovery order
        std::vector<int64_t> newid(nb, -1);
        std::vector<uint32_t> order;
        newid[0] = 0;
        order.push_back(0);
        auto visit = [&](uint32_t b) { if (newid[b] < 0) { newid[b] = (int64_t)order.size(); order.push_back(b); } };
        std::vector<uint32_t> rep_of(nb, 0);
        for (size_t s = n; s-- > 0;) rep_of[blk[s]] = (uint32_t)s;
        visit(blk[1]);
        for (size_t i = 1; i < order.size(); i++) {
            const uint32_t s = rep_of[order[i]];
            for (int c = 0; c < nc; c++) visit(blk[tr[s * nc + c]]);
        }
        const size_t m = order.size();
        out.nstates = (uint32_t)m;
        out.start = (uint32_t)newid[blk[1]];
        out.trans.assign(m * 256, 0);
        out.accept.assign(m, 0);
        out.dead.assign(m, 0);
        out.dead[0] = 1;
        for (size_t i = 1; i < m; i++) {
            const uint32_t s = rep_of[order[i]];
            out.accept[i] = acc[s];
            for (int b = 0; b < 256; b++) out.trans[i * 256 + b] = (uint32_t)newid[blk[tr[s * nc + cls_of[b]]]];
        }
    }
};

}  // namespace

int zs_regex_build(const std::string& pattern, zs_host_dfa& out, std::string& err) {
    std::vector<Node> ar;
    int root;
    try {
        Parser p(pattern, ar);
        root = p.parse();
    } catch (const ParseError& e) {
        err = "regex parse error: " + e.msg;
        return -1;
    }
    const size_t limit = (size_t)ZS_REGEX_DFA_LIMIT;
    NfaBuilder nb(limit / 4);
    uint32_t start;
    try {
        uint32_t match = nb.add(N_MATCH);
        start = nb.build(ar, root, match);
    } catch (const TooBig&) {
        err = "regex exceeds the size limit";
        return -1;
    }
    Determinizer d(nb.st, start, limit);
    if (!d.run(out, err)) return -1;
    return 0;
}
