// zs_schema.cpp -- JSON schema -> anchored regex (json_schema.rs:78-268), the
// shapeless JSON value grammar (:84-91, :114-127) and the multi-tool call
// envelope (:99-112), plus the small JSON reader / compact writer they need.
//
// Properties are emitted in declaration order (the reader of zs_json.h keeps
// document order, as serde_json with `preserve_order` does). The writer prints
// f64 in the shortest round-trip form with ryu's layout rules (what
// serde_json's to_string prints), so `enum` / `const` literals match byte for
// byte.
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#include <cmath>
#include <string>
#include <utility>
#include <vector>
#include "zs_grammar.h"
#include "zs_json.h"

using zsj::JV;
using zsj::JsonError;
using zsj::Reader;
using zsj::f64_text;
using zsj::write_str;

namespace {

// compact serialization (serde_json::to_string)
void write_json(std::string& o, const JV& v) {
    switch (v.t) {
        case JV::NUL: o += "null"; break;
        case JV::BOOL: o += v.b ? "true" : "false"; break;
        case JV::POS: o += std::to_string(v.u); break;
        case JV::NEG: o += std::to_string(v.i); break;
        case JV::F64: o += f64_text(v.d); break;
        case JV::STR: write_str(o, v.s); break;
        case JV::ARR:
            o += '[';
            for (size_t i = 0; i < v.a.size(); i++) { if (i) o += ','; write_json(o, v.a[i]); }
            o += ']';
            break;
        case JV::OBJ:
            o += '{';
            for (size_t i = 0; i < v.o.size(); i++) {
                if (i) o += ',';
                write_str(o, v.o[i].first);
                o += ':';
                write_json(o, v.o[i].second);
            }
            o += '}';
            break;
    }
}

// Rust's `{:?}` of a str, for error messages
std::string dbg(const std::string& s) {
    std::string o = "\"";
    for (unsigned char c : s) {
        if (c == '"' || c == '\\') { o += '\\'; o += (char)c; }
        else if (c == '\n') o += "\\n";
        else if (c == '\r') o += "\\r";
        else if (c == '\t') o += "\\t";
        else if (c < 0x20 || c == 0x7f) { char b[16]; snprintf(b, sizeof b, "\\u{%x}", c); o += b; }
        else o += (char)c;
    }
    return o + "\"";
}

// ---------------------------------------------------------------- regex pieces
// JSON primitive shapes of json_schema.rs:44-53 (RFC 8259, compact) and the
// optional single space after structural ':' and ','.
const char* const RX_STRING = "\"([^\"\\\\]|\\\\([\"\\\\/bfnrt]|u[0-9a-fA-F]{4}))*\"";
const char* const RX_NUMBER = "-?(0|[1-9][0-9]*)(\\.[0-9]+)?([eE][+-]?[0-9]+)?";
const char* const RX_INTEGER = "-?(0|[1-9][0-9]*)";
const char* const RX_BOOL = "(true|false)";
const char* const RX_NULL = "null";
const std::string SP = " ?";
const int MAX_DEPTH = 32;
const int ANY_DEPTH = 5;

// regex metacharacters escaped so a literal matches itself (json_schema.rs:58-67)
std::string esc(const std::string& s) {
    std::string o;
    for (char c : s) {
        if (strchr("\\.+*?()|[]{}^$", c) && c != '\0') o += '\\';
        o += c;
    }
    return o;
}

std::string literal(const JV& v) {
    std::string j;
    write_json(j, v);
    return esc(j);
}

std::string join(const std::vector<std::string>& v, const std::string& sep) {
    std::string o;
    for (size_t i = 0; i < v.size(); i++) { if (i) o += sep; o += v[i]; }
    return o;
}

std::string any_value(int depth) {
    std::vector<std::string> alts = {RX_STRING, RX_NUMBER, RX_BOOL, RX_NULL};
    if (depth > 0) {
        const std::string in = any_value(depth - 1);
        alts.push_back("\\[" + SP + "(" + in + "(" + SP + "," + SP + in + ")*)?" + SP + "\\]");
        const std::string mem = std::string(RX_STRING) + SP + ":" + SP + in;
        alts.push_back("\\{" + SP + "(" + mem + "(" + SP + "," + SP + mem + ")*)?" + SP + "\\}");
    }
    return "(" + join(alts, "|") + ")";
}

struct SchemaError {
    std::string msg;
};

std::string compile(const JV& sc, int depth);

std::string compile_array(const JV& sc, int depth) {
    const JV* items = sc.get("items");
    if (!items) throw SchemaError{"array schema needs \"items\""};
    const std::string item = compile(*items, depth + 1);
    const JV* jmin = sc.get("minItems");
    const JV* jmax = sc.get("maxItems");
    const uint64_t mn = (jmin && jmin->t == JV::POS) ? jmin->u : 0;
    const bool has_max = jmax && jmax->t == JV::POS;
    const uint64_t mx = has_max ? jmax->u : 0;
    if (has_max) {
        if (mx < mn) throw SchemaError{"maxItems < minItems"};
        if (mx == 0) return "\\[" + SP + "\\]";
    }
    const std::string sep = SP + "," + SP;
    auto times = [&](uint64_t n) {
        if (n > 100000) throw SchemaError{"array bounds too large to unroll"};
        std::vector<std::string> v((size_t)n, item);
        return join(v, sep);
    };
    std::string body;
    if (!has_max) {
        if (mn == 0) body = "(" + item + "(" + sep + item + ")*)?";
        else body = times(mn) + "(" + sep + item + ")*";
    } else {
        std::vector<std::string> parts;
        for (uint64_t c = mn > 1 ? mn : 1; c <= mx; c++) parts.push_back(times(c));
        body = "(" + join(parts, "|") + ")";
        if (mn == 0) body = "(" + body + ")?";
    }
    return "\\[" + SP + body + SP + "\\]";
}

std::string compile_object(const JV& sc, int depth) {
    const JV* props = sc.get("properties");
    if (!props || props->t != JV::OBJ) {
        int d = ANY_DEPTH - depth - 1;
        if (d < 0) d = 0;
        const std::string v = any_value(d);
        const std::string mem = std::string(RX_STRING) + SP + ":" + SP + v;
        return "\\{" + SP + "(" + mem + "(" + SP + "," + SP + mem + ")*)?" + SP + "\\}";
    }
    if (props->o.empty()) return "\\{" + SP + "\\}";
    std::vector<std::string> pairs;
    for (auto& m : props->o) {
        const std::string val = compile(m.second, depth + 1);
        pairs.push_back("\"" + esc(m.first) + "\"" + SP + ":" + SP + val);
    }
    return "\\{" + SP + join(pairs, SP + "," + SP) + SP + "\\}";
}

std::string compile(const JV& sc, int depth) {
    if (depth > MAX_DEPTH)
        throw SchemaError{"schema nesting exceeds " + std::to_string(MAX_DEPTH) + " \xE2\x80\x94 refusing to unroll"};
    if (sc.t != JV::OBJ) throw SchemaError{"schema must be a JSON object"};
    for (const char* k : {"$ref", "oneOf", "anyOf", "allOf", "not", "patternProperties", "if"})
        if (sc.get(k)) throw SchemaError{"schema keyword " + dbg(k) + " is not supported by the regex compiler"};
    if (const JV* c = sc.get("const")) return literal(*c);
    if (const JV* e = sc.get("enum"); e && e->t == JV::ARR) {
        if (e->a.empty()) throw SchemaError{"enum must be non-empty"};
        std::vector<std::string> alts;
        for (auto& v : e->a) alts.push_back(literal(v));
        return "(" + join(alts, "|") + ")";
    }
    const JV* ty = sc.get("type");
    if (!ty || ty->t != JV::STR)
        throw SchemaError{"schema needs a \"type\" (or enum/const); unions via type-arrays are not supported"};
    const std::string& t = ty->s;
    if (t == "string") {
        const JV* p = sc.get("pattern");
        if (p && p->t == JV::STR) return "\"" + p->s + "\"";
        return RX_STRING;
    }
    if (t == "integer") return RX_INTEGER;
    if (t == "number") return RX_NUMBER;
    if (t == "boolean") return RX_BOOL;
    if (t == "null") return RX_NULL;
    if (t == "array") return compile_array(sc, depth);
    if (t == "object") return compile_object(sc, depth);
    throw SchemaError{"unsupported schema type " + dbg(t)};
}

}  // namespace

int zs_schema_regex(const std::string& schema_json, std::string& out, std::string& err) {
    JV sc;
    try {
        sc = Reader(schema_json).parse();
    } catch (const JsonError& e) {
        err = "json_schema: invalid JSON schema: " + e.msg;
        return -1;
    }
    try {
        out = compile(sc, 0);
    } catch (const SchemaError& e) {
        err = e.msg;
        return -1;
    }
    return 0;
}

std::string zs_any_json(uint32_t depth) { return any_value((int)(depth < (uint32_t)MAX_DEPTH ? depth : MAX_DEPTH)); }

int zs_tool_envelope(const std::vector<std::string>& names, const std::vector<std::string>& schemas,
                     std::string& out, std::string& err) {
    if (names.empty()) {
        err = "no tools to build a call envelope from";
        return -1;
    }
    std::vector<std::string> alts;
    for (size_t i = 0; i < names.size(); i++) {
        JV name;
        name.t = JV::STR;
        name.s = names[i];
        JV params;
        try {
            params = Reader(schemas[i]).parse();
        } catch (const JsonError& e) {
            err = "json_schema: invalid JSON schema: " + e.msg;
            return -1;
        }
        std::string args;
        try {
            args = compile(params, 0);
        } catch (const SchemaError& e) {
            err = e.msg;
            return -1;
        }
        alts.push_back("\\{" + SP + "\"name\"" + SP + ":" + SP + literal(name) + SP + "," + SP + "\"arguments\"" + SP +
                       ":" + SP + args + SP + "\\}");
    }
    out = "(" + join(alts, "|") + ")";
    return 0;
}
