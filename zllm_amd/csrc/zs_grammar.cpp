// zs_grammar.cpp -- C ABI of the host-side grammar compilers (zs.h): regex ->
// anchored byte DFA (zs_regex.cpp) and JSON schema -> regex (zs_schema.cpp).
// Errors are returned as user-facing strings (logit_fsm.rs:190-228 turns them
// into 400s); nothing throws across the boundary.
#include <string.h>
#include <new>
#include <string>
#include <vector>
#include "../../include/zs.h"
#include "zs_grammar.h"

struct zs_grammar {
    zs_host_dfa dfa;
};

namespace {
void put_err(char* err, size_t cap, const std::string& m) {
    if (!err || !cap) return;
    size_t n = m.size() < cap - 1 ? m.size() : cap - 1;
    memcpy(err, m.data(), n);
    err[n] = '\0';
}
// copy a string result: *need = bytes including the terminator; ZS_ELIMIT when
// cap is too small (nothing written)
int put_out(const std::string& s, char* out, size_t cap, size_t* need) {
    if (need) *need = s.size() + 1;
    if (!out || cap < s.size() + 1) return ZS_ELIMIT;
    memcpy(out, s.data(), s.size());
    out[s.size()] = '\0';
    return ZS_OK;
}
}  // namespace

extern "C" int zs_regex_compile(const char* pattern, size_t len, zs_grammar** out, char* err, size_t errcap) {
    if (!out || (!pattern && len)) {
        put_err(err, errcap, "null argument");
        return ZS_EINVAL;
    }
    *out = nullptr;
    zs_grammar* g = new (std::nothrow) zs_grammar;
    if (!g) {
        put_err(err, errcap, "out of host memory");
        return ZS_ENOMEM;
    }
    std::string e;
    int rc;
    try {
        rc = zs_regex_build(std::string(pattern ? pattern : "", len), g->dfa, e);
    } catch (const std::bad_alloc&) {
        rc = -1;
        e = "out of host memory";
    }
    if (rc != 0) {
        delete g;
        put_err(err, errcap, "regex compile failed: " + e);
        return ZS_EINVAL;
    }
    *out = g;
    return ZS_OK;
}

extern "C" void zs_grammar_destroy(zs_grammar* g) { delete g; }

extern "C" int zs_grammar_info(const zs_grammar* g, uint32_t* nstates, uint32_t* start) {
    if (!g) return ZS_EINVAL;
    if (nstates) *nstates = g->dfa.nstates;
    if (start) *start = g->dfa.start;
    return ZS_OK;
}
extern "C" const uint32_t* zs_grammar_trans(const zs_grammar* g) { return g ? g->dfa.trans.data() : nullptr; }
extern "C" const uint8_t* zs_grammar_accept(const zs_grammar* g) { return g ? g->dfa.accept.data() : nullptr; }
extern "C" const uint8_t* zs_grammar_dead(const zs_grammar* g) { return g ? g->dfa.dead.data() : nullptr; }

extern "C" int zs_json_schema_regex(const char* schema, size_t len, char* out, size_t cap, size_t* need, char* err,
                                    size_t errcap) {
    if (!schema && len) {
        put_err(err, errcap, "null argument");
        return ZS_EINVAL;
    }
    std::string re, e;
    try {
        if (zs_schema_regex(std::string(schema ? schema : "", len), re, e) != 0) {
            put_err(err, errcap, e);
            return ZS_EINVAL;
        }
    } catch (const std::bad_alloc&) {
        put_err(err, errcap, "out of host memory");
        return ZS_ENOMEM;
    }
    int rc = put_out(re, out, cap, need);
    if (rc) put_err(err, errcap, "output buffer too small");
    return rc;
}

extern "C" int zs_any_json_regex(uint32_t depth, char* out, size_t cap, size_t* need) {
    try {
        return put_out(zs_any_json(depth), out, cap, need);
    } catch (const std::bad_alloc&) {
        return ZS_ENOMEM;
    }
}

extern "C" int zs_tool_call_envelope_regex(const char* const* names, const char* const* schemas, uint32_t n,
                                           char* out, size_t cap, size_t* need, char* err, size_t errcap) {
    if (n && (!names || !schemas)) {
        put_err(err, errcap, "null argument");
        return ZS_EINVAL;
    }
    std::vector<std::string> nm, sc;
    for (uint32_t i = 0; i < n; i++) {
        if (!names[i] || !schemas[i]) {
            put_err(err, errcap, "null argument");
            return ZS_EINVAL;
        }
        nm.emplace_back(names[i]);
        sc.emplace_back(schemas[i]);
    }
    std::string re, e;
    try {
        if (zs_tool_envelope(nm, sc, re, e) != 0) {
            put_err(err, errcap, e);
            return ZS_EINVAL;
        }
    } catch (const std::bad_alloc&) {
        put_err(err, errcap, "out of host memory");
        return ZS_ENOMEM;
    }
    int rc = put_out(re, out, cap, need);
    if (rc) put_err(err, errcap, "output buffer too small");
    return rc;
}
