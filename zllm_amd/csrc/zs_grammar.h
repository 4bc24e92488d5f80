// zs_grammar.h -- host-side grammar compilers shared by the C ABI
// (zs_grammar.cpp): regex -> byte DFA (zs_regex.cpp) and JSON schema -> regex
// (zs_schema.cpp).
#pragma once
#include <stdint.h>
#include <string>
#include <vector>

// DFA size bound of logit_fsm.rs:72 (24 MB), applied to the dense table
// (states x power-of-two stride over the byte classes plus one x 4 bytes).
#define ZS_REGEX_DFA_LIMIT (24u * 1024u * 1024u)

// Anchored byte DFA of the language "the whole text matches": state 0 is the
// dead state (no match reachable); trans[s * 256 + b].
struct zs_host_dfa {
    uint32_t nstates = 0;
    uint32_t start = 0;
    std::vector<uint32_t> trans;
    std::vector<uint8_t> accept;
    std::vector<uint8_t> dead;
};

int zs_regex_build(const std::string& pattern, zs_host_dfa& out, std::string& err);

// json_schema.rs:78-91, 99-112, 114-268
int zs_schema_regex(const std::string& schema_json, std::string& out, std::string& err);
std::string zs_any_json(uint32_t depth);
int zs_tool_envelope(const std::vector<std::string>& names, const std::vector<std::string>& schemas,
                     std::string& out, std::string& err);
