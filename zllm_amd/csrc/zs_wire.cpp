// zs_wire.cpp -- OpenAI wire output fed from the sampler's per-token outputs
// (host only): the hallucination report (Detector::report,
// hallucination.rs:101-125, and its JSON view rest.rs:1494-1503) and the chat
// / legacy-completions logprobs objects (rest.rs:1710-1744).
//
// The JSON text is what serde_json writes for those json! values: compact,
// keys in insertion order (preserve_order; a repeated legacy top_logprobs key
// keeps its first position with the last value), f32 numbers widened to f64
// and printed in ryu's shortest form, non-finite floats as null, strings with
// serde_json's escapes, `bytes` as arrays of integers.
#include <math.h>
#include <stdint.h>
#include <string.h>
#include <new>
#include <string>
#include <utility>
#include <vector>
#include "../../include/zs.h"
#include "zs_json.h"

namespace {

void num(std::string& o, float f) {
    if (!std::isfinite(f)) o += "null";
    else o += zsj::f64_text((double)f);
}

int put_out(const std::string& s, char* out, size_t cap, size_t* need) {
    if (need) *need = s.size() + 1;
    if (!out || cap < s.size() + 1) return ZS_ELIMIT;
    memcpy(out, s.data(), s.size());
    out[s.size()] = '\0';
    return ZS_OK;
}

struct Texts {
    const uint32_t* off;
    const uint8_t* bytes;
    uint32_t n;
    // decode([id]) text; ids the table does not hold decode to ""
    std::string operator()(uint32_t id) const {
        if (id >= n) return std::string();
        return std::string((const char*)bytes + off[id], off[id + 1] - off[id]);
    }
};

void bytes_array(std::string& o, const std::string& s) {
    o += '[';
    for (size_t i = 0; i < s.size(); i++) {
        if (i) o += ',';
        o += std::to_string((unsigned)(unsigned char)s[i]);
    }
    o += ']';
}

}  // namespace

extern "C" int zs_hallucination_report(const float* entropy, const float* max_prob, uint64_t n, uint64_t vocab,
                                       float entropy_threshold, float max_prob_threshold, zs_halluc_report* out) {
    if (!out || (n && (!entropy || !max_prob))) return ZS_EINVAL;
    memset(out, 0, sizeof *out);
    out->peak_token = -1;
    if (n == 0) return ZS_OK;
    // Detector::observe counts a risky token, report() then averages in f32
    // with sequential sums (Iterator::sum::<f32>)
    uint64_t risky = 0;
    float se = -0.0f, sr = -0.0f;
    uint64_t peak = 0;
    for (uint64_t i = 0; i < n; i++) {
        if (entropy[i] > entropy_threshold || max_prob[i] < max_prob_threshold) risky++;
        se = se + entropy[i];
        float r = 1.0f - max_prob[i];  // TokenUncertainty::risk, clamp(0, 1)
        r = r < 0.0f ? 0.0f : (r > 1.0f ? 1.0f : r);
        sr = sr + r;
        // max_by(partial_cmp, unordered = Equal): a later element wins ties
        if (i > 0 && !(entropy[peak] > entropy[i])) peak = i;
    }
    const float mean_e = se / (float)n;
    const float ln_v = logf((float)(vocab > 2 ? vocab : 2));
    float ne = mean_e / ln_v;
    ne = ne < 0.0f ? 0.0f : (ne > 1.0f ? 1.0f : ne);
    out->risk_score = sr / (float)n;
    out->mean_entropy = mean_e;
    out->normalized_entropy = ne;
    out->risky_fraction = (float)risky / (float)n;
    out->peak_token = (int64_t)peak;
    out->n_tokens = n;
    return ZS_OK;
}

extern "C" int zs_hallucination_json(const zs_halluc_report* r, float risk_threshold, char* out, size_t cap,
                                     size_t* need) {
    if (!r) return ZS_EINVAL;
    std::string o = "{\"risk_score\":";
    num(o, r->risk_score);
    o += ",\"mean_entropy\":";
    num(o, r->mean_entropy);
    o += ",\"normalized_entropy\":";
    num(o, r->normalized_entropy);
    o += ",\"risky_fraction\":";
    num(o, r->risky_fraction);
    o += ",\"n_tokens\":" + std::to_string(r->n_tokens);
    o += ",\"peak_token_index\":";
    o += r->peak_token < 0 ? std::string("null") : std::to_string(r->peak_token);
    o += ",\"flagged\":";
    o += r->risk_score >= risk_threshold ? "true" : "false";  // HallucinationReport::flagged
    o += '}';
    try {
        return put_out(o, out, cap, need);
    } catch (const std::bad_alloc&) {
        return ZS_ENOMEM;
    }
}

extern "C" int zs_logprobs_json(int kind, uint32_t n, const uint32_t* ids, const float* logprobs,
                                const uint32_t* top_count, uint32_t top_stride, const uint32_t* top_ids,
                                const float* top_logprobs, const uint32_t* text_offsets, const uint8_t* text,
                                uint32_t ntext, char* out, size_t cap, size_t* need) {
    if ((kind != ZS_LOGPROBS_CHAT && kind != ZS_LOGPROBS_LEGACY) ||
        (n && (!ids || !logprobs || !top_count)) || (!text_offsets && ntext))
        return ZS_EINVAL;
    for (uint32_t i = 0; i < n; i++)
        if (top_count[i] > top_stride || (top_count[i] && (!top_ids || !top_logprobs))) return ZS_EINVAL;
    const Texts dec{text_offsets, text, ntext};
    try {
        std::string o;
        if (kind == ZS_LOGPROBS_CHAT) {
            o = "{\"content\":[";
            for (uint32_t i = 0; i < n; i++) {
                if (i) o += ',';
                const std::string t = dec(ids[i]);
                o += "{\"token\":";
                zsj::write_str(o, t);
                o += ",\"logprob\":";
                num(o, logprobs[i]);
                o += ",\"bytes\":";
                bytes_array(o, t);
                o += ",\"top_logprobs\":[";
                for (uint32_t k = 0; k < top_count[i]; k++) {
                    if (k) o += ',';
                    const size_t q = (size_t)i * top_stride + k;
                    const std::string tt = dec(top_ids[q]);
                    o += "{\"token\":";
                    zsj::write_str(o, tt);
                    o += ",\"logprob\":";
                    num(o, top_logprobs[q]);
                    o += ",\"bytes\":";
                    bytes_array(o, tt);
                    o += '}';
                }
                o += "]}";
            }
            o += "]}";
        } else {
            o = "{\"tokens\":[";
            for (uint32_t i = 0; i < n; i++) {
                if (i) o += ',';
                zsj::write_str(o, dec(ids[i]));
            }
            o += "],\"token_logprobs\":[";
            for (uint32_t i = 0; i < n; i++) {
                if (i) o += ',';
                num(o, logprobs[i]);
            }
            o += "],\"top_logprobs\":[";
            for (uint32_t i = 0; i < n; i++) {
                if (i) o += ',';
                // Map<String, Value> in insertion order; a repeated key keeps
                // its first slot and takes the later value
                std::vector<std::pair<std::string, float>> m;
                for (uint32_t k = 0; k < top_count[i]; k++) {
                    const size_t q = (size_t)i * top_stride + k;
                    std::string key = dec(top_ids[q]);
                    bool found = false;
                    for (auto& e : m)
                        if (e.first == key) { e.second = top_logprobs[q]; found = true; break; }
                    if (!found) m.emplace_back(std::move(key), top_logprobs[q]);
                }
                o += '{';
                for (size_t k = 0; k < m.size(); k++) {
                    if (k) o += ',';
                    zsj::write_str(o, m[k].first);
                    o += ':';
                    num(o, m[k].second);
                }
                o += '}';
            }
            o += "]}";
        }
        return put_out(o, out, cap, need);
    } catch (const std::bad_alloc&) {
        return ZS_ENOMEM;
    }
}
