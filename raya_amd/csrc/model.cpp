// The decision model on the device: checkpoint config (crates/raya-core/src/config),
// safetensors weights under raya-weights' names (crates/raya-weights/src/{store,mapping}.rs),
// and a batched forward pass equivalent to Network::forward
// (crates/raya-core/src/model.rs:261-348) run once per sequence.
//
// Weights are uploaded once per device.  A forward call packs the valid tokens of
// the batch into one [tokens, hidden] activation (padded positions never exist on
// the device: valid rows do not depend on them, forward_golden.rs:238-262), runs
// every layer as a handful of kernels (LayerNorm, MFMA GEMMs with fused epilogues,
// fused attention), and copies back only the per-sequence outputs.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cerrno>
#include <cinttypes>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <set>
#include <string>
#include <unordered_map>
#include <vector>

#include "internal.hpp"
#include "json.hpp"
#include "raya_hip.h"

namespace raya {
namespace {

// ---------------------------------------------------------------------------------------------
// Errors (crates/raya-core/src/error.rs:5-33): the Display text goes to raya_last_error().

int fail_config(const std::string &field, const std::string &reason) {
    return fail(RAYA_ERR_CONFIG, "invalid config: `%s`: %s", field.c_str(), reason.c_str());
}
int fail_io(const std::string &path, int err) {
    return fail(RAYA_ERR_CONFIG, "cannot read %s: %s (os error %d)", path.c_str(), strerror(err), err);
}
int fail_json(const std::string &path, const std::string &what) {
    return fail(RAYA_ERR_CONFIG, "cannot parse %s: %s", path.c_str(), what.c_str());
}
int fail_unimplemented(const std::string &what) {
    return fail(RAYA_ERR_UNIMPLEMENTED, "not implemented: %s", what.c_str());
}
int fail_input(const std::string &what) { return fail(RAYA_ERR_INPUT, "invalid input: %s", what.c_str()); }

std::string shape_str(const std::vector<uint64_t> &s) {
    std::string out = "[";
    for (size_t i = 0; i < s.size(); ++i) out += (i ? ", " : "") + std::to_string(s[i]);
    return out + "]";
}

int read_file(const std::string &path, std::string &out) {
    FILE *f = fopen(path.c_str(), "rb");
    if (!f) return fail_io(path, errno);
    int rc = RAYA_OK;
    if (fseek(f, 0, SEEK_END) != 0) {
        rc = fail_io(path, errno);
    } else {
        const long size = ftell(f);
        if (size < 0 || fseek(f, 0, SEEK_SET) != 0) {
            rc = fail_io(path, errno);
        } else {
            out.resize((size_t)size);
            if (size > 0 && fread(&out[0], 1, (size_t)size, f) != (size_t)size) rc = fail_io(path, EIO);
        }
    }
    fclose(f);
    return rc;
}

// ---------------------------------------------------------------------------------------------
// Configuration

enum Kind { Uint, Float, Bool, Str, FloatList, FloatMap };

bool accepts(Kind k, const json::Value &v) {
    switch (k) {
    case Uint: return v.is_number() && v.is_u64;
    case Float: return v.is_number();
    case Bool: return v.is_bool();
    case Str: return v.is_string();
    case FloatList:
        if (!v.is_array()) return false;
        for (const auto &x : *v.arr)
            if (!x.is_number()) return false;
        return true;
    default:
        if (!v.is_object()) return false;
        for (const auto &kv : *v.obj)
            if (!kv.second.is_number()) return false;
        return true;
    }
}

const char *expected_of(Kind k) {
    switch (k) {
    case Uint: return "a non-negative integer";
    case Float: return "a number";
    case Bool: return "a boolean";
    case Str: return "a string";
    case FloatList: return "a list of numbers";
    default: return "an object with numeric values";
    }
}

// config/fields.rs:43-58: the keys we read must have the right JSON type; null counts as absent.
int check_types(const json::Value &v, const std::vector<std::pair<const char *, Kind>> &fields) {
    if (!v.is_object()) return fail_config("<root>", "expected a JSON object");
    for (const auto &f : fields) {
        const json::Value *x = v.field(f.first);
        if (x && !accepts(f.second, *x))
            return fail_config(f.first, std::string("expected ") + expected_of(f.second) + ", found " + x->dump());
    }
    return RAYA_OK;
}

int need(const json::Value &v, const char *key, const json::Value **out) {
    *out = v.field(key);
    if (!*out) return fail_config(key, std::string("missing field `") + key + "`");
    return RAYA_OK;
}

struct Config {
    // EncoderConfig (config/encoder.rs:13-35)
    uint64_t hidden = 0, inter = 0, layers = 0, heads = 0, global_every = 0, local_attention = 0;
    uint64_t max_pos = 0, vocab = 0;
    double global_theta = 0, local_theta = 0, norm_eps = 0;
    bool norm_bias = false, attention_bias = false, mlp_bias = false;
    // AgentConfig (config/agent.rs:7-24)
    uint64_t head_layers = 2, max_len = 512, head_max_len = 192, n_act = 1;
    // HeadConfig (config/mod.rs:63-78)
    uint64_t head_heads = 1, head_ffn = 0;

    bool is_global(uint64_t layer) const { return layer % global_every == 0; }
};

int parse_encoder(const json::Value &v, Config &c) {
    int rc = check_types(v, {{"hidden_size", Uint},
                             {"intermediate_size", Uint},
                             {"num_hidden_layers", Uint},
                             {"num_attention_heads", Uint},
                             {"global_attn_every_n_layers", Uint},
                             {"local_attention", Uint},
                             {"max_position_embeddings", Uint},
                             {"vocab_size", Uint},
                             {"norm_eps", Float},
                             {"global_rope_theta", Float},
                             {"local_rope_theta", Float},
                             {"norm_bias", Bool},
                             {"attention_bias", Bool},
                             {"mlp_bias", Bool},
                             {"hidden_activation", Str},
                             {"pad_token_id", Uint},
                             {"cls_token_id", Uint},
                             {"sep_token_id", Uint},
                             {"bos_token_id", Uint},
                             {"eos_token_id", Uint}});
    if (rc) return rc;
    // Required fields, in the order serde reports the first missing one (encoder.rs:160-183).
    const json::Value *x;
    struct U {
        const char *key;
        uint64_t *dst;
    };
    const U ints_a[] = {{"hidden_size", &c.hidden},
                        {"intermediate_size", &c.inter},
                        {"num_hidden_layers", &c.layers},
                        {"num_attention_heads", &c.heads},
                        {"global_attn_every_n_layers", &c.global_every},
                        {"local_attention", &c.local_attention}};
    for (const auto &u : ints_a) {
        if ((rc = need(v, u.key, &x))) return rc;
        *u.dst = x->u64;
    }
    if ((rc = need(v, "norm_eps", &x))) return rc;
    c.norm_eps = x->num;
    const std::pair<const char *, bool *> bools[] = {
        {"norm_bias", &c.norm_bias}, {"attention_bias", &c.attention_bias}, {"mlp_bias", &c.mlp_bias}};
    for (const auto &b : bools) {
        if ((rc = need(v, b.first, &x))) return rc;
        *b.second = x->b;
    }
    const json::Value *act;
    if ((rc = need(v, "hidden_activation", &act))) return rc;
    if ((rc = need(v, "max_position_embeddings", &x))) return rc;
    c.max_pos = x->u64;
    if ((rc = need(v, "vocab_size", &x))) return rc;
    c.vocab = x->u64;

    // Rope thetas (encoder.rs:197-218): rope_parameters per layer type, else the flat 4.x
    // keys, else rope_parameters.rope_theta.
    const json::Value *rp = v.field("rope_parameters");
    const json::Value *flat = rp ? rp->field("rope_theta") : nullptr;
    auto pick = [&](const char *typed, const char *legacy, double *dst) {
        const json::Value *t = rp ? rp->field(typed) : nullptr;
        const json::Value *val = t ? t->field("rope_theta") : nullptr;
        if (!val) val = v.field(legacy);
        if (!val) val = flat;
        if (!val || !val->is_number()) return false;
        *dst = val->num;
        return true;
    };
    if (!pick("full_attention", "global_rope_theta", &c.global_theta))
        return fail_config("global_rope_theta", "missing");
    if (!pick("sliding_attention", "local_rope_theta", &c.local_theta))
        return fail_config("local_rope_theta", "missing");
    if (act->str != "gelu")
        return fail_unimplemented("hidden_activation `" + act->str + "` (only `gelu` is supported)");

    // encoder.rs:118-157
    const std::pair<const char *, uint64_t> positive[] = {
        {"hidden_size", c.hidden},        {"intermediate_size", c.inter},
        {"num_hidden_layers", c.layers},  {"num_attention_heads", c.heads},
        {"global_attn_every_n_layers", c.global_every}, {"local_attention", c.local_attention},
        {"max_position_embeddings", c.max_pos}, {"vocab_size", c.vocab}};
    for (const auto &p : positive)
        if (p.second == 0) return fail_config(p.first, "must be at least 1");
    if (c.hidden % c.heads != 0)
        return fail_config("hidden_size", std::to_string(c.hidden) + " is not divisible by num_attention_heads " +
                                              std::to_string(c.heads));
    const std::pair<const char *, double> positive_f[] = {
        {"global_rope_theta", c.global_theta}, {"local_rope_theta", c.local_theta}, {"norm_eps", c.norm_eps}};
    for (const auto &p : positive_f)
        if (!(std::isfinite(p.second) && p.second > 0.0))
            return fail_config(p.first, "must be a positive finite number");
    return RAYA_OK;
}

int parse_agent(const json::Value &v, Config &c) {
    int rc = check_types(v, {{"encoder", Str},
                             {"head_layers", Uint},
                             {"max_len", Uint},
                             {"head_max_len", Uint},
                             {"temperature", FloatList},
                             {"temperature_by_options", FloatMap},
                             {"act_costs", FloatMap}});
    if (rc) return rc;
    if (const json::Value *x = v.field("head_layers")) c.head_layers = x->u64;
    if (const json::Value *x = v.field("max_len")) c.max_len = x->u64;
    if (const json::Value *x = v.field("head_max_len")) c.head_max_len = x->u64;
    size_t n_temp = 3;
    bool temp_finite = true;
    if (const json::Value *t = v.field("temperature")) {
        n_temp = t->arr->size();
        for (const auto &e : *t->arr) temp_finite = temp_finite && std::isfinite((float)e.num);
    }
    // act_costs: one action per entry plus the default one (agent.rs:43-45); BTreeMap keys
    // are unique, so duplicates in the file count once.
    std::set<std::string> acts;
    bool costs_finite = true, temp_map_finite = true;
    if (const json::Value *a = v.field("act_costs"))
        for (const auto &kv : *a->obj) {
            acts.insert(kv.first);
            costs_finite = costs_finite && std::isfinite((float)kv.second.num);
        }
    if (const json::Value *a = v.field("temperature_by_options"))
        for (const auto &kv : *a->obj) temp_map_finite = temp_map_finite && std::isfinite((float)kv.second.num);
    c.n_act = acts.size() + 1;
    // agent.rs:69-95
    if (c.max_len == 0) return fail_config("max_len", "must be at least 1");
    if (c.head_max_len == 0) return fail_config("head_max_len", "must be at least 1");
    if (n_temp != 3 || !temp_finite) return fail_config("temperature", "must be a list of 3 finite numbers");
    if (!temp_map_finite) return fail_config("temperature_by_options", "values must be finite");
    if (!costs_finite) return fail_config("act_costs", "values must be finite");
    return RAYA_OK;
}

int load_json(const std::string &path, json::Value &out) {
    std::string text;
    int rc = read_file(path, text);
    if (rc) return rc;
    try {
        out = json::parse(text);
    } catch (const json::ParseError &e) {
        return fail_json(path, e.what());
    }
    return RAYA_OK;
}

// ModelConfig::from_dir (config/mod.rs:26-61).
int load_config(const std::string &dir, Config &c) {
    json::Value enc, agent;
    int rc = load_json(dir + "/encoder/config.json", enc);
    if (rc) return rc;
    if ((rc = load_json(dir + "/rl_agent_config.json", agent))) return rc;
    if ((rc = parse_encoder(enc, c))) return rc;
    if ((rc = parse_agent(agent, c))) return rc;
    c.head_heads = std::max<uint64_t>(1, c.hidden / 64);
    if (c.hidden % c.head_heads != 0)
        return fail_config("hidden_size", std::to_string(c.hidden) + " is not divisible by the decision head's " +
                                              std::to_string(c.head_heads) + " heads");
    c.head_ffn = 4 * c.hidden;
    return RAYA_OK;
}

// ---------------------------------------------------------------------------------------------
// Weights: raya-weights' expected parameter set (mapping.rs:19-143) and loader (store.rs:66-151)

struct Entry {
    std::string name;
    std::vector<uint64_t> shape;
    size_t offset = 0;  // in floats, into the packed fp32 parameter buffer
    size_t numel() const {
        size_t n = 1;
        for (uint64_t s : shape) n *= s;
        return n;
    }
};

std::vector<Entry> expected(const Config &c) {
    const uint64_t d = c.hidden, i = c.inter;
    std::vector<Entry> out;
    auto add = [&](const std::string &name, std::vector<uint64_t> shape) { out.push_back({name, std::move(shape)}); };
    add("encoder.embeddings.tok_embeddings.weight", {c.vocab, d});
    add("encoder.embeddings.norm.weight", {d});
    for (uint64_t n = 0; n < c.layers; ++n) {
        const std::string p = "encoder.layers." + std::to_string(n);
        if (n > 0) add(p + ".attn_norm.weight", {d});  // layer 0 has no attn_norm
        add(p + ".attn.Wqkv.weight", {3 * d, d});
        add(p + ".attn.Wo.weight", {d, d});
        add(p + ".mlp_norm.weight", {d});
        add(p + ".mlp.Wi.weight", {2 * i, d});
        add(p + ".mlp.Wo.weight", {d, i});
    }
    add("encoder.final_norm.weight", {d});
    for (uint64_t n = 0; n < c.head_layers; ++n) {
        const std::string p = "head.layers." + std::to_string(n);
        add(p + ".self_attn.in_proj_weight", {3 * d, d});
        add(p + ".self_attn.in_proj_bias", {3 * d});
        add(p + ".self_attn.out_proj.weight", {d, d});
        add(p + ".self_attn.out_proj.bias", {d});
        add(p + ".linear1.weight", {4 * d, d});
        add(p + ".linear1.bias", {4 * d});
        add(p + ".linear2.weight", {d, 4 * d});
        add(p + ".linear2.bias", {d});
        add(p + ".norm1.weight", {d});
        add(p + ".norm1.bias", {d});
        add(p + ".norm2.weight", {d});
        add(p + ".norm2.bias", {d});
    }
    add("type_emb.weight", {3, d});
    add("scorer.0.weight", {d});
    add("scorer.0.bias", {d});
    add("scorer.1.weight", {d, d});
    add("scorer.1.bias", {d});
    add("scorer.3.weight", {1, d});
    add("scorer.3.bias", {1});
    add("act_head.0.weight", {256, d + 4});
    add("act_head.0.bias", {256});
    add("act_head.2.weight", {c.n_act, 256});
    add("act_head.2.bias", {c.n_act});
    add("temperature", {3});
    return out;
}

float bf16_to_f32(uint16_t h) {
    const uint32_t bits = (uint32_t)h << 16;
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

// IEEE binary16 -> binary32, exact (subnormals, infinities and NaN payloads kept).
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const uint32_t exp = (h >> 10) & 0x1f, man = h & 0x3ff;
    uint32_t bits;
    if (exp == 0 && man == 0) {
        bits = sign;
    } else if (exp == 0) {
        uint32_t p = 31 - __builtin_clz(man);  // top set bit, 0..9
        bits = sign | ((p + 103) << 23) | ((man << (23 - p)) & 0x007fffff);
    } else if (exp == 31) {
        bits = sign | 0x7f800000 | (man << 13);
    } else {
        bits = sign | ((exp + 112) << 23) | (man << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

struct Weights {
    std::vector<Entry> entries;
    std::unordered_map<std::string, size_t> index;  // name -> entry
    std::vector<float> host;                        // packed fp32, each tensor 64-float aligned
};

int load_weights(const std::string &path, const Config &c, Weights &w) {
    const std::pair<bool, const char *> flags[] = {
        {c.attention_bias, "attention_bias"}, {c.mlp_bias, "mlp_bias"}, {c.norm_bias, "norm_bias"}};
    for (const auto &f : flags)
        if (f.first) return fail_unimplemented(std::string(f.second) + "=true (bias tensors are not part of Raya-L)");
    w.entries = expected(c);
    std::string buf;
    int rc = read_file(path, buf);
    if (rc) return rc;

    // LoadReport (error.rs:35-91)
    std::vector<std::string> missing, unused, duplicate, shape_lines;
    auto report = [&](const std::string &detail) {
        std::string s = "invalid weights file " + path;
        if (!detail.empty()) s += ": " + detail;
        const std::pair<const char *, std::vector<std::string> *> groups[] = {
            {"missing tensors", &missing}, {"unexpected tensors", &unused}, {"duplicate tensors", &duplicate}};
        for (const auto &g : groups) {
            if (g.second->empty()) continue;
            std::vector<std::string> sorted = *g.second;
            std::sort(sorted.begin(), sorted.end());
            s += std::string("\n  ") + g.first + ":";
            for (const auto &n : sorted) s += "\n    " + n;
        }
        if (!shape_lines.empty()) {
            std::vector<std::string> sorted = shape_lines;
            std::sort(sorted.begin(), sorted.end());
            s += "\n  shape mismatches:";
            for (const auto &n : sorted) s += "\n    " + n;
        }
        return fail(RAYA_ERR_WEIGHTS, "%s", s.c_str());
    };

    // safetensors layout: u64 LE header length, JSON header, then the data buffer.
    if (buf.size() < 8) return report("header too small");
    uint64_t hlen = 0;
    memcpy(&hlen, buf.data(), 8);
    if (hlen > buf.size() - 8) return report("invalid header length");
    json::Value header;
    try {
        header = json::parse(buf.data() + 8, (size_t)hlen);
    } catch (const json::ParseError &e) {
        return report(std::string("invalid header: ") + e.what());
    }
    if (!header.is_object()) return report("invalid header: not a JSON object");
    const char *data = buf.data() + 8 + hlen;
    const uint64_t data_len = buf.size() - 8 - hlen;

    struct Tensor {
        std::string dtype;
        std::vector<uint64_t> shape;
        uint64_t begin = 0, end = 0;
    };
    std::map<std::string, Tensor> tensors;
    std::set<std::string> seen;
    std::set<std::string> dup_set;
    std::vector<std::string> unsupported;
    for (const auto &kv : *header.obj) {
        if (kv.first == "__metadata__") continue;
        if (!seen.insert(kv.first).second) dup_set.insert(kv.first);
        const json::Value &t = kv.second;
        const json::Value *dt = t.get("dtype"), *sh = t.get("shape"), *off = t.get("data_offsets");
        if (!dt || !dt->is_string() || !sh || !sh->is_array() || !off || !off->is_array() || off->arr->size() != 2)
            return report("invalid header entry for " + kv.first);
        Tensor x;
        x.dtype = dt->str;
        for (const auto &e : *sh->arr) {
            if (!e.is_u64) return report("invalid shape for " + kv.first);
            x.shape.push_back(e.u64);
        }
        if (!(*off->arr)[0].is_u64 || !(*off->arr)[1].is_u64) return report("invalid offsets for " + kv.first);
        x.begin = (*off->arr)[0].u64;
        x.end = (*off->arr)[1].u64;
        uint64_t numel = 1;
        for (uint64_t s : x.shape) numel *= s;
        const uint64_t size = x.dtype == "F32" || x.dtype == "I32" || x.dtype == "U32" ? 4
                              : x.dtype == "F16" || x.dtype == "BF16" || x.dtype == "I16" || x.dtype == "U16" ? 2
                              : x.dtype == "F64" || x.dtype == "I64" || x.dtype == "U64" ? 8
                                                                                      : 1;
        if (x.end < x.begin || x.end > data_len || x.end - x.begin != numel * size)
            return report("invalid data offsets for " + kv.first);
        if (x.dtype != "F32" && x.dtype != "F16" && x.dtype != "BF16")
            unsupported.push_back(kv.first + " (" + x.dtype + ")");
        tensors[kv.first] = x;
    }
    if (!unsupported.empty()) {
        std::sort(unsupported.begin(), unsupported.end());
        std::string list;
        for (size_t i = 0; i < unsupported.size(); ++i) list += (i ? ", " : "") + unsupported[i];
        return fail_unimplemented("unsupported tensor dtypes in " + path + ": " + list +
                                  " (only F32, F16 and BF16 are loaded; F16 and BF16 are widened to fp32)");
    }
    duplicate.assign(dup_set.begin(), dup_set.end());
    std::set<std::string> known;
    for (const auto &e : w.entries) known.insert(e.name);
    for (const auto &kv : tensors)
        if (!known.count(kv.first)) unused.push_back(kv.first);
    for (const auto &e : w.entries) {
        auto it = tensors.find(e.name);
        if (it == tensors.end()) {
            missing.push_back(e.name);
            continue;
        }
        if (it->second.shape != e.shape || it->second.end == it->second.begin)
            shape_lines.push_back(e.name + ": expected " + shape_str(e.shape) + ", found " + shape_str(it->second.shape));
    }
    if (!missing.empty() || !unused.empty() || !duplicate.empty() || !shape_lines.empty()) return report("");

    // Pack every parameter as fp32 (F16/BF16 widened exactly, store.rs:198-232).
    size_t total = 0;
    for (auto &e : w.entries) {
        e.offset = total;
        total += (e.numel() + 63) / 64 * 64;
    }
    w.host.assign(total, 0.0f);
    for (size_t k = 0; k < w.entries.size(); ++k) {
        const Entry &e = w.entries[k];
        w.index[e.name] = k;
        const Tensor &t = tensors[e.name];
        const char *src = data + t.begin;
        float *dst = w.host.data() + e.offset;
        const size_t n = e.numel();
        if (t.dtype == "F32") {
            memcpy(dst, src, n * 4);
        } else if (t.dtype == "F16") {
            for (size_t j = 0; j < n; ++j) {
                uint16_t h;
                memcpy(&h, src + 2 * j, 2);
                dst[j] = f16_to_f32(h);
            }
        } else {
            for (size_t j = 0; j < n; ++j) {
                uint16_t h;
                memcpy(&h, src + 2 * j, 2);
                dst[j] = bf16_to_f32(h);
            }
        }
    }
    return RAYA_OK;
}

// ---------------------------------------------------------------------------------------------
// Device state

struct DeviceBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
    DeviceBuf() = default;
    DeviceBuf(const DeviceBuf &) = delete;  // one owner per allocation
    DeviceBuf &operator=(const DeviceBuf &) = delete;
    ~DeviceBuf() {
        if (ptr) (void)hipFree(ptr);
    }
    int reserve(size_t want) {
        if (bytes >= want) return RAYA_OK;
        if (ptr) {
            hipError_t e = hipFree(ptr);
            ptr = nullptr;
            bytes = 0;
            if (e != hipSuccess) return fail_device(e, "hipFree");
        }
        hipError_t e = hipMalloc(&ptr, want);
        if (e != hipSuccess) return fail_device(e, "hipMalloc");
        bytes = want;
        return RAYA_OK;
    }
};

// Rotary tables of one theta: [positions][head_dim / 2] cos and sin, as rope_in_place builds
// them (ops.rs:124-132): inv_freq = 1 / theta^(2i / head_dim) and angle = pos * inv_freq in f32.
void rope_table(float theta, int head_dim, int positions, std::vector<float> &cos_t, std::vector<float> &sin_t) {
    const int half = head_dim / 2;
    std::vector<float> inv(half);
    for (int i = 0; i < half; ++i) inv[i] = 1.0f / powf(theta, (float)(2 * i) / (float)head_dim);
    cos_t.resize((size_t)positions * half);
    sin_t.resize((size_t)positions * half);
    for (int p = 0; p < positions; ++p)
        for (int i = 0; i < half; ++i) {
            const float angle = (float)p * inv[i];
            cos_t[(size_t)p * half + i] = cosf(angle);
            sin_t[(size_t)p * half + i] = sinf(angle);
        }
}

// The encoder's pre-LN LayerNorms folded into the GEMMs that read them (GemmLaunch::in_stats):
// per layer, Wqkv (layers >= 1, after attn_norm) and Wi (after mlp_norm) with the norm's gain
// multiplied into their columns, and each folded weight row's sum.  Offsets in floats into `buf`.
struct FoldedNorms {
    DeviceBuf buf;
    std::vector<size_t> qkv, qkv_sum, wi, wi_sum;
};

struct DeviceModel {
    int device = -1;
    DeviceBuf params;
    DeviceBuf rope;  // global cos, global sin, local cos, local sin: [rope_len][head_dim / 2] each
    int rope_len = 0;
    DeviceBuf work;
    DeviceBuf act_w;  // act_head.0.weight [256][d + 4] with its rows padded by zeros to ld_act
    FoldedNorms folded;
};

}  // namespace

struct Model {
    Config cfg;
    Weights w;
    std::mutex mu;
    std::unordered_map<int, std::unique_ptr<DeviceModel>> dev;
    int profile = 0;                                    // stage timing level (0: off)
    std::vector<std::pair<std::string, double>> stages;  // the last forward's stage times, ms
};

namespace {

const float *param(const Model &m, const DeviceModel &dm, const std::string &name) {
    auto it = m.w.index.find(name);
    if (it == m.w.index.end()) return nullptr;
    return (const float *)dm.params.ptr + m.w.entries[it->second].offset;
}

int ensure_device(Model &m, DeviceModel **out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail_device(e, "hipGetDevice");
    auto &slot = m.dev[dev];
    if (!slot) {
        auto dm = std::make_unique<DeviceModel>();
        dm->device = dev;
        int rc = dm->params.reserve(m.w.host.size() * sizeof(float));
        if (rc) return rc;
        e = hipMemcpy(dm->params.ptr, m.w.host.data(), m.w.host.size() * sizeof(float), hipMemcpyHostToDevice);
        if (e != hipSuccess) return fail_device(e, "upload weights");
        slot = std::move(dm);
    }
    *out = slot.get();
    return RAYA_OK;
}

int ensure_act_weight(const Model &m, DeviceModel &dm, uint64_t ld_act) {
    if (dm.act_w.ptr) return RAYA_OK;
    auto it = m.w.index.find("act_head.0.weight");
    if (it == m.w.index.end()) return fail(RAYA_ERR_WEIGHTS, "missing act_head.0.weight");
    const uint64_t k = m.cfg.hidden + 4, rows = 256;
    const float *src = m.w.host.data() + m.w.entries[it->second].offset;
    std::vector<float> host(rows * ld_act, 0.0f);
    for (uint64_t r = 0; r < rows; ++r) memcpy(host.data() + r * ld_act, src + r * k, k * sizeof(float));
    int rc = dm.act_w.reserve(host.size() * sizeof(float));
    if (rc) return rc;
    const hipError_t e = hipMemcpy(dm.act_w.ptr, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail_device(e, "upload the padded act head weight");
    return RAYA_OK;
}

// LN(x) W^T = rstd ((x - c) (g * W)^T - (mean - c) colsum) with g the norm's gain, colsum[j]
// the row sums of g * W and c a per-row centre (0, or the mean's leading part for rows far
// from zero; GemmLaunch::in_stats).  Built on the host once per device: the products
// g_t W[j][t] in f32 (as LN's output times W rounds them) and their row sums in f64.  The
// residual GEMMs that produce the statistics need whole 64-column chunks (hidden a multiple of
// 64) and the ring kernel (every GEMM depth a multiple of 16: hidden and the MLP's intermediate
// size); other shapes keep the LayerNorm kernels.
bool norms_foldable(const Config &c) { return c.hidden % 64 == 0 && c.inter % 16 == 0; }

int ensure_folded(const Model &m, DeviceModel &dm) {
    const Config &c = m.cfg;
    if (!dm.folded.qkv.empty() || !norms_foldable(c)) return RAYA_OK;
    const uint64_t d = c.hidden, n3 = 3 * d, n2 = 2 * c.inter;
    std::vector<float> host;
    host.reserve((size_t)c.layers * (n3 + n2) * (d + 1));
    FoldedNorms f;
    std::vector<float> sums;
    // Appends the folded block (rows x d) and then its row sums; blocks stay 16-byte aligned
    // because d and every row count here are multiples of 4.
    auto fold = [&](const std::string &w, const std::string &gain, uint64_t rows, std::vector<size_t> &off,
                    std::vector<size_t> &off_sum) -> int {
        const auto iw = m.w.index.find(w), ig = m.w.index.find(gain);
        if (iw == m.w.index.end() || ig == m.w.index.end())
            return fail(RAYA_ERR_WEIGHTS, "missing %s", (iw == m.w.index.end() ? w : gain).c_str());
        const float *wp = m.w.host.data() + m.w.entries[iw->second].offset;
        const float *gp = m.w.host.data() + m.w.entries[ig->second].offset;
        off.push_back(host.size());
        sums.assign(rows, 0.0f);
        for (uint64_t j = 0; j < rows; ++j) {
            double sum = 0.0;
            for (uint64_t t = 0; t < d; ++t) {
                const float x = wp[j * d + t] * gp[t];
                host.push_back(x);
                sum += x;
            }
            sums[j] = (float)sum;
        }
        off_sum.push_back(host.size());
        host.insert(host.end(), sums.begin(), sums.end());
        return RAYA_OK;
    };
    for (uint64_t i = 0; i < c.layers; ++i) {
        const std::string p = "encoder.layers." + std::to_string(i);
        int rc = RAYA_OK;
        if (i > 0) {
            rc = fold(p + ".attn.Wqkv.weight", p + ".attn_norm.weight", n3, f.qkv, f.qkv_sum);
        } else {  // layer 0 has no attn_norm
            f.qkv.push_back(0);
            f.qkv_sum.push_back(0);
        }
        if (!rc) rc = fold(p + ".mlp.Wi.weight", p + ".mlp_norm.weight", n2, f.wi, f.wi_sum);
        if (rc) return rc;
    }
    // Empty offsets mean "not built": they are set only once the upload has succeeded.
    int rc = dm.folded.buf.reserve(host.size() * sizeof(float));
    if (rc) return rc;
    const hipError_t e = hipMemcpy(dm.folded.buf.ptr, host.data(), host.size() * sizeof(float), hipMemcpyHostToDevice);
    if (e != hipSuccess) return fail_device(e, "upload folded norm weights");
    dm.folded.qkv = std::move(f.qkv);
    dm.folded.qkv_sum = std::move(f.qkv_sum);
    dm.folded.wi = std::move(f.wi);
    dm.folded.wi_sum = std::move(f.wi_sum);
    return RAYA_OK;
}

// RAYA_LN_FUSION=0 keeps the LayerNorm kernels (for comparison); otherwise the pre-LN norms
// are folded whenever the hidden size allows.
bool fuse_norms(const Config &c) {
    const char *e = std::getenv("RAYA_LN_FUSION");
    return norms_foldable(c) && !(e && !std::strcmp(e, "0"));
}

int ensure_rope(const Model &m, DeviceModel &dm, int len) {
    if (dm.rope_len >= len) return RAYA_OK;
    int want = 1024;
    while (want < len) want *= 2;
    const int hd = (int)(m.cfg.hidden / m.cfg.heads), half = hd / 2;
    const size_t one = (size_t)want * half;
    int rc = dm.rope.reserve(4 * one * sizeof(float));
    if (rc) return rc;
    std::vector<float> c, s;
    const double thetas[2] = {m.cfg.global_theta, m.cfg.local_theta};
    for (int t = 0; t < 2; ++t) {
        rope_table((float)thetas[t], hd, want, c, s);
        hipError_t e = hipMemcpy((float *)dm.rope.ptr + (2 * t) * one, c.data(), one * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess)
            e = hipMemcpy((float *)dm.rope.ptr + (2 * t + 1) * one, s.data(), one * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) return fail_device(e, "upload rope tables");
    }
    dm.rope_len = want;
    return RAYA_OK;
}

// Sub-allocation of the per-call workspace.
struct Carve {
    char *base;
    size_t off = 0;
    template <typename T>
    T *take(size_t n) {
        T *p = (T *)(base + off);
        off += (n * sizeof(T) + 255) / 256 * 256;
        return p;
    }
};

#define TRY_HIP(expr, what)                                   \
    do {                                                      \
        hipError_t e_ = (expr);                               \
        if (e_ != hipSuccess) return fail_device(e_, (what)); \
    } while (0)

}  // namespace
}  // namespace raya

using namespace raya;

extern "C" {

int raya_model_load(const char *checkpoint_dir, const char *weights_path, raya_model **out) {
    if (!checkpoint_dir || !out) return fail(RAYA_ERR_CONFIG, "invalid config: `<root>`: no checkpoint directory");
    *out = nullptr;
    auto m = std::make_unique<Model>();
    int rc = load_config(checkpoint_dir, m->cfg);
    if (rc) return rc;
    const std::string wpath = weights_path ? weights_path : std::string(checkpoint_dir) + "/model.safetensors";
    if ((rc = load_weights(wpath, m->cfg, m->w))) return rc;
    *out = (raya_model *)m.release();
    return ok();
}

void raya_model_free(raya_model *model) { delete (Model *)model; }

int raya_expected_params(const char *checkpoint_dir, raya_param_entry *out, uint64_t capacity,
                         uint64_t *count) {
    if (!checkpoint_dir || !count) return fail(RAYA_ERR_CONFIG, "invalid config: `<root>`: no checkpoint directory");
    Config c;
    int rc = load_config(checkpoint_dir, c);
    if (rc) return rc;
    const std::pair<bool, const char *> flags[] = {
        {c.attention_bias, "attention_bias"}, {c.mlp_bias, "mlp_bias"}, {c.norm_bias, "norm_bias"}};
    for (const auto &f : flags)
        if (f.first) return fail_unimplemented(std::string(f.second) + "=true (bias tensors are not part of Raya-L)");
    const std::vector<Entry> e = expected(c);
    *count = e.size();
    for (uint64_t i = 0; i < e.size() && i < capacity && out; ++i) {
        snprintf(out[i].name, sizeof out[i].name, "%s", e[i].name.c_str());
        out[i].ndim = (uint32_t)e[i].shape.size();
        for (size_t j = 0; j < 4; ++j) out[i].shape[j] = j < e[i].shape.size() ? e[i].shape[j] : 0;
    }
    return ok();
}

int raya_model_get_info(const raya_model *model, raya_model_info *info) {
    if (!model || !info) return fail(RAYA_ERR_INPUT, "invalid input: null model or info");
    const Config &c = ((const Model *)model)->cfg;
    info->hidden_size = c.hidden;
    info->intermediate_size = c.inter;
    info->num_hidden_layers = c.layers;
    info->num_attention_heads = c.heads;
    info->global_attn_every_n_layers = c.global_every;
    info->local_attention = c.local_attention;
    info->vocab_size = c.vocab;
    info->max_position_embeddings = c.max_pos;
    info->global_rope_theta = c.global_theta;
    info->local_rope_theta = c.local_theta;
    info->norm_eps = c.norm_eps;
    info->head_layers = c.head_layers;
    info->head_heads = c.head_heads;
    info->head_ffn = c.head_ffn;
    info->n_act = c.n_act;
    info->param_floats = ((const Model *)model)->w.host.size();
    return ok();
}

int raya_model_set_profiling(raya_model *model, int level) {
    if (!model) return fail(RAYA_ERR_INPUT, "invalid input: null model");
    if (level < 0 || level > 2) return fail(RAYA_ERR_INPUT, "invalid input: profiling level must be 0, 1 or 2");
    Model &m = *(Model *)model;
    std::lock_guard<std::mutex> lock(m.mu);
    m.profile = level;
    m.stages.clear();
    return ok();
}

int raya_model_stage_times(raya_model *model, raya_stage_time *out, uint64_t capacity, uint64_t *count) {
    if (!model || !count) return fail(RAYA_ERR_INPUT, "invalid input: null model or count");
    Model &m = *(Model *)model;
    std::lock_guard<std::mutex> lock(m.mu);
    *count = m.stages.size();
    for (uint64_t i = 0; i < m.stages.size() && i < capacity && out; ++i) {
        memset(out[i].name, 0, sizeof out[i].name);
        strncpy(out[i].name, m.stages[i].first.c_str(), sizeof out[i].name - 1);
        out[i].ms = m.stages[i].second;
    }
    return ok();
}

int raya_model_forward(raya_model *model, const raya_forward_batch *in, raya_forward_output *out,
                       raya_trace_fn trace, void *user, void *stream_ptr) {
    if (!model || !in || !out) return fail(RAYA_ERR_INPUT, "invalid input: null model, batch or output");
    Model &m = *(Model *)model;
    const Config &c = m.cfg;
    const uint64_t B = in->batch, L = in->seq, K = in->markers;
    const uint64_t d = c.hidden;

    // Network::check (model.rs:221-258) per sequence, in its order.
    if (B == 0) return fail_input("empty batch");
    if (!in->input_ids || !in->valid_len || !in->marker_pos || !in->marker_mask || !in->qtype)
        return fail_input("null input array");
    for (uint64_t b = 0; b < B; ++b) {
        const uint32_t *ids = in->input_ids + b * L;
        for (uint64_t t = 0; t < L; ++t)
            if (ids[t] >= c.vocab)
                return fail_input("token id " + std::to_string(ids[t]) + " is outside the vocabulary of " +
                                  std::to_string(c.vocab));
        const uint64_t valid = in->valid_len[b];
        if (valid == 0 || valid > L)
            return fail_input("valid_len " + std::to_string(valid) + " is not in 1..=" + std::to_string(L));
        if (K == 0) return fail_input("marker_pos and marker_mask must be non-empty and the same length");
        bool any = false;
        for (uint64_t j = 0; j < K; ++j) {
            const uint64_t pos = in->marker_pos[b * K + j];
            const bool mv = in->marker_mask[b * K + j] != 0;
            if (pos >= L || (mv && pos >= valid))
                return fail_input("marker position " + std::to_string(pos) + " is outside the sequence (valid_len " +
                                  std::to_string(valid) + ", length " + std::to_string(L) + ")");
            any = any || mv;
        }
        if (!any) return fail_input("no valid marker");
        if (in->qtype[b] > 2) return fail_input("qtype " + std::to_string(in->qtype[b]) + " is not 0, 1 or 2");
    }
    const uint64_t hd = d / c.heads, hh = c.head_heads, hhd = d / hh;
    for (uint64_t dim : {hd, hhd}) {
        if (dim % 8 != 0)
            return fail(RAYA_ERR_KERNEL, "attention kernel: invalid shape: head_dim %" PRIu64 " is not a multiple of 8",
                        dim);
        if (dim > (uint64_t)kMaxHeadDim)
            return fail(RAYA_ERR_KERNEL,
                        "attention kernel: unsupported: head_dim %" PRIu64 " (the HIP kernel handles up to %d)", dim,
                        kMaxHeadDim);
    }
    int32_t local_kind = RAYA_MASK_SLIDING;
    uint64_t local_arg = c.local_attention / 2;  // encoder.rs:119
    if (in->local_override) {
        local_kind = in->local_mask_kind;
        local_arg = in->local_mask_arg;
        if (local_kind < RAYA_MASK_BLOCK3 || local_kind > RAYA_MASK_BLOCKDIAG)
            return fail(RAYA_ERR_KERNEL, "attention kernel: unsupported: mask kind %d", local_kind);
        if (local_kind == RAYA_MASK_BLOCKDIAG && local_arg == 0)
            return fail(RAYA_ERR_KERNEL, "attention kernel: invalid shape: block_diag width must be at least 1");
    }

    // Pack the valid tokens.
    std::vector<int32_t> ints;  // ids | positions | row_seq | seq_start | valid | qtype | marker rows
    uint64_t T = 0, Lmax = 0;
    for (uint64_t b = 0; b < B; ++b) {
        T += in->valid_len[b];
        Lmax = std::max(Lmax, in->valid_len[b]);
    }
    if (T > 0x7fffffffULL / std::max<uint64_t>(3 * d, 4 * d) || L >= (1ULL << 30))
        return fail(RAYA_ERR_UNSUPPORTED, "unsupported: %" PRIu64 " tokens in one batch", T);
    const size_t o_ids = 0, o_pos = T, o_rs = 2 * T, o_start = 3 * T, o_valid = o_start + B, o_q = o_valid + B,
                 o_mrow = o_q + B, n_ints = o_mrow + B * K;
    ints.resize(n_ints);
    std::vector<uint8_t> mask(B * K);
    {
        uint64_t row = 0;
        for (uint64_t b = 0; b < B; ++b) {
            const uint64_t valid = in->valid_len[b];
            ints[o_start + b] = (int32_t)row;
            ints[o_valid + b] = (int32_t)valid;
            ints[o_q + b] = (int32_t)in->qtype[b];
            for (uint64_t t = 0; t < valid; ++t) {
                ints[o_ids + row + t] = (int32_t)in->input_ids[b * L + t];
                ints[o_pos + row + t] = (int32_t)t;
                ints[o_rs + row + t] = (int32_t)b;
            }
            for (uint64_t j = 0; j < K; ++j) {
                const uint64_t pos = in->marker_pos[b * K + j];
                // An invalid marker may point at padding, which is not materialised: its
                // logit is replaced by -1e4 regardless of the row it reads.
                ints[o_mrow + b * K + j] = pos < valid ? (int32_t)(row + pos) : -1;
                mask[b * K + j] = in->marker_mask[b * K + j] ? 1 : 0;
            }
            row += valid;
        }
    }

    std::lock_guard<std::mutex> lock(m.mu);
    DeviceModel *dmp = nullptr;
    int rc = ensure_device(m, &dmp);
    if (rc) return rc;
    DeviceModel &dm = *dmp;
    if ((rc = ensure_rope(m, dm, (int)Lmax))) return rc;
    const bool fused = fuse_norms(c);
    if (fused && (rc = ensure_folded(m, dm))) return rc;
    hipStream_t stream = (hipStream_t)stream_ptr;

    const uint64_t inter = c.inter, big = std::max(inter, c.head_ffn), nact = c.n_act;
    const uint64_t BK = B * K;
    // The act head's first Linear has depth d + 4; its input rows and weight are padded with
    // zeros to a multiple of 16 so that it runs on the ring kernel (and splits K).
    const uint64_t ld_act = (d + 4 + 15) / 16 * 16;
    if ((rc = ensure_act_weight(m, dm, ld_act))) return rc;
    // Split-K partials for the encoder GEMMs when the tokens are too few for their tiles to
    // fill the compute units (a single short sequence); other GEMMs split only if they fit.
    size_t split_cap = 0;
    {
        const uint64_t shapes[4][3] = {{3 * d, d, RAYA_EPI_NONE}, {d, d, RAYA_EPI_NONE}, {inter, d, RAYA_EPI_GEGLU},
                                       {d, inter, RAYA_EPI_NONE}};
        for (const auto &sh : shapes) {
            const int act = (int)sh[2];
            split_cap = std::max(split_cap, gemm_split_floats((int)T, (int)sh[0], act,
                                                              gemm_splits((int)T, (int)sh[0], (int)sh[1], act)));
        }
    }
    size_t need = 0;
    {
        Carve probe{nullptr};
        probe.take<int32_t>(n_ints);
        probe.take<uint8_t>(BK);
        probe.take<float>(T * d);        // h
        probe.take<float>(T * d);        // normed
        probe.take<float>(T * 3 * d);    // qkv
        probe.take<float>(T * d);        // ctx
        probe.take<float>(T * big);      // gated / head hidden
        probe.take<float>(BK * d * 3);   // states, normed states, scorer hidden
        probe.take<float>(BK * 3);       // raw logits, logits, probabilities
        probe.take<float>(B * 4);        // features
        probe.take<float>(B * d);        // pooled
        probe.take<float>(B * ld_act);   // act input, rows padded to the act head's depth
        probe.take<float>(B * 256);      // act hidden
        probe.take<float>(B * nact);     // act logits
        probe.take<float4>(T * (d / 64));   // LayerNorm chunk statistics of h
        probe.take<float4>(T);              // and each row's (mean_hi, mean_lo, rstd)
        probe.take<float>(split_cap);         // split-K partial tiles
        need = probe.off;
    }
    if ((rc = dm.work.reserve(need))) return rc;
    Carve cv{(char *)dm.work.ptr};
    int32_t *d_ints = cv.take<int32_t>(n_ints);
    uint8_t *d_mask = cv.take<uint8_t>(BK);
    float *h = cv.take<float>(T * d), *nb = cv.take<float>(T * d), *qkv = cv.take<float>(T * 3 * d);
    float *ctx = cv.take<float>(T * d), *gated = cv.take<float>(T * big);
    float *states = cv.take<float>(BK * d * 3);
    float *s_norm = states + BK * d, *s_hid = states + 2 * BK * d;
    float *raw = cv.take<float>(BK * 3);
    float *d_logits = raw + BK, *d_probs = raw + 2 * BK;
    float *d_feat = cv.take<float>(B * 4), *d_pooled = cv.take<float>(B * d);
    float *act_in = cv.take<float>(B * ld_act), *act_hid = cv.take<float>(B * 256);
    float *d_act = cv.take<float>(B * nact);
    float4 *hstats = cv.take<float4>(T * (d / 64));
    float4 *hrow = cv.take<float4>(T);
    float *partials = cv.take<float>(split_cap);
    const int32_t *d_ids = d_ints + o_ids, *d_pos = d_ints + o_pos, *d_rowseq = d_ints + o_rs;
    const int32_t *d_start = d_ints + o_start, *d_valid = d_ints + o_valid, *d_qtype = d_ints + o_q;
    const int32_t *d_mrow = d_ints + o_mrow;

    TRY_HIP(hipMemcpyAsync(d_ints, ints.data(), n_ints * 4, hipMemcpyHostToDevice, stream), "upload inputs");
    TRY_HIP(hipMemcpyAsync(d_mask, mask.data(), BK, hipMemcpyHostToDevice, stream), "upload inputs");

    // Trace: the stage buffer, unpacked to [B][L][width] with zero padded rows.
    std::vector<float> host_rows, host_full;
    auto record_rows = [&](const char *name, const float *buf, uint64_t width) -> int {
        if (!trace) return RAYA_OK;
        TRY_HIP(hipStreamSynchronize(stream), "trace sync");
        host_rows.resize(T * width);
        TRY_HIP(hipMemcpy(host_rows.data(), buf, T * width * 4, hipMemcpyDeviceToHost), "trace copy");
        host_full.assign(B * L * width, 0.0f);
        for (uint64_t b = 0; b < B; ++b)
            memcpy(host_full.data() + b * L * width, host_rows.data() + (uint64_t)ints[o_start + b] * width,
                   in->valid_len[b] * width * 4);
        const uint64_t shape[3] = {B, L, width};
        trace(user, name, shape, 3, host_full.data());
        return RAYA_OK;
    };
    auto record_dense = [&](const char *name, const float *buf, std::vector<uint64_t> shape) -> int {
        if (!trace) return RAYA_OK;
        TRY_HIP(hipStreamSynchronize(stream), "trace sync");
        uint64_t n = 1;
        for (uint64_t s : shape) n *= s;
        host_rows.resize(n);
        TRY_HIP(hipMemcpy(host_rows.data(), buf, n * 4, hipMemcpyDeviceToHost), "trace copy");
        trace(user, name, shape.data(), (uint32_t)shape.size(), host_rows.data());
        return RAYA_OK;
    };
#define RECORD(expr)        \
    do {                    \
        int r_ = (expr);    \
        if (r_) return r_;  \
    } while (0)

    // Stage timing: an event pair on the stream around each span whose level is
    // at most the model's profiling level; read back after the final sync.
    struct Span {
        std::string name;
        hipEvent_t e0 = nullptr, e1 = nullptr;
    };
    struct Spans {
        std::vector<Span> v;
        ~Spans() {
            for (auto &s : v) {
                if (s.e0) (void)hipEventDestroy(s.e0);
                if (s.e1) (void)hipEventDestroy(s.e1);
            }
        }
    } spans;
    const int profile = m.profile;
    m.stages.clear();
    auto span_begin = [&](int level, const std::string &nm, int *idx) -> int {
        *idx = -1;
        if (profile < level) return RAYA_OK;
        Span sp;
        sp.name = nm;
        TRY_HIP(hipEventCreate(&sp.e0), "stage event");
        spans.v.push_back(sp);
        TRY_HIP(hipEventCreate(&spans.v.back().e1), "stage event");
        TRY_HIP(hipEventRecord(spans.v.back().e0, stream), "stage event");
        *idx = (int)spans.v.size() - 1;
        return RAYA_OK;
    };
    auto span_end = [&](int idx) -> int {
        if (idx < 0) return RAYA_OK;
        TRY_HIP(hipEventRecord(spans.v[idx].e1, stream), "stage event");
        return RAYA_OK;
    };
    int sp_stage = -1, sp_op = -1;
#define SPAN(level, nm, slot) RECORD(span_begin(level, nm, &slot))
#define SPAN_END(slot) RECORD(span_end(slot))

    auto P = [&](const std::string &name) { return param(m, dm, name); };
    // Split-K for a ring-kernel launch whose tiles leave compute units idle, when its
    // partials fit the carved space (the launches run in order on one stream and share it).
    auto set_split = [&](GemmLaunch &g) {
        const bool ring = g.k % 16 == 0 && g.lda % 4 == 0 && g.ldb % 4 == 0 && ((uintptr_t)g.a & 15) == 0 &&
                          ((uintptr_t)g.b & 15) == 0;
        const int sp = ring ? gemm_splits(g.m, g.n, g.k, g.act) : 1;
        if (sp > 1 && gemm_split_floats(g.m, g.n, g.act, sp) <= split_cap) {
            g.splits = sp;
            g.partials = partials;
        }
    };
    auto gemm = [&](float *o, int64_t ldo, const float *a, int64_t lda, const float *wt, uint64_t rows, uint64_t n,
                    uint64_t k, int act, const float *bias, const float *res) -> int {
        GemmLaunch g{};
        g.out = o;
        g.ldo = ldo;
        g.a = a;
        g.lda = lda;
        g.b = wt;
        g.ldb = (int64_t)k;
        g.m = (int32_t)rows;
        g.n = (int32_t)n;
        g.k = (int32_t)k;
        g.n_rows_b = (int32_t)(act == RAYA_EPI_GEGLU ? 2 * n : n);
        g.act = act;
        g.bias = bias;
        g.residual = res;
        g.ldr = ldo;
        set_split(g);
        TRY_HIP(launch_gemm(g, stream), "gemm");
        return RAYA_OK;
    };
    // The residual GEMMs of an encoder layer: h += a W^T, and with fused norms also the
    // LayerNorm chunk statistics of the new h for the next GEMM.
    auto gemm_residual = [&](const float *a, uint64_t k, const float *wt, bool stats) -> int {
        GemmLaunch g{};
        g.out = h;
        g.ldo = (int64_t)d;
        g.a = a;
        g.lda = (int64_t)k;
        g.b = wt;
        g.ldb = (int64_t)k;
        g.m = (int32_t)T;
        g.n = (int32_t)d;
        g.k = (int32_t)k;
        g.n_rows_b = (int32_t)d;
        g.act = RAYA_EPI_NONE;
        g.residual = h;
        g.ldr = (int64_t)d;
        g.out_stats = stats ? hstats : nullptr;
        set_split(g);
        TRY_HIP(launch_gemm(g, stream), "residual gemm");
        if (stats)
            TRY_HIP(launch_ln_stats(hstats, (int)T, (int)(d / 64), (float)c.norm_eps, hrow, stream), "ln stats");
        return RAYA_OK;
    };
    const float *folded = (const float *)dm.folded.buf.ptr;
    auto layer_norm = [&](const float *x, const int32_t *gather, const float *wt, const float *bias, float eps,
                          uint64_t rows, float *o, const float *add, float *o_add) -> int {
        LayerNormLaunch l{};
        l.x = x;
        l.ldx = (int64_t)d;
        l.gather = gather;
        l.w = wt;
        l.b = bias;
        l.eps = eps;
        l.rows = (int32_t)rows;
        l.d = (int32_t)d;
        l.out = o;
        l.ldo = (int64_t)d;
        l.add = add;
        l.row_seq = d_rowseq;
        l.seq_index = d_qtype;
        l.out_add = o_add;
        TRY_HIP(launch_layer_norm(l, stream), "layer_norm");
        return RAYA_OK;
    };
    // Attention over the packed [T][3d] projection, context written to [T][d].
    auto attend = [&](const float *q3, uint64_t heads, uint64_t head_dim, int32_t kind, uint64_t arg) -> int {
        AttnLaunch a{};
        a.q = q3;
        a.k = q3 + d;
        a.v = q3 + 2 * d;
        a.out = ctx;
        a.valid_len = d_valid;
        a.q_rs = a.k_rs = a.v_rs = (int64_t)(3 * d);
        a.q_hs = a.k_hs = a.v_hs = a.o_hs = (int64_t)head_dim;
        a.o_rs = (int64_t)d;
        a.batch = (int32_t)B;
        a.heads = (int32_t)heads;
        a.seq = (int32_t)Lmax;
        a.head_dim = (int32_t)head_dim;
        a.mask_kind = kind;
        a.mask_arg = (kind == RAYA_MASK_SLIDING || kind == RAYA_MASK_BLOCKDIAG)
                         ? (int32_t)std::min<uint64_t>(arg, std::max<uint64_t>(Lmax, 1))
                         : 0;
        a.scale = 1.0f / sqrtf((float)head_dim);  // AttnParams::new, attention.rs:98-105
        a.seq_start = d_start;
        TRY_HIP(launch_attention(a, stream), "attention");
        return RAYA_OK;
    };

    const float eps = (float)c.norm_eps, head_eps = 1e-5f;  // head.rs:8
    const size_t half = hd / 2, rope_one = (size_t)dm.rope_len * half;
    const float *rope_t = (const float *)dm.rope.ptr;

    // encoder::embed (encoder.rs:15-32)
    SPAN(1, "embedding", sp_stage);
    RECORD(layer_norm(P("encoder.embeddings.tok_embeddings.weight"), d_ids, P("encoder.embeddings.norm.weight"),
                      nullptr, eps, T, h, nullptr, nullptr));
    SPAN_END(sp_stage);
    RECORD(record_rows("embedding_output", h, d));
    char name[64];
    for (uint64_t i = 0; i < c.layers; ++i) {
        const std::string p = "encoder.layers." + std::to_string(i);
        snprintf(name, sizeof name, "encoder_layer_%02d", (int)i);
        const std::string sn = name;
        SPAN(1, sn, sp_stage);
        const float *x = h;
        if (i > 0 && !fused) {
            SPAN(2, sn + "/attn_norm", sp_op);
            RECORD(layer_norm(h, nullptr, P(p + ".attn_norm.weight"), nullptr, eps, T, nb, nullptr, nullptr));
            SPAN_END(sp_op);
            x = nb;
        }
        SPAN(2, sn + "/qkv", sp_op);
        const bool global = c.is_global(i);
        const float *cos_t = rope_t + (global ? 0 : 2) * rope_one, *sin_t = cos_t + rope_one;
        {
            // attn_norm (layers >= 1) folded in when fused: h's statistics from the last
            // layer's MLP residual GEMM.
            const bool norm_in = fused && i > 0;
            GemmLaunch g{};
            g.out = qkv;
            g.ldo = (int64_t)(3 * d);
            g.a = x;
            g.lda = (int64_t)d;
            g.b = norm_in ? folded + dm.folded.qkv[i] : P(p + ".attn.Wqkv.weight");
            g.ldb = (int64_t)d;
            g.m = (int32_t)T;
            g.n = (int32_t)(3 * d);
            g.k = (int32_t)d;
            g.n_rows_b = g.n;
            g.act = RAYA_EPI_NONE;
            if (norm_in) {
                g.in_stats = hrow;
                g.colsum = folded + dm.folded.qkv_sum[i];
            }
            if (hd == (uint64_t)kRopeHeadDim) {
                g.rope_cos = cos_t;
                g.rope_sin = sin_t;
                g.positions = d_pos;
                g.rope_cols = (int32_t)(2 * d);
            }
            set_split(g);
            TRY_HIP(launch_gemm(g, stream), "qkv gemm");
            if (hd != (uint64_t)kRopeHeadDim)
                TRY_HIP(launch_rope(qkv, (int64_t)(3 * d), d_pos, cos_t, sin_t, (int)T, (int)d, (int)hd, stream),
                        "rope");
        }
        SPAN_END(sp_op);
        SPAN(2, sn + "/attention", sp_op);
        if (global) RECORD(attend(qkv, c.heads, hd, RAYA_MASK_FULL, 0));
        else RECORD(attend(qkv, c.heads, hd, local_kind, local_arg));
        SPAN_END(sp_op);
        SPAN(2, sn + "/attn_out", sp_op);
        RECORD(gemm_residual(ctx, d, P(p + ".attn.Wo.weight"), fused));
        SPAN_END(sp_op);
        if (!fused) {
            SPAN(2, sn + "/mlp_norm", sp_op);
            RECORD(layer_norm(h, nullptr, P(p + ".mlp_norm.weight"), nullptr, eps, T, nb, nullptr, nullptr));
            SPAN_END(sp_op);
        }
        SPAN(2, sn + "/mlp_in_geglu", sp_op);
        if (fused) {  // mlp_norm folded in: h's statistics from the attention residual GEMM
            GemmLaunch g{};
            g.out = gated;
            g.ldo = (int64_t)inter;
            g.a = h;
            g.lda = (int64_t)d;
            g.b = folded + dm.folded.wi[i];
            g.ldb = (int64_t)d;
            g.m = (int32_t)T;
            g.n = (int32_t)inter;
            g.k = (int32_t)d;
            g.n_rows_b = (int32_t)(2 * inter);
            g.act = RAYA_EPI_GEGLU;
            g.in_stats = hrow;
            g.colsum = folded + dm.folded.wi_sum[i];
            set_split(g);
            TRY_HIP(launch_gemm(g, stream), "mlp in gemm");
        } else {
            RECORD(gemm(gated, inter, nb, d, P(p + ".mlp.Wi.weight"), T, inter, d, RAYA_EPI_GEGLU, nullptr, nullptr));
        }
        SPAN_END(sp_op);
        SPAN(2, sn + "/mlp_out", sp_op);
        // the last layer's h goes to the final norm, a kernel of its own
        RECORD(gemm_residual(gated, inter, P(p + ".mlp.Wo.weight"), fused && i + 1 < c.layers));
        SPAN_END(sp_op);
        SPAN_END(sp_stage);
        RECORD(record_rows(sn.c_str(), h, d));
    }
    // final norm, then + type_emb[qtype] (model.rs:283-304); nb holds the normed rows
    SPAN(1, "final_norm", sp_stage);
    RECORD(layer_norm(h, nullptr, P("encoder.final_norm.weight"), nullptr, eps, T, trace ? nb : nullptr,
                      P("type_emb.weight"), h));
    SPAN_END(sp_stage);
    if (trace) {
        RECORD(record_rows("encoder_final_norm", nb, d));
        RECORD(record_rows("encoder_output", nb, d));
        const float *rows3 = m.w.host.data() + m.w.entries[m.w.index.at("type_emb.weight")].offset;
        std::vector<float> temb(B * d);
        for (uint64_t b = 0; b < B; ++b) memcpy(temb.data() + b * d, rows3 + in->qtype[b] * d, d * 4);
        const uint64_t shape[3] = {B, 1, d};
        trace(user, "type_emb_add", shape, 3, temb.data());
        RECORD(record_rows("head_input", h, d));
    }
    // head layers: nn.TransformerEncoderLayer(norm_first=True) (head.rs:14-48)
    for (uint64_t i = 0; i < c.head_layers; ++i) {
        const std::string p = "head.layers." + std::to_string(i);
        snprintf(name, sizeof name, "head_layer_%02d", (int)i);
        SPAN(1, name, sp_stage);
        RECORD(layer_norm(h, nullptr, P(p + ".norm1.weight"), P(p + ".norm1.bias"), head_eps, T, nb, nullptr, nullptr));
        RECORD(gemm(qkv, 3 * d, nb, d, P(p + ".self_attn.in_proj_weight"), T, 3 * d, d, RAYA_EPI_NONE,
                    P(p + ".self_attn.in_proj_bias"), nullptr));
        RECORD(attend(qkv, hh, hhd, RAYA_MASK_FULL, 0));
        RECORD(gemm(h, d, ctx, d, P(p + ".self_attn.out_proj.weight"), T, d, d, RAYA_EPI_NONE,
                    P(p + ".self_attn.out_proj.bias"), h));
        RECORD(layer_norm(h, nullptr, P(p + ".norm2.weight"), P(p + ".norm2.bias"), head_eps, T, nb, nullptr, nullptr));
        RECORD(gemm(gated, c.head_ffn, nb, d, P(p + ".linear1.weight"), T, c.head_ffn, d, RAYA_EPI_RELU,
                    P(p + ".linear1.bias"), nullptr));
        RECORD(gemm(h, d, gated, c.head_ffn, P(p + ".linear2.weight"), T, d, c.head_ffn, RAYA_EPI_NONE,
                    P(p + ".linear2.bias"), h));
        SPAN_END(sp_stage);
        RECORD(record_rows(name, h, d));
    }
    // marker scorer (head.rs:50-67), then the per-sequence tail
    SPAN(1, "scorer_and_act_head", sp_stage);
    TRY_HIP(launch_gather_rows(h, (int64_t)d, d_mrow, (int)BK, (int)d, states, stream), "gather markers");
    RECORD(record_dense("marker_states", states, {B, K, d}));
    {
        LayerNormLaunch l{};
        l.x = states;
        l.ldx = (int64_t)d;
        l.w = P("scorer.0.weight");
        l.b = P("scorer.0.bias");
        l.eps = head_eps;
        l.rows = (int32_t)BK;
        l.d = (int32_t)d;
        l.out = s_norm;
        l.ldo = (int64_t)d;
        TRY_HIP(launch_layer_norm(l, stream), "scorer norm");
    }
    RECORD(gemm(s_hid, d, s_norm, d, P("scorer.1.weight"), BK, d, d, RAYA_EPI_GELU, P("scorer.1.bias"), nullptr));
    RECORD(gemm(raw, 1, s_hid, d, P("scorer.3.weight"), BK, 1, d, RAYA_EPI_NONE, P("scorer.3.bias"), nullptr));
    TRY_HIP(launch_head_finish(raw, d_mask, (int)B, (int)K, h, (int64_t)d, d_start, (int)d, d_logits, d_probs, d_feat,
                               d_pooled, act_in, (int)ld_act, stream),
            "head finish");
    RECORD(record_dense("logits", d_logits, {B, K}));
    RECORD(record_dense("probabilities", d_probs, {B, K}));
    RECORD(record_dense("act_features", d_feat, {B, 4}));
    RECORD(record_dense("pooled", d_pooled, {B, d}));
    RECORD(gemm(act_hid, 256, act_in, ld_act, (const float *)dm.act_w.ptr, B, 256, ld_act, RAYA_EPI_GELU,
                P("act_head.0.bias"), nullptr));
    RECORD(gemm(d_act, nact, act_hid, 256, P("act_head.2.weight"), B, nact, 256, RAYA_EPI_NONE, P("act_head.2.bias"),
                nullptr));
    SPAN_END(sp_stage);
    RECORD(record_dense("act_logits", d_act, {B, nact}));

    const std::pair<float *, const float *> outs[] = {{out->logits, d_logits},
                                                      {out->probabilities, d_probs},
                                                      {out->act_logits, d_act},
                                                      {out->features, d_feat},
                                                      {out->pooled, d_pooled}};
    const uint64_t sizes[] = {BK, BK, B * nact, B * 4, B * d};
    for (int i = 0; i < 5; ++i)
        if (outs[i].first)
            TRY_HIP(hipMemcpyAsync(outs[i].first, outs[i].second, sizes[i] * 4, hipMemcpyDeviceToHost, stream),
                    "download outputs");
    TRY_HIP(hipStreamSynchronize(stream), "forward");
    for (const auto &sp : spans.v) {
        float ms = 0.f;
        TRY_HIP(hipEventElapsedTime(&ms, sp.e0, sp.e1), "stage time");
        m.stages.emplace_back(sp.name, (double)ms);
    }
#undef SPAN
#undef SPAN_END
#undef RECORD
    return ok();
}

}  // extern "C"
