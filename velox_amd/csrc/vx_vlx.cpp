// vx_vlx.cpp -- reads a .vlx model source into the decode backend's model configuration.
//
// The reference compiles a .vlx file (src/cli.rs:1214-1388: lex, parse, sema, IR, optimizer,
// memory planner, codegen) into an emitted runner whose compile-time constants (src/codegen.rs:936-
// 1102) size every kernel. This backend's kernels are generic over the model, so the part of that
// pipeline the decode step needs is what the file declares about the model:
//   * the `target hardware { ... }` block: device, vram_capacity (a constant expression over
//     KiB/MiB/GiB/TiB/KB/MB/GB/TB, as src/parser.rs:497-525 evaluates it) and safety_factor
//     (default 0.95, src/ast.rs:78), giving the planner's budget floor(vram * safety_factor) minus
//     the driver reserve of src/memory_planner.rs:478-488;
//   * the `model Name< const X: usize = N, ... >` header: VOCAB, HIDDEN_DIM, INTERMEDIATE_DIM,
//     NUM_LAYERS, NUM_HEADS, NUM_KV_HEADS, HEAD_DIM, S_MAX, B_MAX, and ROPE_THETA where given;
//   * the weight declarations: q/k/v biases (`b_q`, `b_k`, `b_v`) and an LM head (`w_head` or
//     `w_lm_head`, src/codegen.rs:1063; without one the head is tied to the embedding);
//   * the first weight binding's file, `safetensors("file", "key")`, which the CLI hands the runner
//     as its --weights (src/cli.rs:1400-1414).
// The RMSNorm epsilon follows the model's name as the reference's lowering sets it
// (src/ir.rs:549-553: Qwen/K2/Horizon 1e-6, else 1e-5), whatever `eps =` the source writes; theta
// is ROPE_THETA or, where the file does not say, the name rule of src/codegen.rs:962-975 (llama
// 5e5, qwen 1e6, else 1e4).
// MLA models (LATENT_KV_DIM, src examples/deepseek_v3_mla.vlx) map to the MLA layer's
// configuration instead.
#include <cctype>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "vx_common.h"

namespace {

struct VxTok {
    enum Kind { Ident, Number, String, Punct, End } kind = End;
    std::string text;
    double num = 0.0;
    bool integral = false;
};

// Comments dropped; identifiers, numbers (decimal, 0x hex, 0b binary, floats with an exponent,
// `_` digit separators), "strings" and single-character punctuation.
bool vx_lex(const std::string& s, std::vector<VxTok>& out) {
    size_t i = 0;
    const size_t n = s.size();
    while (i < n) {
        const char c = s[i];
        if (std::isspace((unsigned char)c)) { ++i; continue; }
        if (c == '/' && i + 1 < n && s[i + 1] == '/') {
            while (i < n && s[i] != '\n') ++i;
            continue;
        }
        if (c == '/' && i + 1 < n && s[i + 1] == '*') {
            const size_t e = s.find("*/", i + 2);
            if (e == std::string::npos) return false;
            i = e + 2;
            continue;
        }
        VxTok t;
        if (std::isalpha((unsigned char)c) || c == '_') {
            size_t j = i;
            while (j < n && (std::isalnum((unsigned char)s[j]) || s[j] == '_')) ++j;
            t.kind = VxTok::Ident;
            t.text = s.substr(i, j - i);
            i = j;
        } else if (std::isdigit((unsigned char)c)) {
            size_t j = i;
            std::string digits;
            if (c == '0' && i + 1 < n && (s[i + 1] == 'x' || s[i + 1] == 'X' || s[i + 1] == 'b' || s[i + 1] == 'B')) {
                const int base = (s[i + 1] == 'x' || s[i + 1] == 'X') ? 16 : 2;
                j = i + 2;
                while (j < n && (std::isxdigit((unsigned char)s[j]) || s[j] == '_')) {
                    if (s[j] != '_') digits += s[j];
                    ++j;
                }
                if (digits.empty()) return false;
                t.num = (double)std::strtoull(digits.c_str(), nullptr, base);
                t.integral = true;
            } else {
                bool fl = false;
                while (j < n) {
                    const char d = s[j];
                    if (std::isdigit((unsigned char)d) || d == '_') {
                        if (d != '_') digits += d;
                        ++j;
                    } else if (d == '.' && j + 1 < n && std::isdigit((unsigned char)s[j + 1])) {
                        fl = true;
                        digits += d;
                        ++j;
                    } else if ((d == 'e' || d == 'E') && j + 1 < n &&
                               (std::isdigit((unsigned char)s[j + 1]) ||
                                ((s[j + 1] == '-' || s[j + 1] == '+') && j + 2 < n &&
                                 std::isdigit((unsigned char)s[j + 2])))) {
                        fl = true;
                        digits += d;
                        digits += s[j + 1];
                        j += 2;
                    } else {
                        break;
                    }
                }
                t.num = std::strtod(digits.c_str(), nullptr);
                t.integral = !fl;
            }
            t.kind = VxTok::Number;
            t.text = s.substr(i, j - i);
            i = j;
        } else if (c == '"') {
            const size_t e = s.find('"', i + 1);
            if (e == std::string::npos) return false;
            t.kind = VxTok::String;
            t.text = s.substr(i + 1, e - i - 1);
            i = e + 1;
        } else {
            t.kind = VxTok::Punct;
            t.text = std::string(1, c);
            ++i;
        }
        out.push_back(t);
    }
    out.push_back(VxTok());
    return true;
}

struct VxParser {
    const std::vector<VxTok>& t;
    size_t p = 0;
    bool ok = true;
    explicit VxParser(const std::vector<VxTok>& toks) : t(toks) {}
    const VxTok& peek(size_t k = 0) const { return t[p + k < t.size() ? p + k : t.size() - 1]; }
    bool is(const char* s, size_t k = 0) const {
        const VxTok& x = peek(k);
        return (x.kind == VxTok::Punct || x.kind == VxTok::Ident) && x.text == s;
    }
    bool eat(const char* s) {
        if (is(s)) { ++p; return true; }
        ok = false;
        return false;
    }
    // Constant expression: + - over * / over primaries (numbers, size units, parentheses),
    // evaluated in double and truncated to an integer where the reference's const evaluator is
    // integral (src/parser.rs:497-525).
    double primary() {
        const VxTok& x = peek();
        if (x.kind == VxTok::Number) { ++p; return x.num; }
        if (x.kind == VxTok::Ident) {
            ++p;
            static const std::map<std::string, double> units = {
                {"KiB", 1024.0}, {"MiB", 1048576.0}, {"GiB", 1073741824.0}, {"TiB", 1099511627776.0},
                {"KB", 1e3}, {"MB", 1e6}, {"GB", 1e9}, {"TB", 1e12}};
            const auto it = units.find(x.text);
            if (it == units.end()) { ok = false; return 0.0; }
            return it->second;
        }
        if (is("(")) {
            ++p;
            const double v = expr();
            eat(")");
            return v;
        }
        ok = false;
        return 0.0;
    }
    double term() {
        double v = primary();
        while (ok && (is("*") || is("/"))) {
            const bool mul = is("*");
            ++p;
            const double r = primary();
            v = mul ? v * r : (r != 0.0 ? v / r : 0.0);
        }
        return v;
    }
    double expr() {
        double v = term();
        while (ok && (is("+") || is("-"))) {
            const bool add = is("+");
            ++p;
            const double r = term();
            v = add ? v + r : v - r;
        }
        return v;
    }
};

struct VxVlx {
    std::string device, model;
    double vram = 0.0, safety = 0.95;
    bool has_target = false;
    std::map<std::string, double> consts;
    std::vector<std::string> weights;
    std::string weights_file;  // the first `safetensors("file", "key")` binding's file
};

bool vx_parse(const std::string& src, VxVlx& v) {
    std::vector<VxTok> toks;
    if (!vx_lex(src, toks)) return false;
    VxParser P(toks);
    while (P.peek().kind != VxTok::End && P.ok) {
        if (P.is("target") && P.is("hardware", 1)) {
            P.p += 2;
            if (!P.eat("{")) return false;
            v.has_target = true;
            while (P.ok && !P.is("}") && P.peek().kind != VxTok::End) {
                const VxTok key = P.peek();
                if (key.kind != VxTok::Ident) return false;
                ++P.p;
                if (!P.eat(":")) return false;
                if (key.text == "device") {
                    if (P.peek().kind != VxTok::String) return false;
                    v.device = P.peek().text;
                    ++P.p;
                } else if (key.text == "vram_capacity") {
                    v.vram = std::floor(P.expr());
                } else if (key.text == "safety_factor") {
                    v.safety = P.expr();
                } else {
                    P.expr();  // compute_capability and others: parsed, unused here
                }
                if (!P.eat(";")) return false;
            }
            if (!P.eat("}")) return false;
        } else if (P.is("model") && P.peek(1).kind == VxTok::Ident && P.is("<", 2)) {
            v.model = P.peek(1).text;
            P.p += 3;
            while (P.ok && !P.is(">")) {
                if (!P.eat("const")) return false;
                const VxTok name = P.peek();
                if (name.kind != VxTok::Ident) return false;
                ++P.p;
                if (!P.eat(":")) return false;
                if (P.peek().kind != VxTok::Ident) return false;  // the type (usize)
                ++P.p;
                if (!P.eat("=")) return false;
                const double val = P.expr();
                if (!P.ok) return false;
                v.consts[name.text] = val;
                if (P.is(",")) ++P.p;
            }
            if (!P.eat(">")) return false;
        } else if (P.is("weight") && P.peek(1).kind == VxTok::Ident) {
            v.weights.push_back(P.peek(1).text);
            P.p += 2;
        } else if (P.is("safetensors") && P.is("(", 1) && P.peek(2).kind == VxTok::String) {
            // a weight binding (src/ast.rs:1084); the CLI runs the model on the first one's file
            // (src/cli.rs:1400-1414)
            if (v.weights_file.empty()) v.weights_file = P.peek(2).text;
            P.p += 3;
        } else {
            ++P.p;
        }
    }
    return P.ok && !v.model.empty();
}

bool vx_read_file(const char* path, std::string& out) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return false;
    char buf[65536];
    size_t n;
    while ((n = std::fread(buf, 1, sizeof(buf), f)) > 0) out.append(buf, n);
    const bool ok = !std::ferror(f);
    std::fclose(f);
    return ok;
}

bool vx_contains_ci(const std::string& s, const char* sub) {
    std::string a = s, b = sub;
    for (char& c : a) c = (char)std::tolower((unsigned char)c);
    for (char& c : b) c = (char)std::tolower((unsigned char)c);
    return a.find(b) != std::string::npos;
}

bool vx_has_weight(const VxVlx& v, const char* a, const char* b = nullptr) {
    for (const std::string& w : v.weights)
        if (w == a || (b && w == b)) return true;
    return false;
}

// src/memory_planner.rs:478-488
uint64_t vx_system_reserve(uint64_t vram) {
    const uint64_t gib = 1024ull * 1024ull * 1024ull;
    if (vram >= 24 * gib) return 512ull * 1024ull * 1024ull;
    if (vram >= 2 * gib) return 256ull * 1024ull * 1024ull;
    return vram / 32;
}

// A header constant as a 32-bit count: `dflt` when absent, false when negative, fractional or
// beyond 2^32 - 1 (a malformed source).
bool vx_const_u32(const VxVlx& v, const char* k, uint32_t dflt, uint32_t* out) {
    const auto it = v.consts.find(k);
    if (it == v.consts.end()) { *out = dflt; return true; }
    const double x = it->second;
    if (!(x >= 0.0 && x <= 4294967295.0) || x != std::floor(x)) return false;
    *out = (uint32_t)x;
    return true;
}

bool vx_fill_target(const VxVlx& v, VeloxHipVlxTarget* t) {
    uint32_t b_max, s_max;
    if (!vx_const_u32(v, "B_MAX", 0, &b_max) || !vx_const_u32(v, "S_MAX", 0, &s_max)) return false;
    if (!(v.vram >= 0.0 && v.vram < 1.8e19) || !(v.safety >= 0.0 && v.safety <= 1.0e3)) return false;
    if (!t) return true;
    std::memset(t, 0, sizeof(*t));
    std::snprintf(t->device, sizeof(t->device), "%s", v.device.c_str());
    t->vram_capacity_bytes = (uint64_t)v.vram;
    t->safety_factor = v.safety;
    t->system_reserve_bytes = vx_system_reserve(t->vram_capacity_bytes);
    t->safe_budget_bytes = (uint64_t)std::floor((double)t->vram_capacity_bytes * v.safety);
    t->b_max = b_max;
    t->s_max = s_max;
    std::snprintf(t->weights_file, sizeof(t->weights_file), "%s", v.weights_file.c_str());
    return true;
}

// The planner's budget for this backend's own regions: the safe budget less the driver reserve
// (the reference counts the reserve inside its total, src/memory_planner.rs:372-386).
uint64_t vx_budget(const VxVlx& v) {
    if (!v.has_target || v.vram <= 0.0) return 0;  // no target block: the default 288 GB
    const uint64_t vram = (uint64_t)v.vram, safe = (uint64_t)std::floor((double)vram * v.safety);
    const uint64_t res = vx_system_reserve(vram);
    return safe > res ? safe - res : 1;
}

int vx_config_from(const VxVlx& v, uint32_t max_seq_len, VeloxHipModelConfig* out, VeloxHipVlxTarget* target) {
    bool in_range = true;
    auto get = [&](const char* k, uint32_t dflt) -> uint32_t {
        uint32_t x = 0;
        if (!vx_const_u32(v, k, dflt, &x)) in_range = false;
        return x;
    };
    if (v.consts.count("LATENT_KV_DIM")) return VELOX_HIP_EINVAL;  // an MLA model: velox_hip_vlx_mla_config
    VeloxHipModelConfig c;
    std::memset(&c, 0, sizeof(c));
    std::snprintf(c.name, sizeof(c.name), "%s", v.model.c_str());
    c.vocab_size = get("VOCAB", 0);
    c.hidden_dim = get("HIDDEN_DIM", 0);
    c.intermediate_dim = get("INTERMEDIATE_DIM", 0);
    c.num_layers = get("NUM_LAYERS", 0);
    c.num_heads = get("NUM_HEADS", 0);
    c.num_kv_heads = get("NUM_KV_HEADS", c.num_heads);
    c.head_dim = get("HEAD_DIM", c.num_heads ? c.hidden_dim / c.num_heads : 0);
    c.max_seq_len = max_seq_len ? max_seq_len : get("S_MAX", 2048);  // src/codegen.rs:955 default
    if (!in_range || !c.vocab_size || !c.hidden_dim || !c.intermediate_dim || !c.num_layers || !c.num_heads || !c.head_dim)
        return VELOX_HIP_EINVAL;
    const auto th = v.consts.find("ROPE_THETA");
    if (th != v.consts.end()) c.rope_theta = (float)th->second;
    else c.rope_theta = vx_contains_ci(v.model, "llama") ? 500000.0f : vx_contains_ci(v.model, "qwen") ? 1000000.0f
                                                                                                     : 10000.0f;
    // epsilon by the model's name, as the reference lowers every rmsnorm (src/ir.rs:549-553): an
    // `eps =` argument in the source does not reach its emitted kernels either
    c.rms_norm_eps = (v.model.find("Qwen") != std::string::npos || v.model.find("K2") != std::string::npos ||
                      v.model.find("Horizon") != std::string::npos) ? 1e-6f : 1e-5f;
    c.qkv_bias = vx_has_weight(v, "b_q") && vx_has_weight(v, "b_k") && vx_has_weight(v, "b_v") ? 1u : 0u;
    c.tied_lm_head = vx_has_weight(v, "w_head", "w_lm_head") ? 0u : 1u;
    c.quant_mode = VELOX_QUANT_GGML_Q4_0;
    c.vram_budget_bytes = vx_budget(v);
    if (!vx_fill_target(v, target)) return VELOX_HIP_EINVAL;
    *out = c;
    return VELOX_HIP_OK;
}

// Builtin benchmark configurations, declared in the DSL and read like any .vlx file. Their target
// is one MI355X: 288 GB of HBM3E, the whole of it usable.
const char* const kBuiltinVlx[][2] = {
    {"smollm_135m",
     "target hardware { device: \"amd_mi355x\"; vram_capacity: 288 * GB; safety_factor: 1.0; }\n"
     "model SmolLM_135M<const B_MAX: usize = 1, const S_MAX: usize = 2048, const VOCAB: usize = 49152,\n"
     "  const HIDDEN_DIM: usize = 576, const INTERMEDIATE_DIM: usize = 1536, const NUM_LAYERS: usize = 30,\n"
     "  const NUM_HEADS: usize = 9, const NUM_KV_HEADS: usize = 3, const HEAD_DIM: usize = 64> {\n"
     "  @vram_immutable weight w_embed: Tensor<[VOCAB, HIDDEN_DIM], f32>;\n"
     "  scope decode<const B: usize>(t: Tensor<[B, 1], u32>) { let x = rmsnorm(h, w_norm, eps = 1e-5); }\n}\n"},
    {"llama3_8b",
     "target hardware { device: \"amd_mi355x\"; vram_capacity: 288 * GB; safety_factor: 1.0; }\n"
     "model Llama3_8B<const B_MAX: usize = 1, const S_MAX: usize = 8192, const VOCAB: usize = 128256,\n"
     "  const HIDDEN_DIM: usize = 4096, const INTERMEDIATE_DIM: usize = 14336, const NUM_LAYERS: usize = 32,\n"
     "  const NUM_HEADS: usize = 32, const NUM_KV_HEADS: usize = 8, const HEAD_DIM: usize = 128> {\n"
     "  @vram_immutable weight w_embed: Tensor<[VOCAB, HIDDEN_DIM], q4_0>;\n"
     "  @vram_immutable weight w_lm_head: Tensor<[HIDDEN_DIM, VOCAB], q4_0>;\n"
     "  scope decode<const B: usize>(t: Tensor<[B, 1], u32>) { let x = rmsnorm(h, w_norm, eps = 1e-5); }\n}\n"},
    {"qwen2_5_7b",
     "target hardware { device: \"amd_mi355x\"; vram_capacity: 288 * GB; safety_factor: 1.0; }\n"
     "model Qwen2_5_7B<const B_MAX: usize = 1, const S_MAX: usize = 4096, const VOCAB: usize = 152064,\n"
     "  const HIDDEN_DIM: usize = 3584, const INTERMEDIATE_DIM: usize = 18944, const NUM_LAYERS: usize = 28,\n"
     "  const NUM_HEADS: usize = 28, const NUM_KV_HEADS: usize = 4, const HEAD_DIM: usize = 128> {\n"
     "  @vram_immutable weight w_embed: Tensor<[VOCAB, HIDDEN_DIM], q4_0>;\n"
     "  @vram_immutable weight b_q: Tensor<[NUM_LAYERS, 3584], f32>;\n"
     "  @vram_immutable weight b_k: Tensor<[NUM_LAYERS, 512], f32>;\n"
     "  @vram_immutable weight b_v: Tensor<[NUM_LAYERS, 512], f32>;\n"
     "  scope decode<const B: usize>(t: Tensor<[B, 1], u32>) { let x = rmsnorm(h, w_norm, eps = 1e-6); }\n}\n"},
    {"qwen2_72b",
     "target hardware { device: \"amd_mi355x\"; vram_capacity: 288 * GB; safety_factor: 1.0; }\n"
     "model Qwen2_72B<const B_MAX: usize = 1, const S_MAX: usize = 8448, const VOCAB: usize = 152064,\n"
     "  const HIDDEN_DIM: usize = 8192, const INTERMEDIATE_DIM: usize = 29568, const NUM_LAYERS: usize = 80,\n"
     "  const NUM_HEADS: usize = 64, const NUM_KV_HEADS: usize = 8, const HEAD_DIM: usize = 128> {\n"
     "  @vram_immutable weight w_embed: Tensor<[VOCAB, HIDDEN_DIM], q4_0>;\n"
     "  @vram_immutable weight b_q: Tensor<[NUM_LAYERS, 8192], f32>;\n"
     "  @vram_immutable weight b_k: Tensor<[NUM_LAYERS, 1024], f32>;\n"
     "  @vram_immutable weight b_v: Tensor<[NUM_LAYERS, 1024], f32>;\n"
     "  @vram_immutable weight w_lm_head: Tensor<[HIDDEN_DIM, VOCAB], q4_0>;\n"
     "  scope decode<const B: usize>(t: Tensor<[B, 1], u32>) { let x = rmsnorm(h, w_norm, eps = 1e-6); }\n}\n"},
};

}  // namespace

extern "C" {

int velox_hip_vlx_config(const char* source, uint32_t max_seq_len, VeloxHipModelConfig* out,
                         VeloxHipVlxTarget* target) {
    if (!source || !out) return VELOX_HIP_EINVAL;
    VxVlx v;
    if (!vx_parse(source, v)) return VELOX_HIP_EINVAL;
    return vx_config_from(v, max_seq_len, out, target);
}

int velox_hip_vlx_load(const char* path, uint32_t max_seq_len, VeloxHipModelConfig* out, VeloxHipVlxTarget* target) {
    if (!path || !out) return VELOX_HIP_EINVAL;
    std::string src;
    if (!vx_read_file(path, src)) return VELOX_HIP_ENOTLOADED;
    return velox_hip_vlx_config(src.c_str(), max_seq_len, out, target);
}

int velox_hip_vlx_mla_config(const char* source, uint32_t max_seq_len, uint32_t max_batch, VeloxHipMlaConfig* out,
                             VeloxHipVlxTarget* target) {
    if (!source || !out) return VELOX_HIP_EINVAL;
    VxVlx v;
    if (!vx_parse(source, v)) return VELOX_HIP_EINVAL;
    bool in_range = true;
    auto get = [&](const char* k) -> uint32_t {
        uint32_t x = 0;
        if (!vx_const_u32(v, k, 0, &x)) in_range = false;
        return x;
    };
    if (!in_range) return VELOX_HIP_EINVAL;
    if (!get("LATENT_KV_DIM") || !get("HIDDEN_DIM") || !get("NUM_HEADS") || !get("HEAD_DIM")) return VELOX_HIP_EINVAL;
    VeloxHipMlaConfig c;
    std::memset(&c, 0, sizeof(c));
    c.hidden_dim = get("HIDDEN_DIM");
    c.num_heads = get("NUM_HEADS");
    c.q_lora_rank = get("Q_LATENT_DIM");
    c.kv_lora_rank = get("LATENT_KV_DIM");
    c.qk_nope_dim = get("HEAD_DIM");
    c.qk_rope_dim = get("ROPE_DIM");
    c.v_head_dim = get("HEAD_DIM");
    c.num_layers = get("NUM_LAYERS") ? get("NUM_LAYERS") : 1u;
    c.max_seq_len = max_seq_len ? max_seq_len : (get("S_MAX") ? get("S_MAX") : 2048u);
    const uint32_t bm = max_batch ? max_batch : (get("B_MAX") ? get("B_MAX") : 1u);
    c.max_batch = bm > 32 ? 32 : bm;
    c.kv_norm = 1;  // DeepSeek-V3's kv_a_layernorm
    c.rms_norm_eps = 1e-6f;  // DeepSeek-V3's
    c.rope_theta = get("ROPE_THETA") ? (float)get("ROPE_THETA") : 10000.0f;
    c.softmax_scale = 0.0f;  // 1/sqrt(nope + rope)
    c.vram_budget_bytes = vx_budget(v);
    if (!in_range || !vx_fill_target(v, target)) return VELOX_HIP_EINVAL;
    *out = c;
    return VELOX_HIP_OK;
}

int velox_hip_builtin_config(const char* which, uint32_t max_seq_len, VeloxHipModelConfig* out) {
    if (!which || !out) return VELOX_HIP_EINVAL;
    for (const auto& b : kBuiltinVlx) {
        if (std::strcmp(which, b[0]) != 0) continue;
        const int rc = velox_hip_vlx_config(b[1], max_seq_len, out, nullptr);
        if (rc == VELOX_HIP_OK) std::snprintf(out->name, sizeof(out->name), "%s", which);  // named by its key
        return rc;
    }
    return VELOX_HIP_EINVAL;
}

}  // extern "C"
