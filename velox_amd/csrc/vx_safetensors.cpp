// vx_safetensors.cpp -- safetensors checkpoints, the format the reference's runner and CPU engine
// load (src/runners/velox_cuda_runner.cu:60-199, src/runtime.rs:200-520): an 8-byte little-endian
// header length, a UTF-8 JSON header mapping each tensor name to {"dtype", "shape",
// "data_offsets": [begin, end]} (offsets relative to the end of the header; an optional
// "__metadata__" entry is ignored), then the tensor bytes.
//
// The file is memory-mapped (POSIX). Opening validates the container (length, header bounds, UTF-8,
// JSON); a tensor's data is checked when it is asked for, as the reference's get_tensor_f32 does:
// a missing name or data_offsets outside the file or inverted give VELOX_HIP_ETENSOR (its E013), a
// dtype other than the one asked for VELOX_HIP_EDTYPE (E014). Tensor names are the Hugging Face
// ones the reference resolves (src/runtime.rs:1273-1300), with "lm_head.weight" falling back on the
// embedding when absent (src/runtime.rs:247-259, velox_cuda_runner.cu:128-133).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "velox_hip.h"

struct VxStTensor {
    std::string name, dtype;
    std::vector<uint64_t> shape;
    uint64_t begin = 0, end = 0;
};

struct VeloxHipSafetensors {
    const uint8_t* base = nullptr;
    size_t size = 0;
    uint64_t data_start = 0;
    std::vector<VxStTensor> tensors;
    std::unordered_map<std::string, size_t> index;
};

namespace {

// Strict UTF-8 (no overlong forms, no surrogates, at most U+10FFFF).
bool vx_utf8_ok(const uint8_t* s, size_t n) {
    size_t i = 0;
    while (i < n) {
        const uint8_t c = s[i];
        if (c < 0x80) { ++i; continue; }
        uint32_t cp, len;
        if ((c & 0xE0) == 0xC0) { cp = c & 0x1F; len = 2; }
        else if ((c & 0xF0) == 0xE0) { cp = c & 0x0F; len = 3; }
        else if ((c & 0xF8) == 0xF0) { cp = c & 0x07; len = 4; }
        else return false;
        if (n - i < len) return false;
        for (uint32_t k = 1; k < len; ++k) {
            if ((s[i + k] & 0xC0) != 0x80) return false;
            cp = (cp << 6) | (s[i + k] & 0x3F);
        }
        if ((len == 2 && cp < 0x80) || (len == 3 && cp < 0x800) || (len == 4 && cp < 0x10000) || cp > 0x10FFFF ||
            (cp >= 0xD800 && cp <= 0xDFFF))
            return false;
        i += len;
    }
    return true;
}

// A small JSON reader over the header: every step checks the end, nesting is bounded.
struct VxJson {
    const char* p;
    const char* e;
    bool ok = true;

    void ws() {
        while (p < e && (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r')) ++p;
    }
    bool eat(char c) {
        ws();
        if (p < e && *p == c) { ++p; return true; }
        return false;
    }
    bool peek(char c) {
        ws();
        return p < e && *p == c;
    }
    bool fail() { ok = false; return false; }

    bool str(std::string& out) {
        out.clear();
        if (!eat('"')) return fail();
        while (p < e) {
            const char c = *p++;
            if (c == '"') return true;
            if ((unsigned char)c < 0x20) return fail();
            if (c != '\\') { out.push_back(c); continue; }
            if (p >= e) return fail();
            const char x = *p++;
            switch (x) {
                case '"': case '\\': case '/': out.push_back(x); break;
                case 'b': out.push_back('\b'); break;
                case 'f': out.push_back('\f'); break;
                case 'n': out.push_back('\n'); break;
                case 'r': out.push_back('\r'); break;
                case 't': out.push_back('\t'); break;
                case 'u': {
                    if (e - p < 4) return fail();
                    uint32_t cp = 0;
                    for (int k = 0; k < 4; ++k) {
                        const char h = *p++;
                        cp <<= 4;
                        if (h >= '0' && h <= '9') cp |= (uint32_t)(h - '0');
                        else if (h >= 'a' && h <= 'f') cp |= (uint32_t)(h - 'a' + 10);
                        else if (h >= 'A' && h <= 'F') cp |= (uint32_t)(h - 'A' + 10);
                        else return fail();
                    }
                    // names are ASCII in practice; other code points are kept as UTF-8
                    if (cp < 0x80) out.push_back((char)cp);
                    else if (cp < 0x800) { out.push_back((char)(0xC0 | (cp >> 6))); out.push_back((char)(0x80 | (cp & 0x3F))); }
                    else {
                        out.push_back((char)(0xE0 | (cp >> 12)));
                        out.push_back((char)(0x80 | ((cp >> 6) & 0x3F)));
                        out.push_back((char)(0x80 | (cp & 0x3F)));
                    }
                    break;
                }
                default: return fail();
            }
        }
        return fail();
    }

    // A non-negative integer below 2^63.
    bool u64(uint64_t& v) {
        ws();
        if (p >= e || *p < '0' || *p > '9') return fail();
        v = 0;
        while (p < e && *p >= '0' && *p <= '9') {
            const uint64_t d = (uint64_t)(*p - '0');
            if (v > ((1ull << 63) - 1 - d) / 10) return fail();
            v = v * 10 + d;
            ++p;
        }
        if (p < e && (*p == '.' || *p == 'e' || *p == 'E')) return fail();
        return true;
    }

    bool u64_list(std::vector<uint64_t>& out) {
        out.clear();
        if (!eat('[')) return fail();
        if (eat(']')) return true;
        do {
            uint64_t v;
            if (!u64(v) || out.size() >= 16) return fail();
            out.push_back(v);
        } while (eat(','));
        return eat(']') || fail();
    }

    // Any JSON value, discarded.
    bool skip(int depth = 0) {
        if (depth > 32) return fail();
        ws();
        if (p >= e) return fail();
        if (*p == '"') { std::string t; return str(t); }
        if (*p == '{') {
            ++p;
            if (eat('}')) return true;
            do {
                std::string k;
                if (!str(k) || !eat(':') || !skip(depth + 1)) return fail();
            } while (eat(','));
            return eat('}') || fail();
        }
        if (*p == '[') {
            ++p;
            if (eat(']')) return true;
            do {
                if (!skip(depth + 1)) return fail();
            } while (eat(','));
            return eat(']') || fail();
        }
        for (const char* lit : {"true", "false", "null"}) {
            const size_t n = std::strlen(lit);
            if ((size_t)(e - p) >= n && !std::memcmp(p, lit, n)) { p += n; return true; }
        }
        // a number
        const char* s = p;
        if (p < e && *p == '-') ++p;
        while (p < e && ((*p >= '0' && *p <= '9') || *p == '.' || *p == 'e' || *p == 'E' || *p == '+' || *p == '-')) ++p;
        return p > s || fail();
    }
};

// Parses the header into tensors; false for anything that is not a JSON object of tensor entries.
bool vx_st_parse(const char* json, size_t n, VeloxHipSafetensors& st) {
    VxJson j{json, json + n};
    if (!j.eat('{')) return false;
    if (j.eat('}')) { j.ws(); return j.p == j.e; }
    do {
        std::string key;
        if (!j.str(key) || !j.eat(':')) return false;
        if (key == "__metadata__") {
            if (!j.peek('{') || !j.skip()) return false;
            continue;
        }
        if (!j.eat('{')) return false;
        VxStTensor t;
        t.name = key;
        bool has_dtype = false, has_shape = false, has_off = false;
        if (!j.eat('}')) {
            do {
                std::string f;
                if (!j.str(f) || !j.eat(':')) return false;
                if (f == "dtype") { if (!j.str(t.dtype)) return false; has_dtype = true; }
                else if (f == "shape") { if (!j.u64_list(t.shape)) return false; has_shape = true; }
                else if (f == "data_offsets") {
                    std::vector<uint64_t> o;
                    if (!j.u64_list(o) || o.size() != 2) return false;
                    t.begin = o[0];
                    t.end = o[1];
                    has_off = true;
                } else if (!j.skip()) {
                    return false;
                }
            } while (j.eat(','));
            if (!j.eat('}')) return false;
        }
        if (!has_dtype || !has_shape || !has_off || st.index.count(key)) return false;
        st.index.emplace(key, st.tensors.size());
        st.tensors.push_back(std::move(t));
    } while (j.eat(','));
    if (!j.eat('}')) return false;
    j.ws();
    return j.ok && j.p == j.e;
}

uint64_t vx_st_dtype_bytes(const std::string& dt) {
    if (dt == "F64" || dt == "I64" || dt == "U64") return 8;
    if (dt == "F32" || dt == "I32" || dt == "U32") return 4;
    if (dt == "F16" || dt == "BF16" || dt == "I16" || dt == "U16") return 2;
    if (dt == "F8_E4M3" || dt == "F8_E5M2" || dt == "I8" || dt == "U8" || dt == "BOOL") return 1;
    return 0;
}

const VxStTensor* vx_st_get(const VeloxHipSafetensors* st, const std::string& name) {
    auto it = st->index.find(name);
    if (it == st->index.end() && name == "lm_head.weight") it = st->index.find("model.embed_tokens.weight");
    return it == st->index.end() ? nullptr : &st->tensors[it->second];
}

// Bounds of a tensor's data (E013 when outside the file or inverted) and its size against its shape.
int vx_st_span(const VeloxHipSafetensors* st, const VxStTensor& t, const uint8_t** data, uint64_t* nbytes) {
    const uint64_t avail = st->size - st->data_start;
    if (t.begin > t.end || t.end > avail) return VELOX_HIP_ETENSOR;
    const uint64_t eb = vx_st_dtype_bytes(t.dtype);
    uint64_t count = 1;
    for (uint64_t d : t.shape) {
        if (d && count > (~0ull) / d) return VELOX_HIP_ESHAPE;
        count *= d;
    }
    if (!eb || count > (~0ull) / eb || count * eb != t.end - t.begin) return VELOX_HIP_ESHAPE;
    *data = st->base + st->data_start + t.begin;
    *nbytes = t.end - t.begin;
    return VELOX_HIP_OK;
}

int vx_st_dt_code(const std::string& dt, uint32_t* code) {
    if (dt == "F32") *code = VELOX_DT_F32;
    else if (dt == "F16") *code = VELOX_DT_F16;
    else if (dt == "BF16") *code = VELOX_DT_BF16;
    else return VELOX_HIP_EDTYPE;
    return VELOX_HIP_OK;
}

std::string vx_layer_name(uint32_t l, const char* leaf) { return "model.layers." + std::to_string(l) + "." + leaf; }

// The tensors a model's plan loads: name, kind, layer, expected [rows, cols] (cols 0: a vector).
struct VxStWant {
    std::string name;
    int kind;
    uint32_t layer;
    uint64_t rows, cols;
};

std::vector<VxStWant> vx_st_wants(const VeloxHipModelConfig& c) {
    const uint64_t H = c.hidden_dim, F = c.intermediate_dim, qd = (uint64_t)c.num_heads * c.head_dim,
                   kvd = (uint64_t)c.num_kv_heads * c.head_dim;
    std::vector<VxStWant> w;
    w.push_back({"model.embed_tokens.weight", VELOX_T_EMBED, 0, c.vocab_size, H});
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        w.push_back({vx_layer_name(l, "input_layernorm.weight"), VELOX_T_ATTN_NORM, l, H, 0});
        w.push_back({vx_layer_name(l, "self_attn.q_proj.weight"), VELOX_T_Q, l, qd, H});
        w.push_back({vx_layer_name(l, "self_attn.k_proj.weight"), VELOX_T_K, l, kvd, H});
        w.push_back({vx_layer_name(l, "self_attn.v_proj.weight"), VELOX_T_V, l, kvd, H});
        if (c.qkv_bias) {
            w.push_back({vx_layer_name(l, "self_attn.q_proj.bias"), VELOX_T_BQ, l, qd, 0});
            w.push_back({vx_layer_name(l, "self_attn.k_proj.bias"), VELOX_T_BK, l, kvd, 0});
            w.push_back({vx_layer_name(l, "self_attn.v_proj.bias"), VELOX_T_BV, l, kvd, 0});
        }
        w.push_back({vx_layer_name(l, "self_attn.o_proj.weight"), VELOX_T_O, l, H, qd});
        w.push_back({vx_layer_name(l, "post_attention_layernorm.weight"), VELOX_T_MLP_NORM, l, H, 0});
        w.push_back({vx_layer_name(l, "mlp.gate_proj.weight"), VELOX_T_GATE, l, F, H});
        w.push_back({vx_layer_name(l, "mlp.up_proj.weight"), VELOX_T_UP, l, F, H});
        w.push_back({vx_layer_name(l, "mlp.down_proj.weight"), VELOX_T_DOWN, l, H, F});
    }
    w.push_back({"model.norm.weight", VELOX_T_FINAL_NORM, 0, H, 0});
    if (!c.tied_lm_head) w.push_back({"lm_head.weight", VELOX_T_HEAD, 0, c.vocab_size, H});
    return w;
}

bool vx_st_shape_is(const VxStTensor& t, uint64_t rows, uint64_t cols) {
    if (cols == 0) return t.shape.size() == 1 && t.shape[0] == rows;
    return t.shape.size() == 2 && t.shape[0] == rows && t.shape[1] == cols;
}

}  // namespace

extern "C" {

int velox_hip_st_open(const char* path, VeloxHipSafetensors** out) {
    if (!path || !out) return VELOX_HIP_EINVAL;
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) return VELOX_HIP_ENOTLOADED;
    struct stat sb;
    if (fstat(fd, &sb) != 0 || !S_ISREG(sb.st_mode)) { ::close(fd); return VELOX_HIP_ENOTLOADED; }
    const size_t size = (size_t)sb.st_size;
    if (size < 8) { ::close(fd); return VELOX_HIP_EINVAL; }  // no room for the header length
    void* base = mmap(nullptr, size, PROT_READ, MAP_PRIVATE, fd, 0);
    ::close(fd);
    if (base == MAP_FAILED) return VELOX_HIP_ENOTLOADED;
    VeloxHipSafetensors* st = new VeloxHipSafetensors;
    st->base = (const uint8_t*)base;
    st->size = size;
    uint64_t hlen;
    std::memcpy(&hlen, st->base, 8);  // little-endian, as the host
    int rc = VELOX_HIP_OK;
    if (hlen > size - 8) rc = VELOX_HIP_EINVAL;  // header length beyond the file
    else if (!vx_utf8_ok(st->base + 8, (size_t)hlen)) rc = VELOX_HIP_EINVAL;
    else if (!vx_st_parse((const char*)st->base + 8, (size_t)hlen, *st)) rc = VELOX_HIP_EINVAL;
    if (rc) {
        munmap(base, size);
        delete st;
        return rc;
    }
    st->data_start = 8 + hlen;
    *out = st;
    return VELOX_HIP_OK;
}

void velox_hip_st_close(VeloxHipSafetensors* st) {
    if (!st) return;
    if (st->base) munmap((void*)st->base, st->size);
    delete st;
}

uint64_t velox_hip_st_tensor_count(const VeloxHipSafetensors* st) { return st ? st->tensors.size() : 0; }

int velox_hip_st_tensor_info(const VeloxHipSafetensors* st, uint64_t i, char* name, uint32_t name_cap, char* dtype,
                             uint64_t* shape, uint32_t* n_dims, uint64_t* begin, uint64_t* end) {
    if (!st || i >= st->tensors.size()) return VELOX_HIP_EINVAL;
    const VxStTensor& t = st->tensors[(size_t)i];
    if (name && name_cap) std::snprintf(name, name_cap, "%s", t.name.c_str());
    if (dtype) std::snprintf(dtype, 16, "%s", t.dtype.c_str());
    if (n_dims) *n_dims = (uint32_t)t.shape.size();
    if (shape) for (size_t d = 0; d < t.shape.size() && d < 8; ++d) shape[d] = t.shape[d];
    if (begin) *begin = t.begin;
    if (end) *end = t.end;
    return VELOX_HIP_OK;
}

int velox_hip_st_find(const VeloxHipSafetensors* st, const char* name, uint64_t* index) {
    if (!st || !name) return VELOX_HIP_EINVAL;
    const VxStTensor* t = vx_st_get(st, name);
    if (!t) return VELOX_HIP_ETENSOR;
    if (index) *index = (uint64_t)(t - st->tensors.data());
    return VELOX_HIP_OK;
}

int velox_hip_st_tensor_data(const VeloxHipSafetensors* st, const char* name, const char* dtype, const void** data,
                             uint64_t* nbytes) {
    if (!st || !name || !dtype) return VELOX_HIP_EINVAL;
    const VxStTensor* t = vx_st_get(st, name);
    if (!t) return VELOX_HIP_ETENSOR;
    if (t->dtype != dtype) return VELOX_HIP_EDTYPE;
    const uint8_t* p = nullptr;
    uint64_t n = 0;
    const int rc = vx_st_span(st, *t, &p, &n);
    if (rc) return rc;
    if (data) *data = p;
    if (nbytes) *nbytes = n;
    return VELOX_HIP_OK;
}

int velox_hip_st_config(const VeloxHipSafetensors* st, uint32_t max_seq_len, VeloxHipModelConfig* out) {
    if (!st || !out) return VELOX_HIP_EINVAL;
    const VxStTensor* emb = vx_st_get(st, "model.embed_tokens.weight");
    const VxStTensor* q = vx_st_get(st, "model.layers.0.self_attn.q_proj.weight");
    const VxStTensor* k = vx_st_get(st, "model.layers.0.self_attn.k_proj.weight");
    const VxStTensor* g = vx_st_get(st, "model.layers.0.mlp.gate_proj.weight");
    if (!emb || !q || !k || !g) return VELOX_HIP_ETENSOR;
    if (emb->shape.size() != 2 || q->shape.size() != 2 || k->shape.size() != 2 || g->shape.size() != 2)
        return VELOX_HIP_ESHAPE;
    uint32_t layers = 0;
    while (vx_st_get(st, vx_layer_name(layers, "input_layernorm.weight"))) ++layers;
    const uint32_t bias = vx_st_get(st, "model.layers.0.self_attn.q_proj.bias") ? 1u : 0u;
    const uint32_t tied = st->index.count("lm_head.weight") ? 0u : 1u;
    // safetensors carries no head count or head size: the builtin configuration with the same layer
    // shapes supplies them, with vocabulary, depth and head tying taken from the file
    for (const char* which : {"smollm_135m", "llama3_8b", "qwen2_5_7b", "qwen2_72b"}) {
        VeloxHipModelConfig c;
        if (velox_hip_builtin_config(which, max_seq_len, &c)) continue;
        if (emb->shape[1] != c.hidden_dim || q->shape[0] != (uint64_t)c.num_heads * c.head_dim ||
            k->shape[0] != (uint64_t)c.num_kv_heads * c.head_dim || g->shape[0] != c.intermediate_dim ||
            bias != c.qkv_bias || layers == 0)
            continue;
        c.vocab_size = (uint32_t)emb->shape[0];
        c.num_layers = layers;
        c.tied_lm_head = tied;
        c.quant_mode = VELOX_QUANT_F32;  // the reference runner's default: the checkpoint's fp32 values
        *out = c;
        return VELOX_HIP_OK;
    }
    return VELOX_HIP_EINVAL;
}

int velox_hip_st_check(const VeloxHipSafetensors* st, const VeloxHipModelConfig* cfg) {
    if (!st || !cfg) return VELOX_HIP_EINVAL;
    VeloxHipModelConfig c = *cfg;
    for (const VxStWant& w : vx_st_wants(c)) {
        const VxStTensor* t = vx_st_get(st, w.name);
        if (!t) return VELOX_HIP_ETENSOR;
        uint32_t dt;
        if (vx_st_dt_code(t->dtype, &dt)) return VELOX_HIP_EDTYPE;
        const uint8_t* p;
        uint64_t n;
        const int rc = vx_st_span(st, *t, &p, &n);
        if (rc) return rc;
        if (!vx_st_shape_is(*t, w.rows, w.cols)) return VELOX_HIP_ESHAPE;
    }
    return VELOX_HIP_OK;
}

int velox_hip_st_load(VeloxHipArena* arena, const VeloxHipSafetensors* st, hipStream_t stream) {
    const VeloxHipModel* M = arena ? velox_hip_arena_model(arena) : nullptr;
    if (!M || !st) return VELOX_HIP_EINVAL;
    VeloxHipModelConfig c;
    int rc = velox_hip_model_config(M, &c);
    if (!rc) rc = velox_hip_st_check(st, &c);
    if (rc) return rc;
    for (const VxStWant& w : vx_st_wants(c)) {
        const VxStTensor* t = vx_st_get(st, w.name);
        uint32_t dt = 0;
        const uint8_t* p = nullptr;
        uint64_t n = 0;
        rc = vx_st_dt_code(t->dtype, &dt);
        if (!rc) rc = vx_st_span(st, *t, &p, &n);
        if (!rc) rc = velox_hip_load_tensor(arena, w.kind, w.layer, p, n, dt, stream);
        if (rc) return rc;
    }
    return VELOX_HIP_OK;
}

}  // extern "C"
