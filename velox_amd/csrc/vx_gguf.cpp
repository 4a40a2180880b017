// vx_gguf.cpp -- GGUF checkpoint reader for Q4_0 models (GGML's container: "GGUF" magic, version,
// tensor and metadata counts, typed key/value metadata, a tensor directory, tensor data at
// general.alignment). The reference reads the same container in its K2 runner
// (src/runners/velox_cuda_runner_k2.cu:48-196, tensor type table scripts/test_gguf_kv_dump.c:69,
// llama.cpp tensor names at :1918-1963). Here the file is memory-mapped (POSIX), every read is bounds
// checked, the model configuration comes from the {arch}.* metadata, and the Q4_0 matrices and
// fp32/fp16 vectors load into an arena through the same repack as the synthetic weights.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cmath>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

#include "vx_common.h"

namespace {

struct VxGgufTensor {
    std::string name;
    uint32_t type = 0, n_dims = 0;
    uint64_t dims[4] = {1, 1, 1, 1};
    uint64_t offset = 0, nbytes = 0;
};

enum { GG_U8 = 0, GG_I8, GG_U16, GG_I16, GG_U32, GG_I32, GG_F32, GG_BOOL, GG_STR, GG_ARR, GG_U64, GG_I64, GG_F64 };
enum { GT_F32 = 0, GT_F16 = 1, GT_Q4_0 = 2 };

// Bytes of n elements of a GGML tensor type (block types: bytes per block / elements per block).
bool vx_gguf_type_bytes(uint32_t type, uint64_t n, uint64_t& out) {
    struct B { uint32_t t, blk, bytes; };
    static const B table[] = {{0, 1, 4},    {1, 1, 2},    {2, 32, 18},   {3, 32, 20},  {6, 32, 22},
                              {7, 32, 24},  {8, 32, 34},  {9, 32, 36},   {10, 256, 84}, {11, 256, 110},
                              {12, 256, 144}, {13, 256, 176}, {14, 256, 210}, {15, 256, 292}, {30, 1, 2}};
    for (const B& b : table)
        if (b.t == type) {
            if (n % b.blk) return false;
            out = n / b.blk * b.bytes;
            return true;
        }
    return false;
}

struct VxCursor {
    const uint8_t* base;
    size_t size, pos = 0;
    bool ok = true;
    bool need(size_t n) {
        if (!ok || n > size || pos > size - n) ok = false;
        return ok;
    }
    template <typename T>
    T get() {
        T v{};
        if (need(sizeof(T))) { std::memcpy(&v, base + pos, sizeof(T)); pos += sizeof(T); }
        return v;
    }
    std::string str() {
        const uint64_t n = get<uint64_t>();
        if (!need((size_t)n) || n > (1u << 24)) { ok = false; return std::string(); }
        std::string s((const char*)base + pos, (size_t)n);
        pos += (size_t)n;
        return s;
    }
};

size_t vx_gguf_scalar_size(uint32_t t) {
    switch (t) {
        case GG_U8: case GG_I8: case GG_BOOL: return 1;
        case GG_U16: case GG_I16: return 2;
        case GG_U32: case GG_I32: case GG_F32: return 4;
        case GG_U64: case GG_I64: case GG_F64: return 8;
        default: return 0;
    }
}

double vx_gguf_scalar(VxCursor& c, uint32_t t) {
    switch (t) {
        case GG_U8: return c.get<uint8_t>();
        case GG_I8: return c.get<int8_t>();
        case GG_BOOL: return c.get<uint8_t>();
        case GG_U16: return c.get<uint16_t>();
        case GG_I16: return c.get<int16_t>();
        case GG_U32: return c.get<uint32_t>();
        case GG_I32: return c.get<int32_t>();
        case GG_F32: return c.get<float>();
        case GG_U64: return (double)c.get<uint64_t>();
        case GG_I64: return (double)c.get<int64_t>();
        case GG_F64: return c.get<double>();
        default: c.ok = false; return 0.0;
    }
}

}  // namespace

struct VeloxHipGguf {
    int fd = -1;
    const uint8_t* base = nullptr;
    size_t size = 0;
    uint32_t version = 0, alignment = 32;
    uint64_t data_start = 0;
    std::string arch;
    std::unordered_map<std::string, double> num;
    std::unordered_map<std::string, std::string> text;
    std::vector<VxGgufTensor> tensors;
    std::unordered_map<std::string, size_t> by_name;
};

namespace {

const VxGgufTensor* vx_gguf_find(const VeloxHipGguf* g, const std::string& name) {
    auto it = g->by_name.find(name);
    return it == g->by_name.end() ? nullptr : &g->tensors[it->second];
}

bool vx_gguf_parse(VeloxHipGguf* g) {
    VxCursor c{g->base, g->size};
    if (c.get<uint32_t>() != 0x46554747u) return false;  // "GGUF"
    g->version = c.get<uint32_t>();
    if (g->version < 2 || g->version > 3) return false;
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok || n_tensors > (1u << 20) || n_kv > (1u << 20)) return false;
    for (uint64_t k = 0; k < n_kv && c.ok; ++k) {
        const std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        if (t == GG_STR) {
            g->text[key] = c.str();
        } else if (t == GG_ARR) {
            const uint32_t et = c.get<uint32_t>();
            const uint64_t n = c.get<uint64_t>();
            if (et == GG_STR) {
                for (uint64_t i = 0; i < n && c.ok; ++i) (void)c.str();
            } else {
                const size_t es = vx_gguf_scalar_size(et);
                if (!es || n > c.size || !c.need((size_t)(n * es))) return false;
                c.pos += (size_t)(n * es);
            }
        } else {
            if (!vx_gguf_scalar_size(t)) return false;
            g->num[key] = vx_gguf_scalar(c, t);
        }
    }
    if (!c.ok) return false;
    auto al = g->num.find("general.alignment");
    if (al != g->num.end()) g->alignment = (uint32_t)al->second;
    if (g->alignment == 0 || (g->alignment & (g->alignment - 1))) return false;
    auto ar = g->text.find("general.architecture");
    if (ar != g->text.end()) g->arch = ar->second;
    g->tensors.resize((size_t)n_tensors);
    for (uint64_t i = 0; i < n_tensors && c.ok; ++i) {
        VxGgufTensor& t = g->tensors[(size_t)i];
        t.name = c.str();
        t.n_dims = c.get<uint32_t>();
        if (t.n_dims == 0 || t.n_dims > 4) return false;
        uint64_t n = 1;
        for (uint32_t d = 0; d < t.n_dims; ++d) {
            t.dims[d] = c.get<uint64_t>();
            if (t.dims[d] == 0 || t.dims[d] > (1ull << 32)) return false;
            n *= t.dims[d];
            if (n > (1ull << 40)) return false;
        }
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (!vx_gguf_type_bytes(t.type, n, t.nbytes)) t.nbytes = 0;  // unknown type: not loadable
        g->by_name[t.name] = (size_t)i;
    }
    if (!c.ok) return false;
    g->data_start = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (const VxGgufTensor& t : g->tensors)
        if (t.nbytes && (t.offset > g->size || g->data_start + t.offset + t.nbytes > g->size)) return false;
    return true;
}

double vx_gguf_num(const VeloxHipGguf* g, const std::string& key, double dflt) {
    auto it = g->num.find(key);
    return it == g->num.end() ? dflt : it->second;
}

}  // namespace

extern "C" {

int velox_hip_gguf_open(const char* path, VeloxHipGguf** out) {
    if (!path || !out) return VELOX_HIP_EINVAL;
    *out = nullptr;
    const int fd = ::open(path, O_RDONLY);
    if (fd < 0) return VELOX_HIP_EINVAL;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size < 24) {
        ::close(fd);
        return VELOX_HIP_ESHAPE;
    }
    void* p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    if (p == MAP_FAILED) {
        ::close(fd);
        return VELOX_HIP_ENOMEM;
    }
    VeloxHipGguf* g = new VeloxHipGguf();
    g->fd = fd;
    g->base = (const uint8_t*)p;
    g->size = (size_t)st.st_size;
    if (!vx_gguf_parse(g)) {
        munmap((void*)g->base, g->size);
        ::close(fd);
        delete g;
        return VELOX_HIP_ESHAPE;
    }
    *out = g;
    return VELOX_HIP_OK;
}

void velox_hip_gguf_close(VeloxHipGguf* g) {
    if (!g) return;
    if (g->base) munmap((void*)g->base, g->size);
    if (g->fd >= 0) ::close(g->fd);
    delete g;
}

uint64_t velox_hip_gguf_tensor_count(const VeloxHipGguf* g) { return g ? g->tensors.size() : 0; }

int velox_hip_gguf_tensor_info(const VeloxHipGguf* g, uint64_t i, char* name, uint32_t name_cap, uint32_t* type,
                               uint32_t* n_dims, uint64_t* dims, uint64_t* nbytes) {
    if (!g || i >= g->tensors.size()) return VELOX_HIP_EINVAL;
    const VxGgufTensor& t = g->tensors[(size_t)i];
    if (name && name_cap) std::snprintf(name, name_cap, "%s", t.name.c_str());
    if (type) *type = t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (dims) for (int d = 0; d < 4; ++d) dims[d] = t.dims[d];
    if (nbytes) *nbytes = t.nbytes;
    return VELOX_HIP_OK;
}

int velox_hip_gguf_config(const VeloxHipGguf* g, uint32_t max_seq_len, VeloxHipModelConfig* out) {
    if (!g || !out) return VELOX_HIP_EINVAL;
    const std::string a = g->arch.empty() ? std::string("llama") : g->arch;
    VeloxHipModelConfig c;
    std::memset(&c, 0, sizeof(c));
    std::snprintf(c.name, sizeof(c.name), "%s", a.c_str());
    c.hidden_dim = (uint32_t)vx_gguf_num(g, a + ".embedding_length", 0);
    c.num_layers = (uint32_t)vx_gguf_num(g, a + ".block_count", 0);
    c.intermediate_dim = (uint32_t)vx_gguf_num(g, a + ".feed_forward_length", 0);
    c.num_heads = (uint32_t)vx_gguf_num(g, a + ".attention.head_count", 0);
    c.num_kv_heads = (uint32_t)vx_gguf_num(g, a + ".attention.head_count_kv", c.num_heads);
    c.head_dim = c.num_heads ? (uint32_t)vx_gguf_num(g, a + ".attention.key_length", c.hidden_dim / c.num_heads) : 0;
    c.rms_norm_eps = (float)vx_gguf_num(g, a + ".attention.layer_norm_rms_epsilon", 1e-5);
    c.rope_theta = (float)vx_gguf_num(g, a + ".rope.freq_base", 10000.0);
    const uint32_t ctx = (uint32_t)vx_gguf_num(g, a + ".context_length", 4096);
    c.max_seq_len = max_seq_len ? max_seq_len : ctx;
    const VxGgufTensor* emb = vx_gguf_find(g, "token_embd.weight");
    if (!emb || emb->n_dims != 2) return VELOX_HIP_ESHAPE;
    c.vocab_size = (uint32_t)emb->dims[1];
    c.qkv_bias = vx_gguf_find(g, "blk.0.attn_q.bias") ? 1u : 0u;
    c.tied_lm_head = vx_gguf_find(g, "output.weight") ? 0u : 1u;
    c.quant_mode = VELOX_QUANT_GGML_Q4_0;
    if (!c.hidden_dim || !c.num_layers || !c.intermediate_dim || !c.num_heads || !c.head_dim) return VELOX_HIP_ESHAPE;
    *out = c;
    return VELOX_HIP_OK;
}

int velox_hip_gguf_load(VeloxHipArena* arena, const VeloxHipGguf* g, hipStream_t st) {
    if (!arena || !velox_hip_arena_model(arena) || !g) return VELOX_HIP_EINVAL;
    VeloxHipModelConfig c;
    int rc = velox_hip_gguf_config(g, 0, &c);
    if (rc) return rc;
    // llama.cpp stores llama's q/k rows permuted for its adjacent-pair RoPE: within each head, file
    // row 2i + j holds rotate-half row j * D/2 + i. Rows go back to rotate-half order here.
    const bool permuted_qk = g->arch == "llama";
    std::vector<uint8_t> tmp;
    auto matrix = [&](const std::string& name, int kind, uint32_t layer, uint64_t rows, uint64_t cols,
                      uint32_t heads) -> int {
        const VxGgufTensor* t = vx_gguf_find(g, name);
        if (!t) return VELOX_HIP_ESHAPE;
        if (t->type != GT_Q4_0 || t->n_dims != 2 || t->dims[0] != cols || t->dims[1] != rows) return VELOX_HIP_ESHAPE;
        const uint8_t* src = g->base + g->data_start + t->offset;
        const uint64_t row_bytes = cols / 32 * 18;
        if (heads) {
            const uint64_t D = rows / heads;
            tmp.resize(t->nbytes);
            for (uint64_t h = 0; h < heads; ++h)
                for (uint64_t i = 0; i < D / 2; ++i)
                    for (uint64_t j = 0; j < 2; ++j)
                        std::memcpy(tmp.data() + (h * D + j * (D / 2) + i) * row_bytes,
                                    src + (h * D + 2 * i + j) * row_bytes, row_bytes);
            src = tmp.data();
        }
        return velox_hip_load_q4_0(arena, kind, layer, src, t->nbytes, st);
    };
    auto vector = [&](const std::string& name, int kind, uint32_t layer, uint64_t n, uint32_t heads) -> int {
        const VxGgufTensor* t = vx_gguf_find(g, name);
        if (!t) return VELOX_HIP_ESHAPE;
        if (t->n_dims != 1 || t->dims[0] != n || (t->type != GT_F32 && t->type != GT_F16)) return VELOX_HIP_ESHAPE;
        const uint8_t* src = g->base + g->data_start + t->offset;
        std::vector<float> v((size_t)n);
        for (uint64_t i = 0; i < n; ++i) {
            if (t->type == GT_F32) std::memcpy(&v[(size_t)i], src + 4 * i, 4);
            else { uint16_t h; std::memcpy(&h, src + 2 * i, 2); v[(size_t)i] = vx_f16_bits_to_f32(h); }
        }
        if (heads) {
            const uint64_t D = n / heads;
            std::vector<float> u(v);
            for (uint64_t h = 0; h < heads; ++h)
                for (uint64_t i = 0; i < D / 2; ++i)
                    for (uint64_t j = 0; j < 2; ++j) v[(size_t)(h * D + j * (D / 2) + i)] = u[(size_t)(h * D + 2 * i + j)];
        }
        return velox_hip_load_f32(arena, kind, layer, v.data(), n, st);
    };
    const uint64_t H = c.hidden_dim, F = c.intermediate_dim, D = c.head_dim;
    const uint64_t qd = (uint64_t)c.num_heads * D, kvd = (uint64_t)c.num_kv_heads * D;
    VeloxHipModelConfig mc;
    rc = velox_hip_model_config(velox_hip_arena_model(arena), &mc);
    if (rc) return rc;
    if (mc.hidden_dim != c.hidden_dim || mc.num_layers != c.num_layers || mc.intermediate_dim != c.intermediate_dim ||
        mc.num_heads != c.num_heads || mc.num_kv_heads != c.num_kv_heads || mc.vocab_size != c.vocab_size ||
        mc.qkv_bias != c.qkv_bias || mc.tied_lm_head != c.tied_lm_head || mc.head_dim != c.head_dim ||
        std::fabs(mc.rms_norm_eps - c.rms_norm_eps) > 1e-3f * c.rms_norm_eps ||
        std::fabs(mc.rope_theta - c.rope_theta) > 1e-6f * c.rope_theta)
        return VELOX_HIP_ESHAPE;
    rc = matrix("token_embd.weight", VELOX_T_EMBED, 0, c.vocab_size, H, 0);
    for (uint32_t l = 0; l < c.num_layers && !rc; ++l) {
        const std::string p = "blk." + std::to_string(l) + ".";
        rc = matrix(p + "attn_q.weight", VELOX_T_Q, l, qd, H, permuted_qk ? c.num_heads : 0);
        if (!rc) rc = matrix(p + "attn_k.weight", VELOX_T_K, l, kvd, H, permuted_qk ? c.num_kv_heads : 0);
        if (!rc) rc = matrix(p + "attn_v.weight", VELOX_T_V, l, kvd, H, 0);
        if (!rc) rc = matrix(p + "attn_output.weight", VELOX_T_O, l, H, qd, 0);
        if (!rc) rc = matrix(p + "ffn_gate.weight", VELOX_T_GATE, l, F, H, 0);
        if (!rc) rc = matrix(p + "ffn_up.weight", VELOX_T_UP, l, F, H, 0);
        if (!rc) rc = matrix(p + "ffn_down.weight", VELOX_T_DOWN, l, H, F, 0);
        if (!rc) rc = vector(p + "attn_norm.weight", VELOX_T_ATTN_NORM, l, H, 0);
        if (!rc) rc = vector(p + "ffn_norm.weight", VELOX_T_MLP_NORM, l, H, 0);
        if (!rc && c.qkv_bias) {
            rc = vector(p + "attn_q.bias", VELOX_T_BQ, l, qd, permuted_qk ? c.num_heads : 0);
            if (!rc) rc = vector(p + "attn_k.bias", VELOX_T_BK, l, kvd, permuted_qk ? c.num_kv_heads : 0);
            if (!rc) rc = vector(p + "attn_v.bias", VELOX_T_BV, l, kvd, 0);
        }
    }
    if (!rc) rc = vector("output_norm.weight", VELOX_T_FINAL_NORM, 0, H, 0);
    if (!rc && !c.tied_lm_head) rc = matrix("output.weight", VELOX_T_HEAD, 0, c.vocab_size, H, 0);
    if (!rc) rc = (int)hipStreamSynchronize(st);
    return rc;
}

}  // extern "C"
