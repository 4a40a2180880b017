// vx_mla_host.cpp -- plan, arena, weight synthesis/loading and the layer step of the absorbed MLA
// layer (benchmark configuration 4). The reference runs its simplified MLA as one 256-thread kernel per layer
// (src/codegen.rs:2001-2109, launch at :2993) over fp32 weights the optimizer pre-absorbed
// (src/optimizer.rs:138-184); here the DeepSeek-V3 form streams fp8 weights through MFMA GEMMs and
// keeps the latent cache in bf16, sized for one GPU's 288 GB.
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <utility>
#include <vector>

#include "vx_common.h"
#include "vx_mla.h"

namespace {

inline uint64_t vm_align(uint64_t x, uint64_t a = 256) { return (x + a - 1) / a * a; }

enum {  // synthetic-tensor tags: tag = layer * 256 + kind (the oracle's VXO_T_MLA_*)
    VM_T_NORM = 32, VM_T_QA = 33, VM_T_QA_NORM = 34, VM_T_QB = 35, VM_T_KVA = 36, VM_T_KVA_NORM = 37,
    VM_T_KVB = 38, VM_T_O = 39, VM_T_CACHE = 41
};

struct VmF8Plan {  // one tiled fp8 matrix (or group of per-head matrices)
    uint64_t code_off = 0, scale_off = 0;
    uint32_t groups = 1, rows = 0, cols = 0, n_rt = 0, n_kt = 0, n_kb = 0;
    uint64_t w_gstride = 0, s_gstride = 0;  // uint4 units, floats
    uint64_t code_bytes() const { return (uint64_t)groups * rows * cols; }
    uint64_t scale_bytes() const { return (uint64_t)groups * n_rt * n_kb * 4; }
};

struct VmLayer {
    VmF8Plan a, qb, ukt, uv, o;
    uint64_t norm = 0, q_a_norm = 0, kv_a_norm = 0;  // byte offsets of fp32 gains
};

VmF8Plan vm_plan(uint32_t groups, uint32_t rows, uint32_t cols, uint64_t& code_cur, uint64_t& scale_cur) {
    VmF8Plan p;
    p.groups = groups;
    p.rows = rows;
    p.cols = cols;
    p.n_rt = rows / 16;
    p.n_kt = cols / 64;
    p.n_kb = (p.n_kt + 1) / 2;
    p.w_gstride = (uint64_t)p.n_rt * p.n_kt * 64;
    p.s_gstride = (uint64_t)p.n_rt * p.n_kb;
    p.code_off = code_cur;
    p.scale_off = scale_cur;
    code_cur = vm_align(code_cur + p.code_bytes());
    scale_cur = vm_align(scale_cur + p.scale_bytes());
    return p;
}

}  // namespace

struct VeloxHipMla {
    VeloxHipMlaConfig cfg;
    uint32_t H = 0, nh = 0, ql = 0, lr = 0, dn = 0, dr = 0, dv = 0, R = 0, dq = 0, na = 0, q_part = 0;
    uint32_t s_cap = 0, splits = 1, ks_a = 1, ks_o = 1, B = 1, ldx16 = 0;
    // one sequence: [W_qa; W_kva] over the whole K (8 waves per row tile split it), so W_qb normalizes
    // its q latent itself and one extra W_qb workgroup writes the latent row: no prep launch
    uint32_t ks_a1 = 1;
    float scale = 0.0f;
    std::vector<VmLayer> layers;
    uint64_t code_bytes = 0, scale_bytes = 0, norm_bytes = 0, rope_bytes = 0, cache_bytes = 0, act_bytes = 0;
    uint64_t cache_layer_bytes = 0;
    uint64_t o_rope = 0;  // the RoPE table's offset in the norm region (after the gains)
    // activation offsets (bytes from the activation region)
    uint64_t a_state = 0, a_h = 0, a_x16 = 0, a_parts_a = 0, a_q32 = 0, a_qabs = 0, a_po = 0, a_pml = 0, a_ctx = 0,
             a_oh = 0, a_parts_o = 0;
    // device regions, the fields of a VeloxHipArena: fp8 codes (weight_arena), block scales
    // (weight_scales), gains + RoPE table (norm_weight_arena), latent cache (kv_cache_pool),
    // states + activations (activation_arena). `base` is the one allocation of velox_hip_mla_create;
    // a planned handle bound to caller-owned buffers has none.
    uint8_t *w_codes = nullptr, *w_scales = nullptr, *w_norms = nullptr, *kv = nullptr, *act = nullptr;
    uint8_t* base = nullptr;
};

namespace {

float* vm_act(const VeloxHipMla* m, uint64_t off) { return (float*)(m->act + off); }
const float2* vm_rope(const VeloxHipMla* m) { return (const float2*)(m->w_norms + m->o_rope); }
VeloxDecodeState* vm_states(const VeloxHipMla* m) { return (VeloxDecodeState*)(m->act + m->a_state); }
uint16_t* vm_cache(const VeloxHipMla* m, uint32_t layer) { return (uint16_t*)(m->kv + m->cache_layer_bytes * layer); }

bool vm_valid(const VeloxHipMlaConfig& c) {
    if (c.hidden_dim == 0 || c.num_heads == 0 || c.num_layers == 0 || c.max_seq_len == 0) return false;
    if (c.max_batch == 0 || c.max_batch > 32) return false;
    if (c.hidden_dim % 128 || c.q_lora_rank % 128 || c.qk_nope_dim % 128 || c.v_head_dim % 128) return false;
    if (c.qk_rope_dim != 64 || c.num_heads % 16) return false;
    if (!(c.kv_lora_rank == 512 && c.num_heads % 64 == 0) && c.kv_lora_rank != 128) return false;
    if (c.attn_splits > 64 || c.q_lora_rank > 16384) return false;
    return true;
}

// Packs one logical source matrix (synthesized when src_codes is null) into its destination(s).
hipError_t vm_pack_source(VeloxHipMla* m, uint32_t layer, int kind, const uint8_t* d_src_codes,
                          const float* d_src_scales, uint64_t stream, float coef, hipStream_t st) {
    VmLayer& L = m->layers[layer];
    uint8_t* codes = m->w_codes;
    float* scales = (float*)m->w_scales;
    auto dest = [&](const VmF8Plan& p, uint32_t map, uint32_t rows, uint32_t row_tile0, uint32_t row_off,
                    uint32_t src_rows, uint32_t src_cols) {
        VxF8Dest d;
        std::memset(&d, 0, sizeof(d));
        d.codes = (uint4*)(codes + p.code_off);
        d.scales = scales + p.scale_off / 4;
        d.groups = p.groups;
        d.rows = rows;
        d.cols = p.cols;
        d.n_rt_total = p.n_rt;
        d.n_kt = p.n_kt;
        d.n_kb = p.n_kb;
        d.row_tile0 = row_tile0;
        d.map = map;
        d.row_off = row_off;
        d.dn = m->dn;
        d.dv = m->dv;
        d.src_rows = src_rows;
        d.src_cols = src_cols;
        d.src_codes = d_src_codes;
        d.src_scales = d_src_scales;
        d.stream = stream;
        d.coef = coef;
        d.w_gstride = p.w_gstride;
        d.s_gstride = p.s_gstride;
        return vx_launch_f8_pack(d, st);
    };
    const uint32_t H = m->H, nh = m->nh;
    switch (kind) {
        case VELOX_MLA_Q_A:
            if (!m->ql) return hipErrorInvalidValue;
            return dest(L.a, VX_MAP_DIRECT, m->ql, 0, 0, m->ql, H);
        case VELOX_MLA_Q_B:
            if (m->ql) return dest(L.qb, VX_MAP_DIRECT, nh * m->dq, 0, 0, nh * m->dq, m->ql);
            return dest(L.a, VX_MAP_DIRECT, nh * m->dq, 0, 0, nh * m->dq, H);
        case VELOX_MLA_KV_A:
            return dest(L.a, VX_MAP_DIRECT, m->R, m->q_part / 16, 0, m->R, H);
        case VELOX_MLA_KV_B: {
            const uint32_t rows = nh * (m->dn + m->dv);
            hipError_t e = dest(L.ukt, VX_MAP_UKT, m->lr, 0, 0, rows, m->lr);
            if (e == hipSuccess) e = dest(L.uv, VX_MAP_UV, m->dv, 0, 0, rows, m->lr);
            return e;
        }
        case VELOX_MLA_O:
            return dest(L.o, VX_MAP_DIRECT, H, 0, 0, H, nh * m->dv);
        default:
            return hipErrorInvalidValue;
    }
}

void vm_source_dims(const VeloxHipMla* m, int kind, uint32_t& rows, uint32_t& cols) {
    rows = cols = 0;
    switch (kind) {
        case VELOX_MLA_Q_A: rows = m->ql; cols = m->H; break;
        case VELOX_MLA_Q_B: rows = m->nh * m->dq; cols = m->ql ? m->ql : m->H; break;
        case VELOX_MLA_KV_A: rows = m->R; cols = m->H; break;
        case VELOX_MLA_KV_B: rows = m->nh * (m->dn + m->dv); cols = m->lr; break;
        case VELOX_MLA_O: rows = m->H; cols = m->nh * m->dv; break;
        default: break;
    }
}

uint64_t vm_norm_off(const VeloxHipMla* m, uint32_t layer, int kind, uint32_t& n) {
    const VmLayer& L = m->layers[layer];
    switch (kind) {
        case VELOX_MLA_NORM: n = m->H; return L.norm;
        case VELOX_MLA_Q_A_NORM: n = m->ql; return L.q_a_norm;
        case VELOX_MLA_KV_A_NORM: n = m->lr; return L.kv_a_norm;
        default: n = 0; return 0;
    }
}

}  // namespace

extern "C" {

int velox_hip_mla_builtin_config(const char* which, uint32_t max_seq_len, uint32_t max_batch, VeloxHipMlaConfig* out) {
    if (!which || !out) return VELOX_HIP_EINVAL;
    std::memset(out, 0, sizeof(*out));
    if (std::strcmp(which, "deepseek_v3_mla") != 0) return VELOX_HIP_EINVAL;
    out->hidden_dim = 7168;
    out->num_heads = 128;
    out->q_lora_rank = 1536;
    out->kv_lora_rank = 512;
    out->qk_nope_dim = 128;
    out->qk_rope_dim = 64;
    out->v_head_dim = 128;
    out->num_layers = 1;
    out->max_seq_len = max_seq_len ? max_seq_len : 4096;
    out->max_batch = max_batch ? max_batch : 1;
    out->kv_norm = 1;
    out->rms_norm_eps = 1e-6f;
    out->rope_theta = 10000.0f;
    return VELOX_HIP_OK;
}

int velox_hip_mla_plan(const VeloxHipMlaConfig* cfg, VeloxHipMla** out) {
    if (!cfg || !out) return VELOX_HIP_EINVAL;
    *out = nullptr;
    if (!vm_valid(*cfg)) return VELOX_HIP_ESHAPE;
    VeloxHipMla* m = new VeloxHipMla();
    m->cfg = *cfg;
    const VeloxHipMlaConfig& c = m->cfg;
    m->H = c.hidden_dim;
    m->nh = c.num_heads;
    m->ql = c.q_lora_rank;
    m->lr = c.kv_lora_rank;
    m->dn = c.qk_nope_dim;
    m->dr = c.qk_rope_dim;
    m->dv = c.v_head_dim;
    m->R = m->lr + m->dr;
    m->dq = m->dn + m->dr;
    m->q_part = m->ql ? m->ql : m->nh * m->dq;
    m->na = m->q_part + m->R;
    m->B = c.max_batch;
    m->s_cap = (c.max_seq_len + 31u) & ~31u;
    m->scale = c.softmax_scale > 0.0f ? c.softmax_scale : 1.0f / sqrtf((float)(m->dn + m->dr));
    m->ldx16 = ((m->H > m->ql ? m->H : m->ql) + 7u) & ~7u;

    // weights: per layer [W_qa; W_kva] (or [W_q; W_kva]), W_qb, W_uk^T and W_uv per head, W_o
    uint64_t cc = 0, sc = 0, nc = 0;
    m->layers.resize(c.num_layers);
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        VmLayer& L = m->layers[l];
        L.a = vm_plan(1, m->na, m->H, cc, sc);
        if (m->ql) L.qb = vm_plan(1, m->nh * m->dq, m->ql, cc, sc);
        L.ukt = vm_plan(m->nh, m->lr, m->dn, cc, sc);
        L.uv = vm_plan(m->nh, m->dv, m->lr, cc, sc);
        L.o = vm_plan(1, m->H, m->nh * m->dv, cc, sc);
        L.norm = nc;
        nc = vm_align(nc + (uint64_t)m->H * 4);
        L.q_a_norm = nc;
        nc = vm_align(nc + (uint64_t)(m->ql ? m->ql : 1) * 4);
        L.kv_a_norm = nc;
        nc = vm_align(nc + (uint64_t)m->lr * 4);
    }
    m->code_bytes = cc;
    m->scale_bytes = sc;
    m->norm_bytes = nc;
    m->rope_bytes = vm_align((uint64_t)c.max_seq_len * (m->dr / 2) * 8);
    m->cache_layer_bytes = (uint64_t)m->B * m->s_cap * m->R * 2;
    m->cache_bytes = vm_align(m->cache_layer_bytes * c.num_layers);

    // split counts: at most 512 workgroups for the two skinny GEMMs; attention ~256 workgroups with at
    // least 64 positions per split
    // row tiles per GEMM workgroup: 8 for the LDS-activation forms (up to 16 sequences), else the
    // register form's 4 waves x rows per wave
    const uint32_t tpw = m->B <= 16 ? 8u : 4 * vx_f8gemm_rows_per_wave(m->B);
    const uint32_t wg_a = (m->na / 16 + tpw - 1) / tpw, wg_o = (m->H / 16 + tpw - 1) / tpw;
    // (at most 512 workgroups: one round of two per CU)
    m->ks_a = wg_a >= 512 ? 1u : 512 / wg_a;
    if (m->ks_a > 16) m->ks_a = 16;  // the prep kernel folds at most 16 partials
    if (m->ks_a > m->H / 64) m->ks_a = m->H / 64;
    m->ks_o = wg_o >= 512 ? 1u : 512 / wg_o;
    if (m->ks_o > 32) m->ks_o = 32;  // the next layer's RMSNorm folds at most 32 partials
    if (m->ks_o > m->nh * m->dv / 64) m->ks_o = m->nh * m->dv / 64;
    uint32_t splits = c.attn_splits;
    if (!splits) {
        const uint32_t hg = m->lr == 512 ? m->nh / 64 : m->nh / 16;
        splits = (256 + m->B * hg - 1) / (m->B * hg);
        const uint32_t by_len = (c.max_seq_len + 63) / 64;  // at least two 32-position chunks per split
        if (splits > by_len) splits = by_len;
    }
    if (splits < 1) splits = 1;
    if (splits > 64) splits = 64;
    if (!c.attn_splits) {
        // no split that max_seq_len leaves empty (the attention kernel's split length is this chunk):
        // DeepSeek-V3 at 4201 positions, 64 splits of 96 -> 44, B=1 68.9-69.3 -> 67.9-68.0 us per layer
        // (three alternating runs each; empty splits still wrote partials that W_uv merged)
        const uint32_t chunk = ((c.max_seq_len + splits - 1) / splits + 31) / 32 * 32;
        splits = (c.max_seq_len + chunk - 1) / chunk;
    }
    m->splits = splits;

    uint64_t ac = 0;
    auto take = [&](uint64_t bytes) { const uint64_t o = ac; ac = vm_align(ac + bytes); return o; };
    const uint64_t B = m->B;
    m->a_state = take(B * sizeof(VeloxDecodeState));
    m->a_h = take(B * m->H * 4);
    m->a_x16 = take(B * m->ldx16 * 2);
    m->a_parts_a = take((uint64_t)(m->ks_a > m->ks_a1 ? m->ks_a : m->ks_a1) * B * m->na * 4);
    m->a_q32 = take(B * m->nh * m->dq * 4);
    m->a_qabs = take(B * m->nh * m->lr * 4);
    m->a_po = take(B * m->nh * splits * m->lr * 2);
    m->a_pml = take(B * m->nh * splits * 2 * 4);
    m->a_ctx = take(B * m->nh * m->lr * 4);
    m->a_oh = take(B * m->nh * m->dv * 4);
    m->a_parts_o = take((uint64_t)m->ks_o * B * m->H * 4);
    m->act_bytes = ac;

    m->o_rope = vm_align(m->norm_bytes);
    const uint64_t total = vm_align(m->code_bytes) + vm_align(m->scale_bytes) + m->o_rope + m->rope_bytes +
                           m->cache_bytes + m->act_bytes;
    const uint64_t budget = c.vram_budget_bytes ? c.vram_budget_bytes : 288ULL * 1000 * 1000 * 1000;
    if (total > budget) {  // reference diagnostic E002 (src/memory_planner.rs:398-420)
        delete m;
        return VELOX_HIP_ENOMEM;
    }
    *out = m;
    return VELOX_HIP_OK;
}

}  // extern "C"

namespace {

// Zeroes the regions and writes the RoPE table of the rope part (src/runtime.rs:754-760: fp32 powf,
// product, sin/cos) into the norm region after the gains.
hipError_t vm_init_regions(VeloxHipMla* m) {
    const VeloxHipMlaConfig& c = m->cfg;
    hipError_t e = hipMemset(m->w_codes, 0, m->code_bytes);
    if (e == hipSuccess) e = hipMemset(m->w_scales, 0, m->scale_bytes);
    if (e == hipSuccess) e = hipMemset(m->w_norms, 0, m->o_rope + m->rope_bytes);
    if (e == hipSuccess) e = hipMemset(m->kv, 0, m->cache_bytes);
    if (e == hipSuccess) e = hipMemset(m->act, 0, m->act_bytes);
    if (e != hipSuccess) return e;
    const uint32_t half = m->dr / 2;
    std::vector<float> rope((size_t)c.max_seq_len * half * 2);
    for (uint32_t p = 0; p < c.max_seq_len; ++p)
        for (uint32_t j = 0; j < half; ++j) {
            const float freq = 1.0f / powf(c.rope_theta, (float)(2 * j) / (float)m->dr);
            const float angle = (float)p * freq;
            rope[((size_t)p * half + j) * 2] = cosf(angle);
            rope[((size_t)p * half + j) * 2 + 1] = sinf(angle);
        }
    return hipMemcpy(m->w_norms + m->o_rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice);
}

bool vm_has_buffers(const VeloxHipMla* m) { return m && m->w_codes && m->w_scales && m->w_norms && m->kv && m->act; }

// Arenas over MLA handles (velox_hip_mla_arena / _arena_bind), found by weight_arena.
std::mutex g_mla_mu;
std::vector<std::pair<const uint8_t*, VeloxHipMla*>> g_mla_arenas;

void vm_forget(const VeloxHipMla* m) {
    std::lock_guard<std::mutex> lk(g_mla_mu);
    for (size_t i = 0; i < g_mla_arenas.size();)
        if (g_mla_arenas[i].second == m) g_mla_arenas.erase(g_mla_arenas.begin() + (long)i);
        else ++i;
}

}  // namespace

extern "C" {

int velox_hip_mla_create(const VeloxHipMlaConfig* cfg, VeloxHipMla** out) {
    VeloxHipMla* m = nullptr;
    int rc = velox_hip_mla_plan(cfg, &m);
    if (rc) return rc;
    const uint64_t o_scales = vm_align(m->code_bytes), o_norms = o_scales + vm_align(m->scale_bytes);
    const uint64_t o_cache = o_norms + m->o_rope + m->rope_bytes, o_act = o_cache + m->cache_bytes;
    hipError_t e = hipMalloc((void**)&m->base, o_act + m->act_bytes);
    if (e == hipSuccess) {
        m->w_codes = m->base;
        m->w_scales = m->base + o_scales;
        m->w_norms = m->base + o_norms;
        m->kv = m->base + o_cache;
        m->act = m->base + o_act;
        e = vm_init_regions(m);
    }
    if (e != hipSuccess) {
        if (m->base) hipFree(m->base);
        delete m;
        return (int)e;
    }
    *out = m;
    return VELOX_HIP_OK;
}

void velox_hip_mla_destroy(VeloxHipMla* m) {
    if (!m) return;
    vm_forget(m);
    if (m->base) hipFree(m->base);
    delete m;
}

int velox_hip_mla_buffers(const VeloxHipMla* m, VeloxHipMlaBuffers* out) {
    if (!m || !out) return VELOX_HIP_EINVAL;
    out->hidden = vm_act(m, m->a_h);
    if (!vm_has_buffers(m)) return VELOX_HIP_ENOTLOADED;
    out->latent_cache = vm_cache(m, 0);
    out->states = vm_states(m);
    out->s_cap = m->s_cap;
    out->splits = m->splits;
    out->weight_bytes = m->code_bytes + m->scale_bytes + m->norm_bytes;
    out->cache_bytes = m->cache_bytes;
    out->act_bytes = m->act_bytes;
    return VELOX_HIP_OK;
}

int velox_hip_mla_load_fp8(VeloxHipMla* m, int kind, uint32_t layer, const uint8_t* codes, const float* scales,
                           hipStream_t st) {
    if (!vm_has_buffers(m) || !codes || !scales || layer >= m->cfg.num_layers) return VELOX_HIP_EINVAL;
    uint32_t rows, cols;
    vm_source_dims(m, kind, rows, cols);
    if (!rows) return VELOX_HIP_EINVAL;
    const uint64_t nb = (uint64_t)rows * cols, ns = (uint64_t)((rows + 127) / 128) * ((cols + 127) / 128) * 4;
    uint8_t* tmp = nullptr;
    hipError_t e = hipMalloc((void**)&tmp, vm_align(nb) + ns);
    if (e != hipSuccess) return (int)e;
    e = hipMemcpyAsync(tmp, codes, nb, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipMemcpyAsync(tmp + vm_align(nb), scales, ns, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = vm_pack_source(m, layer, kind, tmp, (const float*)(tmp + vm_align(nb)), 0, 0.0f, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    hipFree(tmp);
    return (int)e;
}

int velox_hip_mla_load_f32(VeloxHipMla* m, int kind, uint32_t layer, const float* data, uint64_t count,
                           hipStream_t st) {
    if (!vm_has_buffers(m) || !data || layer >= m->cfg.num_layers) return VELOX_HIP_EINVAL;
    uint32_t n;
    const uint64_t off = vm_norm_off(m, layer, kind, n);
    if (!n || count != n) return VELOX_HIP_EINVAL;
    hipError_t e = hipMemcpyAsync(m->w_norms + off, data, count * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return (int)e;
}

int velox_hip_mla_synthesize(VeloxHipMla* m, uint64_t seed, float sigma, float norm_sigma, hipStream_t st) {
    if (!vm_has_buffers(m)) return VELOX_HIP_EINVAL;
    // source block scales of the largest matrix
    uint64_t max_blocks = 0;
    for (int kind = VELOX_MLA_Q_A; kind <= VELOX_MLA_O; ++kind) {
        uint32_t r, c;
        vm_source_dims(m, kind, r, c);
        const uint64_t nbk = (uint64_t)((r + 127) / 128) * ((c + 127) / 128);
        if (nbk > max_blocks) max_blocks = nbk;
    }
    float* tmp = nullptr;
    hipError_t e = hipMalloc((void**)&tmp, max_blocks * 4);
    if (e != hipSuccess) return (int)e;
    const float coef = vx_normal_coef(sigma);
    for (uint32_t l = 0; l < m->cfg.num_layers && e == hipSuccess; ++l) {
        const int kinds[5] = {VELOX_MLA_Q_A, VELOX_MLA_Q_B, VELOX_MLA_KV_A, VELOX_MLA_KV_B, VELOX_MLA_O};
        const uint32_t tags[5] = {VM_T_QA, VM_T_QB, VM_T_KVA, VM_T_KVB, VM_T_O};
        for (int i = 0; i < 5 && e == hipSuccess; ++i) {
            if (kinds[i] == VELOX_MLA_Q_A && !m->ql) continue;
            uint32_t r, c;
            vm_source_dims(m, kinds[i], r, c);
            const uint64_t stream = vx_stream(seed, vx_tag(l, tags[i]));
            e = vx_launch_f8_synth_scales(tmp, r, c, stream, coef, st);
            if (e == hipSuccess) e = vm_pack_source(m, l, kinds[i], nullptr, tmp, stream, coef, st);
        }
        const int vk[3] = {VELOX_MLA_NORM, VELOX_MLA_Q_A_NORM, VELOX_MLA_KV_A_NORM};
        const uint32_t vt[3] = {VM_T_NORM, VM_T_QA_NORM, VM_T_KVA_NORM};
        for (int i = 0; i < 3 && e == hipSuccess; ++i) {
            uint32_t n;
            const uint64_t off = vm_norm_off(m, l, vk[i], n);
            if (!n) continue;
            e = vx_launch_fill_normal((float*)(m->w_norms + off), n, vx_stream(seed, vx_tag(l, vt[i])),
                                      norm_sigma > 0.0f ? vx_normal_coef(norm_sigma) : 0.0f, 1.0f, st);
        }
    }
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    hipFree(tmp);
    return (int)e;
}

int velox_hip_mla_fill_cache(VeloxHipMla* m, uint32_t layer, uint32_t seq, uint32_t n_pos, uint64_t seed, float sigma,
                             hipStream_t st) {
    if (!vm_has_buffers(m) || layer >= m->cfg.num_layers || seq >= m->B || n_pos > m->cfg.max_seq_len)
        return VELOX_HIP_EINVAL;
    const uint64_t sseed = seed + (uint64_t)seq * 0x9E3779B97F4A7C15ULL;
    uint16_t* dst = vm_cache(m, layer) + (uint64_t)seq * m->s_cap * m->R;
    hipError_t e = vx_launch_mla_fill_cache(dst, (uint64_t)n_pos * m->R, vx_stream(sseed, vx_tag(layer, VM_T_CACHE)),
                                            vx_normal_coef(sigma), st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return (int)e;
}

int velox_hip_mla_set_position(VeloxHipMla* m, uint32_t seq, uint64_t pos, hipStream_t st) {
    if (!vm_has_buffers(m) || seq >= m->B || pos >= m->cfg.max_seq_len) return VELOX_HIP_EINVAL;
    VeloxDecodeState* s = vm_states(m) + seq;
    hipError_t e = vx_launch_set_state(s, pos, 0u, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return (int)e;
}

}  // extern "C"

namespace {

// One layer's absorbed-MLA sub-block. With one sequence W_o is a GEMV over the whole K that adds
// its rows to h itself. Otherwise W_o leaves K-split partials: fold_prev -- the previous layer's
// partials are still to be added to h, which this layer's RMSNorm does (same split order as the
// residual kernel) before normalizing; finish -- this layer adds its own with the residual kernel.
void vm_layer(VeloxHipMla* m, uint32_t layer, uint32_t batch, uint64_t mask, bool fold_prev, bool finish,
              hipStream_t st) {
    const VmLayer& L = m->layers[layer];
    const bool direct = batch == 1;  // W_o GEMV with the residual epilogue
    fold_prev = fold_prev && !direct;
    finish = finish && !direct;
    const VeloxHipMlaConfig& c = m->cfg;
    const uint4* codes = (const uint4*)m->w_codes;
    const float* scales = (const float*)m->w_scales;
    const float* norms = (const float*)m->w_norms;
    VeloxDecodeState* states = vm_states(m);
    float* h = vm_act(m, m->a_h);
    uint16_t* x16 = (uint16_t*)vm_act(m, m->a_x16);
    uint16_t* cache = vm_cache(m, layer);
    auto gemm_args = [&](const VmF8Plan& p, const void* x, uint32_t ldx, uint64_t x_gstride, uint32_t x_f32, float* y,
                         uint32_t ldy, uint64_t y_gstride, uint32_t ksplit, uint64_t pstride, uint16_t* y16 = nullptr,
                         uint32_t add_y = 0, const float* gain = nullptr, const uint16_t* m_part_o = nullptr,
                         const float* m_part_ml = nullptr, uint32_t m_splits = 0) {
        VxF8GemmArgs g;
        std::memset(&g, 0, sizeof(g));
        g.codes = codes + p.code_off / 16;
        g.scales = scales + p.scale_off / 4;
        g.n_rt = p.n_rt;
        g.n_kt = p.n_kt;
        g.n_kb = p.n_kb;
        g.batch = batch;
        g.x = x;
        g.ldx = ldx;
        g.x_f32 = x_f32;
        g.y = y16 ? nullptr : y;
        g.y16 = y16;
        g.ldy = ldy;
        g.ksplit = ksplit;
        g.w_gstride = p.w_gstride;
        g.s_gstride = p.s_gstride;
        g.x_gstride = x_gstride;
        g.y_gstride = y_gstride;
        g.pstride = pstride;
        g.add_y = add_y;
        g.gain = gain;
        g.eps = c.rms_norm_eps;
        g.active_mask = mask;
        g.m_part_o = m_part_o;
        g.m_part_ml = m_part_ml;
        g.m_splits = m_splits;
        return g;
    };
    auto gemm = [&](const VmF8Plan& p, const void* x, uint32_t ldx, uint64_t x_gstride, uint32_t x_f32, float* y,
                    uint32_t ldy, uint64_t y_gstride, uint32_t ksplit, uint64_t pstride, uint16_t* y16 = nullptr,
                    uint32_t add_y = 0, const float* gain = nullptr, const uint16_t* m_part_o = nullptr,
                    const float* m_part_ml = nullptr, uint32_t m_splits = 0) {
        vx_record_error(vx_launch_f8gemm(gemm_args(p, x, ldx, x_gstride, x_f32, y, ldy, y_gstride, ksplit, pstride, y16,
                                                   add_y, gain, m_part_o, m_part_ml, m_splits),
                                         p.groups, st));
    };
    float* parts_o = vm_act(m, m->a_parts_o);
    const uint64_t pstride_o = (uint64_t)m->B * m->H;
    // 1. x = rmsnorm(h) as fp16 (h first takes the previous layer's W_o partials when they are pending);
    // 2. [W_qa; W_kva] x, split over K. One sequence: the GEMV normalizes h itself.
    const float* g_norm = (const float*)((const uint8_t*)norms + L.norm);
    float* parts_a = vm_act(m, m->a_parts_a);
    const uint64_t pstride_a = (uint64_t)m->B * m->na;
    // one sequence with a q LoRA: W_qb's prologue and the attention fold the partials (no prep)
    const bool folded = direct && m->ql > 0;
    if (direct) {
        gemm(L.a, h, m->H, 0, 1, parts_a, m->na, 0, folded ? m->ks_a1 : m->ks_a, pstride_a, nullptr, 0, g_norm);
    } else {
        vx_record_error(vx_launch_bnorm(h, m->H, fold_prev ? parts_o : nullptr, fold_prev ? m->ks_o : 0u,
                                        fold_prev ? pstride_o : 0u, g_norm, m->H, c.rms_norm_eps, x16, m->ldx16, 32u,
                                        batch, mask, st));
        gemm(L.a, x16, m->ldx16, 0, 0, parts_a, m->na, 0, m->ks_a, pstride_a);
    }
    // 3. q latent RMSNorm (fp16) or q; latent RMSNorm + RoPE(k_rope) appended to the cache
    float* q32 = vm_act(m, m->a_q32);
    {
        VxMlaPrepArgs a;
        std::memset(&a, 0, sizeof(a));
        a.parts = parts_a;
        a.nparts = m->ks_a;
        a.na = m->na;
        a.q_part = m->q_part;
        a.pstride = pstride_a;
        a.q_lora = m->ql;
        a.lr = m->lr;
        a.dr = m->dr;
        a.kv_norm = c.kv_norm;
        a.g_qa = (const float*)((const uint8_t*)norms + L.q_a_norm);
        a.g_kva = (const float*)((const uint8_t*)norms + L.kv_a_norm);
        a.eps = c.rms_norm_eps;
        a.states = states;
        a.s_max = c.max_seq_len;
        a.rope = vm_rope(m);
        a.cache = cache;
        a.cache_bstride = (uint64_t)m->s_cap * m->R;
        a.q16 = x16;
        a.ldq16 = m->ldx16;
        a.q32 = q32;
        a.active_mask = mask;
        if (folded) {
            // 4. q = W_qb q_latent, normalized in W_qb's prologue; its extra workgroup appends the latent row
            a.nparts = m->ks_a1;
            VxF8GemmArgs g = gemm_args(L.qb, parts_a, m->ql, 0, 1, q32, m->nh * m->dq, 0, 1, 0, nullptr, 0, a.g_qa);
            g.x_nparts = m->ks_a1;
            g.x_pstride = pstride_a;
            vx_record_error(vx_launch_f8gemv_prep(g, a, st));
        } else {
            vx_record_error(vx_launch_mla_prep(a, batch, st));
        }
    }
    // 4. q = W_qb q_latent
    if (!folded && m->ql) gemm(L.qb, x16, m->ldx16, 0, 0, q32, m->nh * m->dq, 0, 1, 0);
    // 5. absorption: q_abs[h] = W_uk[h]^T q_nope[h]
    float* qabs = vm_act(m, m->a_qabs);
    gemm(L.ukt, q32, m->nh * m->dq, m->dq, 1, qabs, m->nh * m->lr, m->lr, 1, 0);
    // 6. attention over the latent cache, split over positions; 7. merge
    uint16_t* po = (uint16_t*)vm_act(m, m->a_po);
    float* pml = vm_act(m, m->a_pml);
    float* ctx = vm_act(m, m->a_ctx);
    {
        VxMlaAttnArgs a;
        std::memset(&a, 0, sizeof(a));
        a.qabs = qabs;
        a.q32 = q32;
        a.nh = m->nh;
        a.dq = m->dq;
        a.dn = m->dn;
        a.states = states;
        a.s_max = c.max_seq_len;
        a.s_cap = m->s_cap;
        a.splits = m->splits;
        a.rope = vm_rope(m);
        a.qscale = m->scale * 1.4426950408889634f;
        a.cache = cache;
        a.cache_bstride = (uint64_t)m->s_cap * m->R;
        a.part_o = po;
        a.part_ml = pml;
        a.active_mask = mask;
        vx_record_error(vx_launch_mla_attn(a, m->lr, m->dr, batch, st));
    }
    // 8. o_h = W_uv[h] ctx_h; 9. W_o [o_h], split over K; 10. residual
    // o_h goes to W_o as fp16, the rounding the GEMM applies to fp32 activations: half the bytes.
    // One sequence: the W_uv workgroups of head h merge its split partials into ctx_h themselves
    // (one launch less); several: the merge kernel writes ctx first.
    uint16_t* oh16 = (uint16_t*)vm_act(m, m->a_oh);
    if (direct) {
        gemm(L.uv, ctx, m->nh * m->lr, m->lr, 1, nullptr, m->nh * m->dv, m->dv, 1, 0, oh16, 0, nullptr, po, pml,
             m->splits);
    } else {
        vx_record_error(vx_launch_mla_merge(po, pml, m->nh, m->splits, m->lr, ctx, batch, mask, st));
        gemm(L.uv, ctx, m->nh * m->lr, m->lr, 1, nullptr, m->nh * m->dv, m->dv, 1, 0, oh16);
    }
    if (direct) {
        gemm(L.o, oh16, m->nh * m->dv, 0, 0, h, m->H, 0, 1, 0, nullptr, 1);
        return;
    }
    gemm(L.o, oh16, m->nh * m->dv, 0, 0, parts_o, m->H, 0, m->ks_o, pstride_o);
    if (finish) vx_record_error(vx_launch_mla_resid(h, parts_o, m->ks_o, pstride_o, m->H, batch, mask, st));
}

}  // namespace

extern "C" {

void velox_hip_mla_layer_step(VeloxHipMla* m, uint32_t layer, uint32_t batch, uint64_t mask, hipStream_t st) {
    if (!vm_has_buffers(m) || layer >= m->cfg.num_layers || batch == 0 || batch > m->B) {
        vx_record_error(hipErrorInvalidValue);
        return;
    }
    vm_layer(m, layer, batch, mask, false, true, st);
}

void velox_hip_mla_decode_step(VeloxHipMla* m, uint32_t batch, uint64_t mask, hipStream_t st) {
    if (!vm_has_buffers(m) || batch == 0 || batch > m->B) {
        vx_record_error(hipErrorInvalidValue);
        return;
    }
    const uint32_t n = m->cfg.num_layers;
    for (uint32_t l = 0; l < n; ++l) vm_layer(m, l, batch, mask, l > 0, l + 1 == n, st);
}

int velox_hip_mla_arena_bytes(const VeloxHipMla* m, uint64_t* weight_bytes, uint64_t* scale_bytes,
                              uint64_t* norm_bytes, uint64_t* kv_bytes, uint64_t* act_bytes) {
    if (!m) return VELOX_HIP_EINVAL;
    if (weight_bytes) *weight_bytes = m->code_bytes;
    if (scale_bytes) *scale_bytes = m->scale_bytes;
    if (norm_bytes) *norm_bytes = m->o_rope + m->rope_bytes;
    if (kv_bytes) *kv_bytes = m->cache_bytes;
    if (act_bytes) *act_bytes = m->act_bytes;
    return VELOX_HIP_OK;
}

int velox_hip_mla_arena(VeloxHipMla* m, VeloxHipArena* out) {
    if (!vm_has_buffers(m) || !out) return VELOX_HIP_EINVAL;
    out->weight_arena = m->w_codes;
    out->weight_scales = m->w_scales;
    out->norm_weight_arena = m->w_norms;
    out->kv_cache_pool = m->kv;
    out->activation_arena = m->act;
    out->host_pinned_ring = nullptr;  // the attention stack emits no token
    out->quant_mode = VELOX_QUANT_FP8_E4M3;
    out->tied_lm_head = 0;
    std::lock_guard<std::mutex> lk(g_mla_mu);
    for (const auto& r : g_mla_arenas)
        if (r.first == out->weight_arena) return VELOX_HIP_OK;
    g_mla_arenas.emplace_back(out->weight_arena, m);
    return VELOX_HIP_OK;
}

int velox_hip_mla_arena_bind(VeloxHipMla* m, VeloxHipArena* a) {
    if (!m || !a || m->base || vm_has_buffers(m)) return VELOX_HIP_EINVAL;  // a planned handle, bound once
    if (!a->weight_arena || !a->weight_scales || !a->norm_weight_arena || !a->kv_cache_pool || !a->activation_arena ||
        a->quant_mode != VELOX_QUANT_FP8_E4M3)
        return VELOX_HIP_EINVAL;
    {
        std::lock_guard<std::mutex> lk(g_mla_mu);
        for (const auto& r : g_mla_arenas)
            if (r.first == a->weight_arena) return VELOX_HIP_EINVAL;
    }
    m->w_codes = (uint8_t*)a->weight_arena;
    m->w_scales = (uint8_t*)a->weight_scales;
    m->w_norms = (uint8_t*)a->norm_weight_arena;
    m->kv = a->kv_cache_pool;
    m->act = a->activation_arena;
    const hipError_t e = vm_init_regions(m);
    if (e != hipSuccess) {
        m->w_codes = m->w_scales = m->w_norms = m->kv = m->act = nullptr;
        return (int)e;
    }
    std::lock_guard<std::mutex> lk(g_mla_mu);
    g_mla_arenas.emplace_back(a->weight_arena, m);
    return VELOX_HIP_OK;
}

VeloxHipMla* velox_hip_mla_arena_mla(const VeloxHipArena* a) {
    if (!a) return nullptr;
    std::lock_guard<std::mutex> lk(g_mla_mu);
    for (const auto& r : g_mla_arenas)
        if (r.first == a->weight_arena) return r.second;
    return nullptr;
}

int velox_hip_mla_arena_check(const VeloxHipArena* a, const VeloxHipMlaConfig* want) {
    const VeloxHipMla* m = velox_hip_mla_arena_mla(a);
    if (!m || !want) return VELOX_HIP_EINVAL;
    const VeloxHipMlaConfig& c = m->cfg;
    const bool same = c.hidden_dim == want->hidden_dim && c.num_heads == want->num_heads &&
                      c.q_lora_rank == want->q_lora_rank && c.kv_lora_rank == want->kv_lora_rank &&
                      c.qk_nope_dim == want->qk_nope_dim && c.qk_rope_dim == want->qk_rope_dim &&
                      c.v_head_dim == want->v_head_dim && c.kv_norm == want->kv_norm &&
                      c.rms_norm_eps == want->rms_norm_eps && c.rope_theta == want->rope_theta &&
                      c.softmax_scale == want->softmax_scale;
    return same ? VELOX_HIP_OK : VELOX_HIP_EINVAL;
}

void velox_hip_mla_graph_step(VeloxHipArena* ctx, uint64_t mask, hipStream_t st) {
    VeloxHipMla* m = velox_hip_mla_arena_mla(ctx);
    if (!vm_has_buffers(m)) {
        vx_record_error(hipErrorInvalidValue);
        return;
    }
    velox_hip_mla_decode_step(m, m->B, mask, st);
    vx_record_error(vx_launch_mla_advance(vm_states(m), m->B, mask, st));
}

void velox_hip_mla_decode(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t mask, hipStream_t st) {
    VeloxHipMla* m = velox_hip_mla_arena_mla(ctx);
    if (!vm_has_buffers(m)) {
        vx_record_error(hipErrorInvalidValue);
        return;
    }
    vx_record_error(vx_launch_set_state(vm_states(m), step, token_in, st));
    velox_hip_mla_graph_step(ctx, mask, st);
}

// DeepSeek-V3's MLA model with the reference's emitted names (examples/deepseek_v3_mla.vlx; the
// graph step launches its MLA kernel per layer, src/codegen.rs:2980-3003): the attention stack of
// the arena's plan, checked against DeepSeek-V3's dimensions.
static bool vm_is_deepseek(const VeloxHipArena* a) {
    VeloxHipMlaConfig want;
    if (velox_hip_mla_builtin_config("deepseek_v3_mla", 0, 0, &want) == 0 && velox_hip_mla_arena_check(a, &want) == 0)
        return true;
    velox_hip_record_error(VELOX_HIP_EINVAL);  // an arena of another model, as the dense entry points
    return false;
}
void velox_DeepSeek_V3_MLA_decode_graph_step_hip(VeloxHipArena* ctx, uint64_t mask, hipStream_t s) {
    if (vm_is_deepseek(ctx)) velox_hip_mla_graph_step(ctx, mask, s);
}
void velox_DeepSeek_V3_MLA_decode_hip(VeloxHipArena* ctx, uint32_t t, size_t step, uint64_t mask, hipStream_t s) {
    if (vm_is_deepseek(ctx)) velox_hip_mla_decode(ctx, t, step, mask, s);
}
void velox_DeepSeek_V3_MLA_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t mask, hipStream_t s) {
    if (vm_is_deepseek(ctx)) velox_hip_mla_graph_step(ctx, mask, s);
}
void velox_DeepSeek_V3_MLA_prefill_hip(VeloxHipArena* ctx, uint32_t t, size_t step, uint64_t mask, hipStream_t s) {
    if (vm_is_deepseek(ctx)) velox_hip_mla_decode(ctx, t, step, mask, s);
}

double velox_hip_mla_step_bytes(const VeloxHipMla* m, uint32_t batch, uint64_t pos) {
    if (!m) return 0.0;
    const uint64_t per_layer_w = (m->code_bytes + m->scale_bytes + m->norm_bytes) / m->cfg.num_layers;
    const double latent = (double)batch * (double)(pos + 1) * m->R * 2;
    const double act = (double)batch * (2.0 * m->H * 4 + (double)m->nh * m->dq * 4 + 2.0 * m->nh * m->lr * 4 +
                                        (double)m->nh * m->dv * 4);
    return (double)per_layer_w + latent + act;
}

int velox_hip_mla_run(const char* which, uint32_t batch, uint32_t context_len, uint32_t num_layers, uint32_t warmup,
                      uint32_t steps, uint64_t seed, VeloxHipMlaRunReport* rep) {
    if (!rep || batch == 0 || steps == 0) return VELOX_HIP_EINVAL;
    std::memset(rep, 0, sizeof(*rep));
    VeloxHipMlaConfig cfg;
    int rc = velox_hip_mla_builtin_config(which, context_len + 1, batch, &cfg);
    if (rc) return rc;
    const bool stack = num_layers > 1;  // the decode step over a stack of layers, else one layer step
    if (stack) cfg.num_layers = num_layers;
    VeloxHipMla* m = nullptr;
    rc = velox_hip_mla_create(&cfg, &m);
    if (rc) return rc;
    hipStream_t st;
    hipStreamCreate(&st);
    hipEvent_t e0, e1;
    hipEventCreate(&e0);
    hipEventCreate(&e1);
    rc = velox_hip_mla_synthesize(m, seed, 0.02f, 0.0f, st);
    for (uint32_t b = 0; b < batch && !rc; ++b) {
        for (uint32_t l = 0; l < cfg.num_layers && !rc; ++l)
            rc = velox_hip_mla_fill_cache(m, l, b, context_len, seed, 1.0f, st);
        if (!rc) rc = velox_hip_mla_set_position(m, b, context_len, st);
    }
    VeloxHipMlaBuffers buf;
    velox_hip_mla_buffers(m, &buf);
    if (!rc) {  // hidden state N(0, 1)
        rc = (int)vx_launch_fill_normal(buf.hidden, (uint64_t)batch * cfg.hidden_dim, vx_stream(seed, vx_tag(0, 40)),
                                        vx_normal_coef(1.0f), 0.0f, st);
    }
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    (void)velox_hip_last_error();
    if (!rc) {
        hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            if (stack) velox_hip_mla_decode_step(m, batch, 1ULL, st);
            else velox_hip_mla_layer_step(m, 0, batch, 1ULL, st);
            e = hipStreamEndCapture(st, &graph);
        }
        if (e == hipSuccess) e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        rc = e != hipSuccess ? (int)e : velox_hip_last_error();
    }
    if (!rc) {
        for (uint32_t w = 0; w < warmup; ++w) hipGraphLaunch(exec, st);
        rc = (int)hipStreamSynchronize(st);
    }
    if (!rc) {
        const auto w0 = std::chrono::steady_clock::now();
        hipEventRecord(e0, st);
        for (uint32_t s = 0; s < steps; ++s) hipGraphLaunch(exec, st);
        hipEventRecord(e1, st);
        rc = (int)hipStreamSynchronize(st);
        rep->wall_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - w0).count();
        float ms = 0.0f;
        hipEventElapsedTime(&ms, e0, e1);
        rep->us_per_layer = 1000.0 * ms / steps / cfg.num_layers;
        rep->bytes_per_layer = velox_hip_mla_step_bytes(m, batch, context_len);
        rep->hbm_gbps = rep->us_per_layer > 0 ? rep->bytes_per_layer / (rep->us_per_layer * 1e3) : 0.0;
    }
    if (!rc) {
        // the attention kernel alone, event-timed over a few eager launches of the same arguments
        VxMlaAttnArgs a;
        std::memset(&a, 0, sizeof(a));
        a.qabs = vm_act(m, m->a_qabs);
        a.q32 = vm_act(m, m->a_q32);
        a.nh = m->nh;
        a.dq = m->dq;
        a.dn = m->dn;
        a.states = buf.states;
        a.s_max = cfg.max_seq_len;
        a.s_cap = m->s_cap;
        a.splits = m->splits;
        a.rope = vm_rope(m);
        a.qscale = m->scale * 1.4426950408889634f;
        a.cache = buf.latent_cache;
        a.cache_bstride = (uint64_t)m->s_cap * m->R;
        a.part_o = (uint16_t*)vm_act(m, m->a_po);
        a.part_ml = vm_act(m, m->a_pml);
        a.active_mask = 1;
        const int reps = 20;
        hipEventRecord(e0, st);
        for (int i = 0; i < reps; ++i) vx_record_error(vx_launch_mla_attn(a, m->lr, m->dr, batch, st));
        hipEventRecord(e1, st);
        rc = (int)hipStreamSynchronize(st);
        float ms = 0.0f;
        hipEventElapsedTime(&ms, e0, e1);
        rep->attn_us = 1000.0 * ms / reps;
        rep->attn_bytes = (double)batch * (context_len + 1) * m->R * 2;
        if (!rc) rc = velox_hip_last_error();
    }
    rep->status = rc;
    if (exec) hipGraphExecDestroy(exec);
    if (graph) hipGraphDestroy(graph);
    hipEventDestroy(e0);
    hipEventDestroy(e1);
    hipStreamDestroy(st);
    velox_hip_mla_destroy(m);
    return rc;
}

}  // extern "C"
