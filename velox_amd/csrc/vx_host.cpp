// vx_host.cpp -- static memory plan, arena, loaders, the decode-step launcher and the runner.
//
// Host half of the backend. The reference splits this between the Rust planner
// (src/memory_planner.rs:282-488), the emitted host wrapper (src/codegen.rs:2803-3253) and the
// Windows runner (src/runners/velox_cuda_runner.cu:327-726); here it is one C++ library behind
// the C ABI of include/velox_hip.h.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "vx_common.h"

namespace {

// first error of the calling thread (each host thread drives its own streams)
thread_local int g_last_error = 0;

inline int vx_record(hipError_t e) {
    if (e != hipSuccess && g_last_error == 0) g_last_error = (int)e;
    return (int)e;
}

inline uint64_t vx_align(uint64_t x, uint64_t a = 256) { return (x + a - 1) / a * a; }

}  // namespace

// First-error recording shared with the other host translation units.
int vx_record_error(hipError_t e) { return vx_record(e); }

namespace {

struct VxMatPlan {
    uint64_t code_off = 0, scale_off = 0, code_bytes = 0, scale_bytes = 0;
    uint32_t n = 0, k = 0, s = 0, n_tiles = 0, n_iter = 0, paired = 0;
    uint32_t fmt = VX_FMT_Q4;
    // second copy in the MFMA operand layout of the batched GEMM (arenas planned for more than one row)
    bool has_m = false;
    uint64_t mcode_off = 0, mscale_off = 0;
    uint32_t m_tiles = 0, m_grp = 0;
};

struct VxLayerPlan {
    VxMatPlan qkv, o, gate_up, down;
    uint64_t attn_norm = 0, mlp_norm = 0, bias = 0;
};

// K splits of a batched GEMM over the MFMA layout: enough grid rows for about 1024 workgroups (two
// 16-row tiles each, its 4 waves splitting K again), at most 8 (the partials a batched RMSNorm or
// the partial sum folds in) and at most one group of 4 blocks per split.
uint32_t vx_mgemm_ksplit(const VxMatPlan& m) {
    const uint32_t wgs = vx_mgemm_grid(m.m_tiles);
    uint32_t ks = (1024u + wgs - 1u) / wgs;
    if (ks > 8u) ks = 8u;
    if (ks > m.m_grp) ks = m.m_grp;
    return ks ? ks : 1u;
}

// K splits of the QKV GEMM over more than 16 rows (the LDS-shared GEMM, 8 tiles per workgroup): as
// many as keep the grid within one round of 256 workgroups, where a partial second round would add
// a whole workgroup's time (Llama-3-8B QKV at 128 rows: 48 x 6 workgroups 26.6 us, 48 x 5 21.9 us;
// Qwen2.5-7B at 32 sequences: 36 x 8 9.7 us, 36 x 7 8.3 us).
uint32_t vx_pgemm_ksplit(const VxMatPlan& m) {
    const uint32_t wgs = vx_pgemm_grid(m.m_tiles);
    uint32_t ks = wgs ? 256u / wgs : 1u;
    if (ks > 8u) ks = 8u;
    if (ks > m.m_grp) ks = m.m_grp;
    return ks ? ks : 1u;
}

}  // namespace

struct VeloxHipModel {
    VeloxHipModelConfig cfg;
    std::vector<VxLayerPlan> layers;
    VxMatPlan embed, head;
    uint64_t final_norm = 0, rope = 0;
    uint64_t code_bytes = 0, scale_bytes = 0, norm_bytes = 0, kv_bytes = 0, act_bytes = 0, kv_layer_bytes = 0;
    // activation arena offsets (bytes)
    uint64_t a_state = 0, a_plen = 0, a_argmax_counter = 0, a_counters = 0, a_token = 0, a_prompt = 0;
    uint64_t a_h = 0, a_qkv = 0, a_attn = 0, a_act = 0, a_logits = 0, a_part_o = 0, a_part_ml = 0, a_rope_cur = 0;
    uint64_t a_cand_v = 0, a_cand_i = 0;
    uint32_t splits = 1, max_wgs = 2048, s_cap = 0;
    uint32_t head_wgs = 256;  // the single-sequence LM head's grid cap (below)
    bool fused_merge = false;  // o_proj merges the attention partials
    // the single-sequence step's fused QKV + attention launch (vx_qkv_attn.hip), where the plan
    // allows it: fused_splits > 0 attention splits per KV head, fused_p GEMV workgroups per KV head,
    // and its synchronisation words at a_fsync
    uint32_t fused_splits = 0, fused_p = 0;
    uint64_t a_fsync = 0;
    // batched decode (max_batch > 1): per-sequence states, prompts, fp32 residuals, two fp16 GEMM
    // operands, q/k/v, attention partials, logits and LM-head candidates, sequence-major
    uint32_t batch = 1, xw = 0, head_bwgs = 0;
    // rows of the batched region: max(batch, prefill_chunk) (sequences, or positions of a prompt)
    uint32_t rows = 1;
    uint64_t a_prows = 0;  // prefill: the chunk's rows {position, token}
    uint64_t a_bstate = 0, a_bplen = 0, a_bprompt = 0, a_bh = 0, a_bxa = 0, a_bxb = 0, a_bqkv = 0;
    uint64_t a_bpart_o = 0, a_bpart_ml = 0, a_blogits = 0, a_bcand_v = 0, a_bcand_i = 0;
    // K-split partials of the residual GEMMs (o_proj, down): [ksplit][batch][hidden]
    uint64_t a_bpart_r = 0;
    uint32_t ksplit_o = 1, ksplit_down = 1, ksplit_qkv = 1;
    uint32_t ksplit_qkv_wide = 1;  // QKV over more than 16 rows
    // fp16 activation operands of the batched GEMMs (over the MFMA-layout copies): element k of row m
    // at m * x_ld + (k / 32) * x_bs + k % 32, block-major [k / 32][16-row-padded rows][32] (one operand
    // load = 1 KiB contiguous)
    uint32_t x_ld = 0, x_bs = 32;
};

namespace {

// The plan of every live arena, keyed by its weight_arena pointer: VeloxHipArena keeps the
// reference's eight fields (VeloxCudaArena, src/codegen.rs:1032-1041) and nothing else, so the plan
// cannot travel inside it. Arenas enter through velox_hip_arena_create (library-owned buffers) or
// velox_hip_arena_bind (caller-owned buffers, the reference runner's cudaMalloc pattern).
struct VxArenaRec {
    const uint8_t* key = nullptr;   // weight_arena
    const VeloxHipModel* model = nullptr;
    bool xcd_rr = false;            // the device deals workgroup b to XCD b % 8 (fused QKV + attention)
    uint8_t* base = nullptr;        // the one device allocation (owned arenas), else nullptr
    uint32_t* ring = nullptr;       // the mapped host ring (owned arenas), else nullptr
    uint32_t staged_plen = 0;       // prompt length of the last velox_hip_set_prompt
};
std::mutex g_arena_mu;
std::vector<VxArenaRec> g_arenas;

VxArenaRec* vx_rec_locked(const uint8_t* key) {
    for (VxArenaRec& r : g_arenas)
        if (r.key == key) return &r;
    return nullptr;
}

// The plan `a` was created or bound with; nullptr for an unknown arena. xcd_rr (optional): whether
// its device takes the fused QKV + attention launch.
const VeloxHipModel* vx_model(const VeloxHipArena* a, bool* xcd_rr = nullptr) {
    if (xcd_rr) *xcd_rr = false;
    if (!a || !a->weight_arena) return nullptr;
    std::lock_guard<std::mutex> lock(g_arena_mu);
    const VxArenaRec* r = vx_rec_locked(a->weight_arena);
    if (r && xcd_rr) *xcd_rr = r->xcd_rr;
    return r ? r->model : nullptr;
}

// Process-wide switch of the fused QKV + attention launch (velox_hip_set_fused_attention).
std::atomic<int> g_fused_attention{1};

// Lanes per row S: the largest of {32, 16, 8, 4} wasting at most 1/32 of a row's blocks, else the
// one wasting least. Padded blocks are zero and are streamed with the rest, so waste costs
// bandwidth as well as memory; a larger S means fewer rows per wave tile, so more tiles and
// workgroups (Qwen2-72B's down projection, 924 blocks per row: 512 workgroups at S = 32 with 0.4 %
// padding, against 64 workgroups at S = 4, which tiles the row exactly).
uint32_t vx_choose_s(uint32_t nb) {
    const uint32_t cand[4] = {32, 16, 8, 4};
    uint32_t best = 4;
    double best_w = 2.0;
    for (uint32_t s : cand) {
        const uint32_t it = (nb + s - 1) / s;
        const double waste = (double)(it * s - nb) / (double)(it * s);
        if (waste <= 1.0 / 32.0) return s;
        if (waste < best_w) { best_w = waste; best = s; }
    }
    return best;
}

// The weight format of a quant_mode (GGML Q4_0 or the reference's group-64 format in the tiled
// layout, or the reference's fp32 / fp16 rows).
uint32_t vx_fmt_of(uint32_t quant_mode) {
    switch (quant_mode) {
        case VELOX_QUANT_F32: return VX_FMT_F32;
        case VELOX_QUANT_F16: return VX_FMT_F16;
        case VELOX_QUANT_Q4_GROUP64: return VX_FMT_G64;
        default: return VX_FMT_Q4;
    }
}

bool vx_fmt_tiled(uint32_t fmt) { return fmt == VX_FMT_Q4 || fmt == VX_FMT_G64; }

void vx_mat_layout(uint32_t n, uint32_t k, uint32_t s, uint32_t paired, VxMatPlan& p, uint32_t fmt = VX_FMT_Q4) {
    const uint32_t nb = k / 32;
    p.fmt = fmt;
    if (!vx_fmt_tiled(fmt)) {  // row-major [rows][k] (paired: n gate rows, then n up rows), tiles of 4 rows
        p.n = n;
        p.k = k;
        p.s = 0;
        p.paired = paired;
        p.n_tiles = (n + 3) / 4;
        p.n_iter = 0;
        p.code_bytes = (uint64_t)(paired ? 2 * n : n) * k * (fmt == VX_FMT_F32 ? 4 : 2);
        p.scale_bytes = 0;
        return;
    }
    p.n = n;
    p.k = k;
    p.s = s ? s : vx_choose_s(nb);
    p.paired = paired;
    const uint32_t R = 64 / p.s;
    p.n_tiles = paired ? (n + R / 2 - 1) / (R / 2) : (n + R - 1) / R;
    p.n_iter = (nb + p.s - 1) / p.s;
    p.code_bytes = (uint64_t)p.n_tiles * p.n_iter * 64 * 16;
    p.scale_bytes = (uint64_t)p.n_tiles * p.n_iter * 64 * 2;
}

void vx_place(VxMatPlan& p, uint64_t& code_cursor, uint64_t& scale_cursor) {
    p.code_off = code_cursor;
    p.scale_off = scale_cursor;
    code_cursor = vx_align(code_cursor + p.code_bytes);
    scale_cursor = vx_align(scale_cursor + p.scale_bytes);
}

void vx_place_m(VxMatPlan& p, uint64_t& code_cursor, uint64_t& scale_cursor) {
    VxMMat m;
    vx_mmat_shape(p.n, p.k, p.paired, m);
    p.has_m = true;
    p.m_tiles = m.n_tiles;
    p.m_grp = m.n_grp;
    p.mcode_off = code_cursor;
    p.mscale_off = scale_cursor;
    code_cursor = vx_align(code_cursor + vx_mmat_code_bytes(m));
    scale_cursor = vx_align(scale_cursor + vx_mmat_scale_bytes(m));
}

VxMat vx_view(const VeloxHipArena* a, const VxMatPlan& p) {
    VxMat m;
    m.codes = (const uint4*)(a->weight_arena + p.code_off);
    m.scales = (const uint16_t*)(a->weight_scales + p.scale_off);
    m.n = p.n;
    m.k = p.k;
    m.s = p.s;
    m.n_tiles = p.n_tiles;
    m.n_iter = p.n_iter;
    m.paired = p.paired;
    m.fmt = p.fmt;
    return m;
}

VxMMat vx_mview(const VeloxHipArena* a, const VxMatPlan& p) {
    VxMMat m;
    m.codes = (const uint4*)(a->weight_arena + p.mcode_off);
    m.scales = (const uint2*)(a->weight_scales + p.mscale_off);
    m.n = p.n;
    m.k = p.k;
    m.n_tiles = p.m_tiles;
    m.n_grp = p.m_grp;
    m.paired = p.paired;
    return m;
}

// Rebuilds a matrix's MFMA-layout copy from its tiled layout (after a load or synthesis).
hipError_t vx_build_m(const VeloxHipArena* a, const VxMatPlan& p, hipStream_t st) {
    if (!p.has_m) return hipSuccess;
    return vx_launch_mlayout(vx_view(a, p), vx_mview(a, p), st);
}

// KV cache of (layer, sequence): [layer][sequence][K | V][kv head][position][dim] bf16
uint16_t* vx_kv(const VeloxHipModel* M, const VeloxHipArena* a, uint32_t layer, uint32_t seq) {
    return (uint16_t*)(a->kv_cache_pool + M->kv_layer_bytes * ((uint64_t)layer * M->batch + seq));
}

VxMat vx_view_public(const VeloxHipQ4Matrix* q) {
    VxMat m;
    m.codes = (const uint4*)q->codes;
    m.scales = (const uint16_t*)q->scales;
    m.n = q->n;
    m.k = q->k;
    m.s = q->s_lanes;
    m.n_tiles = q->n_tiles;
    m.n_iter = q->n_iter;
    m.paired = q->paired;
    // format 0: GGML Q4_0 blocks; VELOX_QUANT_Q4_GROUP64: group-64 pairs (anything else is refused
    // by the launchers as an unknown format)
    m.fmt = q->format == 0 ? VX_FMT_Q4 : q->format == VELOX_QUANT_Q4_GROUP64 ? VX_FMT_G64 : 0xFFFFFFFFu;
    return m;
}

bool vx_shape_ok(const VeloxHipModelConfig& c) {
    if (c.hidden_dim == 0 || c.num_layers == 0 || c.num_heads == 0 || c.num_kv_heads == 0) return false;
    if (c.hidden_dim % 32 || c.intermediate_dim % 32 || c.max_seq_len == 0 || c.vocab_size == 0) return false;
    if (c.num_heads % c.num_kv_heads) return false;
    if (c.head_dim != 64 && c.head_dim != 128) return false;
    const uint32_t G = c.num_heads / c.num_kv_heads;
    if (c.head_dim == 64 && !(G == 1 || G == 2 || G == 3 || G == 4 || G == 8)) return false;
    if (c.head_dim == 128 && !(G == 1 || G == 2 || G == 4 || G == 7 || G == 8)) return false;
    if (((uint64_t)c.num_heads * c.head_dim) % 32) return false;
    if (c.quant_mode != VELOX_QUANT_GGML_Q4_0 && c.quant_mode != VELOX_QUANT_F32 && c.quant_mode != VELOX_QUANT_F16 &&
        c.quant_mode != VELOX_QUANT_Q4_GROUP64)
        return false;
    // the reference's formats run the single-sequence decode only (the batched GEMMs read Q4_0)
    if (c.quant_mode != VELOX_QUANT_GGML_Q4_0 && (c.max_batch > 1 || c.prefill_chunk > 1)) return false;
    if (c.quant_mode == VELOX_QUANT_F32 || c.quant_mode == VELOX_QUANT_F16) {
        // fp32 activations of a row in LDS
        if (c.hidden_dim > kVxFloatMaxK || c.intermediate_dim > kVxFloatMaxK ||
            (uint64_t)c.num_heads * c.head_dim > kVxFloatMaxK)
            return false;
    }
    if (c.quant_mode == VELOX_QUANT_Q4_GROUP64 &&
        (c.hidden_dim % 64 || c.intermediate_dim % 64 || ((uint64_t)c.num_heads * c.head_dim) % 64))
        return false;  // whole 64-weight groups along every row
    if (c.num_kv_heads > 64 || c.attn_splits > 64 || c.max_batch > 32 || c.prefill_chunk > 128) return false;
    // batched RMSNorm: float4 rows of at most 8192
    if ((c.max_batch > 1 || c.prefill_chunk > 1) && ((c.hidden_dim & 3u) || c.hidden_dim > 8192)) return false;
    if (c.hidden_dim > 32768 || c.intermediate_dim > 32768 || (uint64_t)c.num_heads * c.head_dim > 32768) return false;
    return true;
}

}  // namespace

#ifdef VX_TIMELINE
// Timeline build: the buffer the single-sequence decode step's GEMV and attention launches stamp,
// 1024 workgroup slots of 64 bytes per launch in launch order (see VX_TIMELINE_FIELDS).
static unsigned long long* g_tl = nullptr;
template <class T>
void vx_tl_slot(T& args, uint32_t& n) {
    args.tl = g_tl;
    args.tl_slot = 1024u * n++;
}
extern "C" void velox_hip_timeline_set(unsigned long long* d_buf) { g_tl = d_buf; }
#else
template <class T>
void vx_tl_slot(T&, uint32_t&) {}
#endif

extern "C" {

void velox_hip_record_error(int status) {
    if (!g_last_error) g_last_error = status;
}

void velox_hip_set_fused_attention(int enable) { g_fused_attention.store(enable ? 1 : 0); }

int velox_hip_fused_attention_status(const VeloxHipArena* a, uint32_t* used, uint32_t* errors) {
    bool xcd_rr = false;
    const VeloxHipModel* M = vx_model(a, &xcd_rr);
    if (!M) return VELOX_HIP_EINVAL;
    const bool on = M->fused_splits && xcd_rr && g_fused_attention.load();
    if (used) *used = on ? M->fused_splits : 0u;
    if (errors) {
        *errors = 0;
        if (M->fused_splits) {
            const uint32_t* w = (const uint32_t*)(a->activation_arena + M->a_fsync) + 2u * M->cfg.num_kv_heads * 64u;
            if (hipMemcpy(errors, w, 4, hipMemcpyDeviceToHost) != hipSuccess) return VELOX_HIP_EINVAL;
        }
    }
    return VELOX_HIP_OK;
}

int velox_hip_last_error(void) {
    const int e = g_last_error;
    g_last_error = 0;
    return e;
}

int velox_hip_q4_layout(uint32_t n, uint32_t k, uint32_t s_lanes, uint32_t paired, VeloxHipQ4Matrix* m,
                        uint64_t* code_bytes, uint64_t* scale_bytes) {
    if (!m || k == 0 || k % 32 || n == 0) return VELOX_HIP_EINVAL;
    if (s_lanes && s_lanes != 4 && s_lanes != 8 && s_lanes != 16 && s_lanes != 32 && s_lanes != 64)
        return VELOX_HIP_EINVAL;
    if (paired && s_lanes == 64) return VELOX_HIP_EINVAL;
    VxMatPlan p;
    vx_mat_layout(n, k, s_lanes, paired, p);
    m->n = n;
    m->k = k;
    m->s_lanes = p.s;
    m->n_tiles = p.n_tiles;
    m->n_iter = p.n_iter;
    m->paired = paired;
    m->format = 0;
    if (code_bytes) *code_bytes = p.code_bytes;
    if (scale_bytes) *scale_bytes = p.scale_bytes;
    return VELOX_HIP_OK;
}

// ---------------------------------------------------------------------------------------------
// Plan: the memory_planner's weight cursor + KV sizing + activation layout
// (src/memory_planner.rs:282-474), re-sized for 288 GB of HBM3E on one GPU.
// ---------------------------------------------------------------------------------------------
int velox_hip_model_create(const VeloxHipModelConfig* cfg, VeloxHipModel** out) {
    if (!cfg || !out) return VELOX_HIP_EINVAL;
    if (!vx_shape_ok(*cfg)) return VELOX_HIP_EINVAL;
    VeloxHipModel* M = new VeloxHipModel();
    M->cfg = *cfg;
    const VeloxHipModelConfig& c = M->cfg;
    const uint32_t H = c.hidden_dim, F = c.intermediate_dim, D = c.head_dim;
    const uint32_t qd = c.num_heads * D, kvd = c.num_kv_heads * D;
    uint64_t cc = 0, sc = 0, nc = 0;
    const uint32_t fmt = vx_fmt_of(c.quant_mode);
    M->layers.resize(c.num_layers);
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        VxLayerPlan& L = M->layers[l];
        vx_mat_layout(qd + 2 * kvd, H, 0, 0, L.qkv, fmt);
        vx_mat_layout(H, qd, 0, 0, L.o, fmt);
        vx_mat_layout(F, H, 0, 1, L.gate_up, fmt);
        vx_mat_layout(H, F, 0, 0, L.down, fmt);
        vx_place(L.qkv, cc, sc);
        vx_place(L.o, cc, sc);
        vx_place(L.gate_up, cc, sc);
        vx_place(L.down, cc, sc);
        L.attn_norm = nc;
        nc = vx_align(nc + (uint64_t)H * 4);
        L.mlp_norm = nc;
        nc = vx_align(nc + (uint64_t)H * 4);
        if (c.qkv_bias) {
            L.bias = nc;
            nc = vx_align(nc + (uint64_t)(qd + 2 * kvd) * 4);
        }
    }
    vx_mat_layout(c.vocab_size, H, 0, 0, M->embed, fmt);
    vx_place(M->embed, cc, sc);
    if (c.tied_lm_head) {
        M->head = M->embed;
    } else {
        vx_mat_layout(c.vocab_size, H, 0, 0, M->head, fmt);
        vx_place(M->head, cc, sc);
    }
    // batched rows (sequences of a batched step, or positions of a prefill chunk): every matrix
    // the batched GEMMs read gets its MFMA-layout copy
    const uint32_t brows = c.max_batch > c.prefill_chunk ? c.max_batch : c.prefill_chunk;
    if (brows > 1) {
        for (VxLayerPlan& L : M->layers) {
            vx_place_m(L.qkv, cc, sc);
            vx_place_m(L.o, cc, sc);
            vx_place_m(L.gate_up, cc, sc);
            vx_place_m(L.down, cc, sc);
        }
        vx_place_m(M->head, cc, sc);  // (a tied head: its copy is made from the embedding table)
    }
    M->final_norm = nc;
    nc = vx_align(nc + (uint64_t)H * 4);
    M->rope = nc;
    nc = vx_align(nc + (uint64_t)c.max_seq_len * (D / 2) * 8);
    M->code_bytes = cc;
    M->scale_bytes = sc;
    M->norm_bytes = nc;
    M->batch = c.max_batch > 1 ? c.max_batch : 1u;
    M->s_cap = (c.max_seq_len + 31u) & ~31u;  // V planes hold blocks of 32 positions
    M->kv_layer_bytes = vx_align((uint64_t)2 * c.num_kv_heads * M->s_cap * D * 2);
    M->kv_bytes = M->kv_layer_bytes * c.num_layers * M->batch;  // [layer][sequence]

    // Split-K over the sequence: up to 1024 positions, a power of two (2, 4) of up to 256
    // positions whose (m, l, o) partials the o_proj GEMV merges in its prologue (no extra launch);
    // longer contexts use 8 splits up to 3072 positions, then 256-position splits and the merge
    // kernel. (Llama-3-8B at 385 positions,
    // MFMA attention, measured: 1 split 702.6 tok/s, 2: 712.7, 4: 707.4, 8: 690.3.)
    uint32_t splits = c.attn_splits;
    const bool auto_splits = splits == 0;
    if (!splits) {
        if (c.max_seq_len <= 1024) {
            const uint32_t want = (c.max_seq_len + 255) / 256;
            splits = 2;
            while (splits < want) splits <<= 1;
        } else {
            splits = (c.max_seq_len + 255) / 256;
            // one round of workgroups: the D = 128 kernel holds one 8-wave workgroup per CU, so
            // splits x KV heads above 256 runs a second round (Qwen2-72B at 8216 positions: 33 x 8
            // workgroups span 13.2 us, 32 x 8 span 8.2 us); take 256 / KV heads longer splits while
            // no wave gets more than two 32-position chunks (splits of up to 512 positions)
            const uint32_t one_round = 256u / c.num_kv_heads, min_splits = (c.max_seq_len + 511) / 512;
            if (splits * c.num_kv_heads > 256u && one_round >= min_splits) splits = one_round;
            if (splits > 64) splits = 64;
            // 5-12 splits of 256 (1025-3072 positions): 8 instead, which o_proj merges in its
            // prologue, no merge launch (Qwen2.5-7B, three alternating runs each: 2083 positions
            // 722-724 -> 734-735 tok/s, 1135: 709-712 -> 745-746, 1535: 691 -> 740-741)
            if (splits >= 5 && splits <= 12) splits = 8;
        }
    }
    M->splits = splits;
    M->cfg.attn_splits = splits;  // reported by velox_hip_model_config
    const uint32_t o_groups_per_thread = (qd / 8 + 511) / 512;
    M->fused_merge = (splits == 1 || splits == 2 || splits == 4 || splits == 8) && o_groups_per_thread <= 4;
    // The fused QKV + attention launch: every KV head's q/k/v rows and its A attention splits on one
    // XCD, the splits' partials merged by o_proj (A of 4 up to 512 positions: each wave pair takes one
    // 32-position chunk at the 133-383 positions of the Llama-3-8B bench; 8 up to 2048). Only with the
    // planner's own split count (an explicit attn_splits keeps the separate attention kernel).
    if (auto_splits && c.max_seq_len <= 2048 && o_groups_per_thread <= 4) {
        VxMat qm;
        std::memset(&qm, 0, sizeof(qm));
        const VxMatPlan& q0 = M->layers.empty() ? M->embed : M->layers[0].qkv;
        qm.n = q0.n;
        qm.k = q0.k;
        qm.s = q0.s;
        qm.n_tiles = q0.n_tiles;
        qm.n_iter = q0.n_iter;
        qm.paired = q0.paired;
        qm.fmt = q0.fmt;
        if (!M->layers.empty() && vx_qkv_attn_supported(qm, c.num_heads, c.num_kv_heads, D)) {
            const uint32_t A = c.max_seq_len <= 512 ? 4u : 8u;
            const uint32_t R = 64u / qm.s, th = (c.num_heads / c.num_kv_heads + 2u) * D / R;
            // one 8-wave tile per GEMV wave, all workgroups within one round (two per CU)
            uint32_t P = (th + 7u) / 8u;
            const uint32_t cap = 512u / c.num_kv_heads - A;
            if (P > cap) P = cap;
            M->fused_splits = A;
            M->fused_p = P;
        }
    }
    const uint32_t part_splits = M->fused_splits > splits ? M->fused_splits : splits;
    M->max_wgs = vx_gemv_max_wgs_default();
    // The LM head streams the largest matrix (Llama-3-8B: 296 MB) in one launch: 256 workgroups (one
    // per CU, 131,072 threads) read it faster than 512 (kernel trace of the decode step: 48.1 against
    // 52.3 us; 384: 57.0), as a plain read kernel does (296 MB: 45.5 us at 256 x 512 threads, 49.6 at
    // 512 x 512); the layers' GEMVs keep 512.
    M->head_wgs = M->max_wgs < 256u ? M->max_wgs : 256u;

    uint64_t ac = 0;
    auto take = [&](uint64_t bytes) { const uint64_t o = ac; ac = vx_align(ac + bytes); return o; };
    M->a_state = take(64);
    M->a_plen = take(64);
    M->a_argmax_counter = take(64);
    M->a_counters = take(256);
    M->a_token = take(64);
    M->a_prompt = take((uint64_t)c.max_seq_len * 4);
    M->a_h = take((uint64_t)H * 4);
    M->a_qkv = take((uint64_t)(qd + 2 * kvd) * 4);
    M->a_attn = take((uint64_t)qd * 4);
    M->a_rope_cur = take((uint64_t)D / 2 * 8);
    M->a_act = take((uint64_t)F * 4);
    M->a_logits = take((uint64_t)c.vocab_size * 4);
    M->a_part_o = take((uint64_t)c.num_heads * part_splits * D * 4);
    M->a_part_ml = take((uint64_t)c.num_heads * part_splits * 2 * 4);
    if (M->fused_splits) M->a_fsync = take((uint64_t)kVxQkvSyncWords(c.num_kv_heads) * 4);
    M->a_cand_v = take((uint64_t)65536 * 4);
    M->a_cand_i = take((uint64_t)65536 * 4);
    M->rows = M->batch;
    if (c.prefill_chunk > M->rows) M->rows = c.prefill_chunk;
    if (M->rows > 1) {
        const uint64_t B = M->rows;
        uint32_t xw = H > qd ? H : qd;
        if (F > xw) xw = F;
        M->xw = (xw + 7u) & ~7u;
        M->head_bwgs = vx_mgemm_grid(M->head.m_tiles);
        const uint64_t S = M->batch;  // per-sequence state, prompt length and prompt
        M->a_bstate = take(S * sizeof(VeloxDecodeState));
        M->a_bplen = take(S * 4);
        M->a_bprompt = take(S * c.max_seq_len * 4);
        M->a_bh = take(B * H * 4);
        const uint64_t R16 = (B + 15u) / 16u * 16u;
        M->x_ld = 32u;
        M->x_bs = (uint32_t)(32u * R16);
        M->a_bxa = take(R16 * M->xw * 2);
        M->a_bxb = take(R16 * M->xw * 2);
        M->a_bqkv = take(B * (qd + 2 * kvd) * 4);
        M->a_bpart_o = take(B * c.num_heads * splits * D * 4);
        M->a_bpart_ml = take(B * c.num_heads * splits * 2 * 4);
        M->a_blogits = take(B * c.vocab_size * 4);
        M->a_bcand_v = take(B * M->head_bwgs * 4);
        M->a_bcand_i = take(B * M->head_bwgs * 4);
        // K-split partials: [8][rows][max(hidden, q/k/v width)]
        M->a_bpart_r = take(8 * B * (H > qd + 2 * kvd ? H : qd + 2 * kvd) * 4);
        M->a_prows = take(B * sizeof(VeloxDecodeState));
        M->ksplit_qkv = vx_mgemm_ksplit(M->layers[0].qkv);
        M->ksplit_qkv_wide = vx_pgemm_ksplit(M->layers[0].qkv);
        M->ksplit_o = vx_mgemm_ksplit(M->layers[0].o);
        M->ksplit_down = vx_mgemm_ksplit(M->layers[0].down);
    }
    M->act_bytes = ac;

    const uint64_t budget = c.vram_budget_bytes ? c.vram_budget_bytes : 288ULL * 1000 * 1000 * 1000;
    const uint64_t total = M->code_bytes + M->scale_bytes + M->norm_bytes + M->kv_bytes + M->act_bytes;
    if (total > budget) {  // reference diagnostic E002 (src/memory_planner.rs:398-420)
        delete M;
        return VELOX_HIP_ENOMEM;
    }
    *out = M;
    return VELOX_HIP_OK;
}

void velox_hip_model_destroy(VeloxHipModel* m) { delete m; }

int velox_hip_model_config(const VeloxHipModel* m, VeloxHipModelConfig* out) {
    if (!m || !out) return VELOX_HIP_EINVAL;
    *out = m->cfg;
    return VELOX_HIP_OK;
}

int velox_hip_model_arena_bytes(const VeloxHipModel* m, uint64_t* weight_bytes, uint64_t* scale_bytes,
                                uint64_t* norm_bytes, uint64_t* kv_bytes, uint64_t* act_bytes) {
    if (!m) return VELOX_HIP_EINVAL;
    if (weight_bytes) *weight_bytes = m->code_bytes;
    if (scale_bytes) *scale_bytes = m->scale_bytes;
    if (norm_bytes) *norm_bytes = m->norm_bytes;
    if (kv_bytes) *kv_bytes = m->kv_bytes;
    if (act_bytes) *act_bytes = m->act_bytes;
    return VELOX_HIP_OK;
}

// Algorithmic bytes of one decode step at position pos: every linear weight once (18 B per 32
// weights), the embedding row, the norm gains (and biases), the KV history read for positions
// 0..pos and the new K/V written.
uint64_t velox_hip_model_step_bytes(const VeloxHipModel* m, uint64_t pos) {
    if (!m) return 0;
    const VeloxHipModelConfig& c = m->cfg;
    const uint64_t H = c.hidden_dim, F = c.intermediate_dim, D = c.head_dim;
    const uint64_t qd = (uint64_t)c.num_heads * D, kvd = (uint64_t)c.num_kv_heads * D;
    const uint64_t per_layer_w = (qd + 2 * kvd) * H + H * qd + 2 * F * H + H * F;
    // bytes per weight read: Q4_0 18 per 32, fp32 4, fp16 2
    const uint64_t wnum = c.quant_mode == VELOX_QUANT_F32 ? 4 : c.quant_mode == VELOX_QUANT_F16 ? 2 : 18;
    const uint64_t wden = c.quant_mode == VELOX_QUANT_F32 || c.quant_mode == VELOX_QUANT_F16 ? 1 : 32;
    uint64_t bytes = (per_layer_w * c.num_layers + (uint64_t)c.vocab_size * H) / wden * wnum;
    bytes += H / wden * wnum;                               // embedding row
    bytes += (2 * (uint64_t)c.num_layers + 1) * H * 4;      // norm gains
    if (c.qkv_bias) bytes += (uint64_t)c.num_layers * (qd + 2 * kvd) * 4;
    const uint64_t p = pos < c.max_seq_len ? pos : c.max_seq_len - 1;
    bytes += (uint64_t)c.num_layers * 2 * kvd * 2 * (p + 1);  // KV read (bf16)
    bytes += (uint64_t)c.num_layers * 2 * kvd * 2;            // KV write
    return bytes;
}

uint64_t velox_hip_model_logits_offset(const VeloxHipModel* m) { return m ? m->a_logits : 0; }
uint64_t velox_hip_model_hidden_offset(const VeloxHipModel* m) { return m ? m->a_h : 0; }

// ---------------------------------------------------------------------------------------------
// Arena
// ---------------------------------------------------------------------------------------------
namespace {

// Clears every region of a planned arena (tile padding, KV pool, state, counters, prompt length)
// and uploads the RoPE table: cos/sin of pos * theta^(-2j/D) evaluated exactly as
// src/runtime.rs:756-760 (fp32 powf, product and sin/cos), once at startup instead of per token.
hipError_t vx_arena_init(const VeloxHipModel* m, const VeloxHipArena* a) {
    hipError_t e = hipMemset((void*)a->weight_arena, 0, m->code_bytes);
    if (e == hipSuccess) e = hipMemset((void*)a->weight_scales, 0, m->scale_bytes);
    if (e == hipSuccess) e = hipMemset((void*)a->norm_weight_arena, 0, m->norm_bytes);
    if (e == hipSuccess) e = hipMemset(a->kv_cache_pool, 0, m->kv_bytes);
    if (e == hipSuccess) e = hipMemset(a->activation_arena, 0, m->act_bytes);
    if (e != hipSuccess) return e;
    std::memset(a->host_pinned_ring, 0, (size_t)VELOX_HIP_RING_SIZE * 4u * m->batch);
    const VeloxHipModelConfig& c = m->cfg;
    const uint32_t half = c.head_dim / 2;
    std::vector<float> rope((size_t)c.max_seq_len * half * 2);
    for (uint32_t p = 0; p < c.max_seq_len; ++p)
        for (uint32_t j = 0; j < half; ++j) {
            const float freq = 1.0f / powf(c.rope_theta, (float)(2 * j) / (float)c.head_dim);
            const float angle = (float)p * freq;
            rope[((size_t)p * half + j) * 2] = cosf(angle);
            rope[((size_t)p * half + j) * 2 + 1] = sinf(angle);
        }
    return hipMemcpy((void*)(a->norm_weight_arena + m->rope), rope.data(), rope.size() * 4, hipMemcpyHostToDevice);
}

int vx_register(const VeloxHipModel* m, const VeloxHipArena* a, uint8_t* base, uint32_t* ring) {
    // (a device check with launches of its own: before the registry's lock)
    const bool xcd_rr = m->fused_splits ? vx_xcd_roundrobin_ok() : false;
    std::lock_guard<std::mutex> lock(g_arena_mu);
    if (vx_rec_locked(a->weight_arena)) return VELOX_HIP_EINVAL;  // already an arena
    VxArenaRec r;
    r.key = a->weight_arena;
    r.model = m;
    r.xcd_rr = xcd_rr;
    r.base = base;
    r.ring = ring;
    g_arenas.push_back(r);
    return VELOX_HIP_OK;
}

}  // namespace

// One device allocation split into the reference's regions (weights, scales, norms + RoPE table,
// KV pool, activations, each 256-byte aligned) plus the mapped host ring.
int velox_hip_arena_create(const VeloxHipModel* m, VeloxHipArena* out) {
    if (!m || !out) return VELOX_HIP_EINVAL;
    std::memset(out, 0, sizeof(*out));
    const uint64_t o_scale = vx_align(m->code_bytes), o_norm = o_scale + vx_align(m->scale_bytes);
    const uint64_t o_kv = o_norm + vx_align(m->norm_bytes), o_act = o_kv + vx_align(m->kv_bytes);
    const uint64_t total = o_act + vx_align(m->act_bytes);
    uint8_t* base = nullptr;
    uint32_t* ring = nullptr;
    hipError_t e = hipMalloc((void**)&base, total);
    // one ring of VELOX_HIP_RING_SIZE tokens per sequence (sequence 0 is the single-sequence ring)
    const size_t ring_bytes = (size_t)VELOX_HIP_RING_SIZE * 4u * m->batch;
    if (e == hipSuccess) e = hipHostMalloc((void**)&ring, ring_bytes, hipHostMallocMapped);
    VeloxHipArena a;
    std::memset(&a, 0, sizeof(a));
    if (e == hipSuccess) {
        a.weight_arena = base;
        a.weight_scales = base + o_scale;
        a.norm_weight_arena = base + o_norm;
        a.kv_cache_pool = base + o_kv;
        a.activation_arena = base + o_act;
        a.host_pinned_ring = ring;
        a.quant_mode = m->cfg.quant_mode;
        a.tied_lm_head = m->cfg.tied_lm_head;
        e = vx_arena_init(m, &a);
    }
    int rc = (int)e;
    if (rc == VELOX_HIP_OK) rc = vx_register(m, &a, base, ring);
    if (rc != VELOX_HIP_OK) {
        hipFree(base);
        if (ring) hipHostFree(ring);
        return rc;
    }
    *out = a;
    return VELOX_HIP_OK;
}

int velox_hip_arena_bind(const VeloxHipModel* m, VeloxHipArena* a) {
    if (!m || !a || !a->weight_arena || !a->weight_scales || !a->norm_weight_arena || !a->kv_cache_pool ||
        !a->activation_arena || !a->host_pinned_ring)
        return VELOX_HIP_EINVAL;
    if (a->quant_mode != m->cfg.quant_mode || a->tied_lm_head != m->cfg.tied_lm_head) return VELOX_HIP_EINVAL;
    const hipError_t e = vx_arena_init(m, a);
    if (e != hipSuccess) return (int)e;
    return vx_register(m, a, nullptr, nullptr);
}

const VeloxHipModel* velox_hip_arena_model(const VeloxHipArena* a) { return vx_model(a); }

int velox_hip_arena_destroy(VeloxHipArena* a) {
    if (!a || !a->weight_arena) return VELOX_HIP_EINVAL;
    VxArenaRec r;
    {
        std::lock_guard<std::mutex> lock(g_arena_mu);
        VxArenaRec* p = vx_rec_locked(a->weight_arena);
        if (!p) return VELOX_HIP_EINVAL;
        r = *p;
        g_arenas.erase(g_arenas.begin() + (p - g_arenas.data()));
    }
    // caller-owned buffers (velox_hip_arena_bind) stay with the caller
    if (r.base) hipFree(r.base);
    if (r.ring) hipHostFree(r.ring);
    std::memset(a, 0, sizeof(*a));
    return VELOX_HIP_OK;
}

// ---------------------------------------------------------------------------------------------
// Loaders
// ---------------------------------------------------------------------------------------------
namespace {
// Target matrix, first logical row, pair part and row count of a weight kind.
bool vx_target(const VeloxHipModel* M, int kind, uint32_t layer, const VxMatPlan** mp, uint32_t* row0,
               uint32_t* pair, uint32_t* rows, uint32_t* cols) {
    const VeloxHipModelConfig& c = M->cfg;
    const uint32_t qd = c.num_heads * c.head_dim, kvd = c.num_kv_heads * c.head_dim;
    *pair = 0;
    *row0 = 0;
    if (kind == VELOX_T_EMBED) { *mp = &M->embed; *rows = c.vocab_size; *cols = c.hidden_dim; return true; }
    if (kind == VELOX_T_HEAD) {
        if (c.tied_lm_head) return false;
        *mp = &M->head; *rows = c.vocab_size; *cols = c.hidden_dim; return true;
    }
    if (layer >= c.num_layers) return false;
    const VxLayerPlan& L = M->layers[layer];
    switch (kind) {
        case VELOX_T_Q: *mp = &L.qkv; *rows = qd; *cols = c.hidden_dim; return true;
        case VELOX_T_K: *mp = &L.qkv; *row0 = qd; *rows = kvd; *cols = c.hidden_dim; return true;
        case VELOX_T_V: *mp = &L.qkv; *row0 = qd + kvd; *rows = kvd; *cols = c.hidden_dim; return true;
        case VELOX_T_O: *mp = &L.o; *rows = c.hidden_dim; *cols = qd; return true;
        case VELOX_T_GATE: *mp = &L.gate_up; *rows = c.intermediate_dim; *cols = c.hidden_dim; return true;
        case VELOX_T_UP: *mp = &L.gate_up; *pair = 1; *rows = c.intermediate_dim; *cols = c.hidden_dim; return true;
        case VELOX_T_DOWN: *mp = &L.down; *rows = c.hidden_dim; *cols = c.intermediate_dim; return true;
        default: return false;
    }
}

bool vx_vec_target(const VeloxHipModel* M, int kind, uint32_t layer, uint64_t* off, uint64_t* count) {
    const VeloxHipModelConfig& c = M->cfg;
    const uint32_t qd = c.num_heads * c.head_dim, kvd = c.num_kv_heads * c.head_dim;
    if (kind == VELOX_T_FINAL_NORM) { *off = M->final_norm; *count = c.hidden_dim; return true; }
    if (layer >= c.num_layers) return false;
    const VxLayerPlan& L = M->layers[layer];
    switch (kind) {
        case VELOX_T_ATTN_NORM: *off = L.attn_norm; *count = c.hidden_dim; return true;
        case VELOX_T_MLP_NORM: *off = L.mlp_norm; *count = c.hidden_dim; return true;
        case VELOX_T_BQ: if (!c.qkv_bias) return false; *off = L.bias; *count = qd; return true;
        case VELOX_T_BK: if (!c.qkv_bias) return false; *off = L.bias + (uint64_t)qd * 4; *count = kvd; return true;
        case VELOX_T_BV:
            if (!c.qkv_bias) return false;
            *off = L.bias + (uint64_t)(qd + kvd) * 4; *count = kvd; return true;
        default: return false;
    }
}
}  // namespace

int velox_hip_arena_matrix(const VeloxHipArena* a, int kind, uint32_t layer, VeloxHipQ4Matrix* out, uint32_t* row0) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || !out) return VELOX_HIP_EINVAL;
    const VxMatPlan* mp;
    uint32_t r0, pair, rows, cols;
    if (kind == VELOX_T_HEAD && M->cfg.tied_lm_head) kind = VELOX_T_EMBED;
    if (!vx_target(M, kind, layer, &mp, &r0, &pair, &rows, &cols)) return VELOX_HIP_EINVAL;
    if (!vx_fmt_tiled(mp->fmt)) return VELOX_HIP_EINVAL;  // a tiled view; fp32 / fp16 rows have none
    out->codes = (void*)(a->weight_arena + mp->code_off);
    out->scales = (void*)(a->weight_scales + mp->scale_off);
    out->n = mp->n;
    out->k = mp->k;
    out->s_lanes = mp->s;
    out->n_tiles = mp->n_tiles;
    out->n_iter = mp->n_iter;
    out->paired = mp->paired;
    out->format = mp->fmt == VX_FMT_G64 ? VELOX_QUANT_Q4_GROUP64 : 0u;
    if (row0) *row0 = pair ? mp->n : r0;  // paired: up rows follow the n gate rows when dequantized
    return VELOX_HIP_OK;
}

int velox_hip_arena_vector(const VeloxHipArena* a, int kind, uint32_t layer, const float** out, uint64_t* count) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || !out) return VELOX_HIP_EINVAL;
    uint64_t off, n;
    if (!vx_vec_target(M, kind, layer, &off, &n)) return VELOX_HIP_EINVAL;
    *out = (const float*)(a->norm_weight_arena + off);
    if (count) *count = n;
    return VELOX_HIP_OK;
}

int velox_hip_load_q4_0(VeloxHipArena* a, int kind, uint32_t layer, const void* blocks, uint64_t nbytes,
                        hipStream_t stream) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || !blocks) return VELOX_HIP_EINVAL;
    const VxMatPlan* mp;
    uint32_t row0, pair, rows, cols;
    if (!vx_target(M, kind, layer, &mp, &row0, &pair, &rows, &cols)) return VELOX_HIP_EINVAL;
    if (mp->fmt != VX_FMT_Q4) return VELOX_HIP_EINVAL;  // GGML blocks load into GGML Q4_0 arenas only
    if (nbytes != (uint64_t)rows * (cols / 32) * 18) return VELOX_HIP_ESHAPE;
    void* staging = nullptr;
    hipError_t e = hipMalloc(&staging, nbytes);
    if (e == hipSuccess) e = hipMemcpyAsync(staging, blocks, nbytes, hipMemcpyHostToDevice, stream);
    if (e == hipSuccess) e = vx_launch_repack(staging, rows, row0, pair, vx_view(a, *mp), stream);
    if (e == hipSuccess) e = vx_build_m(a, *mp, stream);
    if (e == hipSuccess && kind == VELOX_T_EMBED && M->cfg.tied_lm_head) e = vx_build_m(a, M->head, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    hipFree(staging);
    return (int)e;
}

int velox_hip_load_rows(VeloxHipArena* a, int kind, uint32_t layer, const void* rows_data, uint64_t nbytes,
                        hipStream_t stream) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || !rows_data) return VELOX_HIP_EINVAL;
    const VxMatPlan* mp;
    uint32_t row0, pair, rows, cols;
    if (!vx_target(M, kind, layer, &mp, &row0, &pair, &rows, &cols)) return VELOX_HIP_EINVAL;
    if (mp->fmt == VX_FMT_Q4) return VELOX_HIP_EINVAL;  // Q4_0 arenas load blocks (velox_hip_load_q4_0)
    const uint64_t elt = mp->fmt == VX_FMT_F16 ? 2 : 4;
    if (nbytes != (uint64_t)rows * cols * elt) return VELOX_HIP_ESHAPE;
    if (mp->fmt == VX_FMT_G64) {
        // fp32 rows converted on the device, as the reference runner's stream_tensor_converted
        // does for quant_mode 2 (velox_cuda_runner.cu:174-197)
        void* staging = nullptr;
        hipError_t e = hipMalloc(&staging, nbytes);
        if (e == hipSuccess) e = hipMemcpyAsync(staging, rows_data, nbytes, hipMemcpyHostToDevice, stream);
        if (e == hipSuccess) e = vx_launch_g64_from_rows((const float*)staging, rows, row0, pair, vx_view(a, *mp), stream);
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        hipFree(staging);
        return (int)e;
    }
    const uint64_t first = (uint64_t)(pair ? mp->n : 0) + row0;  // paired: up rows follow the n gate rows
    hipError_t e = hipMemcpyAsync((void*)(a->weight_arena + mp->code_off + first * cols * elt), rows_data, nbytes,
                                  hipMemcpyHostToDevice, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    return (int)e;
}

int velox_hip_load_tensor(VeloxHipArena* a, int kind, uint32_t layer, const void* data, uint64_t nbytes,
                          uint32_t dtype, hipStream_t stream) {
    const VeloxHipModel* M = a ? vx_model(a) : nullptr;
    if (!M || !data) return VELOX_HIP_EINVAL;
    if (dtype > VELOX_DT_BF16) return VELOX_HIP_EDTYPE;
    const uint64_t elt = dtype == VELOX_DT_F32 ? 4 : 2;
    uint64_t voff, vn;
    if (vx_vec_target(M, kind, layer, &voff, &vn)) {
        if (nbytes != vn * elt) return VELOX_HIP_ESHAPE;
        float* dst = (float*)(a->norm_weight_arena + voff);
        hipError_t e = hipSuccess;
        if (dtype == VELOX_DT_F32) {
            e = hipMemcpyAsync(dst, data, nbytes, hipMemcpyHostToDevice, stream);
        } else {
            void* staging = nullptr;
            e = hipMalloc(&staging, nbytes);
            if (e == hipSuccess) e = hipMemcpyAsync(staging, data, nbytes, hipMemcpyHostToDevice, stream);
            if (e == hipSuccess) e = vx_launch_convert(staging, dtype, dst, VX_DT_F32, vn, stream);
            if (e == hipSuccess) e = hipStreamSynchronize(stream);
            hipFree(staging);
        }
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
        return (int)e;
    }
    const VxMatPlan* mp;
    uint32_t row0, pair, rows, cols;
    if (kind == VELOX_T_HEAD && M->cfg.tied_lm_head) return VELOX_HIP_EINVAL;  // the head is the embedding
    if (!vx_target(M, kind, layer, &mp, &row0, &pair, &rows, &cols)) return VELOX_HIP_EINVAL;
    if (nbytes != (uint64_t)rows * cols * elt) return VELOX_HIP_ESHAPE;
    // Rows go through the device in chunks of at most 64 MiB of fp32 (the reference stages 64 MiB
    // chunks too, velox_cuda_runner.cu:172-197): upload as stored, widen or narrow on the device,
    // and for the 4-bit formats quantize there into the tiled layout.
    const uint64_t row_f32 = (uint64_t)cols * 4;
    const uint32_t chunk = (uint32_t)std::max<uint64_t>(1, std::min<uint64_t>(rows, (64ull << 20) / row_f32));
    const bool quant = mp->fmt == VX_FMT_Q4 || mp->fmt == VX_FMT_G64;
    const bool direct = mp->fmt == VX_FMT_F32 && dtype == VELOX_DT_F32;
    void *src_st = nullptr, *f32_st = nullptr, *blk_st = nullptr;
    hipError_t e = hipSuccess;
    if (!direct) e = hipMalloc(&src_st, (uint64_t)chunk * cols * elt);
    if (e == hipSuccess && quant && dtype != VELOX_DT_F32) e = hipMalloc(&f32_st, (uint64_t)chunk * row_f32);
    if (e == hipSuccess && mp->fmt == VX_FMT_Q4) e = hipMalloc(&blk_st, (uint64_t)chunk * (cols / 32) * 18);
    const uint64_t first = (uint64_t)(pair ? mp->n : 0) + row0;  // row-major formats: up rows follow the gate rows
    uint8_t* rows_dst = (uint8_t*)a->weight_arena + mp->code_off;
    for (uint32_t r = 0; r < rows && e == hipSuccess; r += chunk) {
        const uint32_t n = std::min(chunk, rows - r);
        const uint64_t cnt = (uint64_t)n * cols;
        const uint8_t* src = (const uint8_t*)data + (uint64_t)r * cols * elt;
        if (direct) {
            e = hipMemcpyAsync(rows_dst + (first + r) * row_f32, src, cnt * 4, hipMemcpyHostToDevice, stream);
            continue;
        }
        e = hipMemcpyAsync(src_st, src, cnt * elt, hipMemcpyHostToDevice, stream);
        if (e != hipSuccess) break;
        if (mp->fmt == VX_FMT_F32 || mp->fmt == VX_FMT_F16) {
            const uint64_t out_elt = mp->fmt == VX_FMT_F32 ? 4 : 2;
            e = vx_launch_convert(src_st, dtype, rows_dst + (first + r) * cols * out_elt,
                                  mp->fmt == VX_FMT_F32 ? VX_DT_F32 : VX_DT_F16, cnt, stream);
        } else {
            const float* x = (const float*)src_st;
            if (dtype != VELOX_DT_F32) {
                e = vx_launch_convert(src_st, dtype, f32_st, VX_DT_F32, cnt, stream);
                x = (const float*)f32_st;
            }
            if (e == hipSuccess && mp->fmt == VX_FMT_G64)
                e = vx_launch_g64_from_rows(x, n, row0 + r, pair, vx_view(a, *mp), stream);
            if (e == hipSuccess && mp->fmt == VX_FMT_Q4) {
                e = vx_launch_quantize(x, n, cols, blk_st, stream);
                if (e == hipSuccess) e = vx_launch_repack(blk_st, n, row0 + r, pair, vx_view(a, *mp), stream);
            }
        }
        // the staging buffers are reused by the next chunk
        if (e == hipSuccess) e = hipStreamSynchronize(stream);
    }
    if (e == hipSuccess && mp->fmt == VX_FMT_Q4) e = vx_build_m(a, *mp, stream);
    if (e == hipSuccess && mp->fmt == VX_FMT_Q4 && kind == VELOX_T_EMBED && M->cfg.tied_lm_head) e = vx_build_m(a, M->head, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    hipFree(src_st);
    hipFree(f32_st);
    hipFree(blk_st);
    return (int)e;
}

int velox_hip_load_f32(VeloxHipArena* a, int kind, uint32_t layer, const float* data, uint64_t count,
                       hipStream_t stream) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || !data) return VELOX_HIP_EINVAL;
    uint64_t off, n;
    if (!vx_vec_target(M, kind, layer, &off, &n)) return VELOX_HIP_EINVAL;
    if (count != n) return VELOX_HIP_ESHAPE;
    hipError_t e = hipMemcpyAsync((void*)(a->norm_weight_arena + off), data, n * 4, hipMemcpyHostToDevice, stream);
    if (e == hipSuccess) e = hipStreamSynchronize(stream);
    return (int)e;
}

int velox_hip_synthesize_model(VeloxHipArena* a, uint64_t seed, float sigma, float norm_sigma, hipStream_t st) {
    const VeloxHipModel* M = vx_model(a);
    if (!M) return VELOX_HIP_EINVAL;
    const VeloxHipModelConfig& c = M->cfg;
    const float coef = vx_normal_coef(sigma), ncoef = norm_sigma == 0.0f ? 0.0f : vx_normal_coef(norm_sigma);
    hipError_t e = hipSuccess;
    auto mat = [&](int kind, uint32_t layer) {
        if (e != hipSuccess) return;
        const VxMatPlan* mp;
        uint32_t row0, pair, rows, cols;
        if (!vx_target(M, kind, layer, &mp, &row0, &pair, &rows, &cols)) return;
        const uint64_t stream = vx_stream(seed, vx_tag(layer, kind));
        if (mp->fmt == VX_FMT_Q4) {
            e = vx_launch_synth_q4(vx_view(a, *mp), rows, row0, pair, stream, coef, st);
            return;
        }
        if (mp->fmt == VX_FMT_G64) {  // the fp32 model's seeded values, quantized to group-64
            e = vx_launch_synth_g64(vx_view(a, *mp), rows, row0, pair, stream, coef, st);
            return;
        }
        // fp32 / fp16 rows: the seeded values themselves (rounded to fp16), row-major
        const uint64_t first = (uint64_t)(pair ? mp->n : 0) + row0, count = (uint64_t)rows * cols;
        uint8_t* dst = (uint8_t*)a->weight_arena + mp->code_off;
        e = mp->fmt == VX_FMT_F32
                ? vx_launch_fill_normal((float*)dst + first * cols, count, stream, coef, 0.0f, st)
                : vx_launch_fill_normal_f16((uint16_t*)dst + first * cols, count, stream, coef, 0.0f, st);
    };
    auto vec = [&](int kind, uint32_t layer, float cf, float mean) {
        if (e != hipSuccess) return;
        uint64_t off, n;
        if (!vx_vec_target(M, kind, layer, &off, &n)) return;
        e = vx_launch_fill_normal((float*)(a->norm_weight_arena + off), n, vx_stream(seed, vx_tag(layer, kind)), cf,
                                  mean, st);
    };
    mat(VELOX_T_EMBED, 0);
    if (!c.tied_lm_head) mat(VELOX_T_HEAD, 0);
    vec(VELOX_T_FINAL_NORM, 0, ncoef, 1.0f);
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        for (int k : {VELOX_T_Q, VELOX_T_K, VELOX_T_V, VELOX_T_O, VELOX_T_GATE, VELOX_T_UP, VELOX_T_DOWN}) mat(k, l);
        vec(VELOX_T_ATTN_NORM, l, ncoef, 1.0f);
        vec(VELOX_T_MLP_NORM, l, ncoef, 1.0f);
        if (c.qkv_bias) {
            vec(VELOX_T_BQ, l, coef, 0.0f);
            vec(VELOX_T_BK, l, coef, 0.0f);
            vec(VELOX_T_BV, l, coef, 0.0f);
        }
    }
    for (const VxLayerPlan& L : M->layers)
        for (const VxMatPlan* p : {&L.qkv, &L.o, &L.gate_up, &L.down})
            if (e == hipSuccess) e = vx_build_m(a, *p, st);
    if (e == hipSuccess) e = vx_build_m(a, M->head, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return (int)e;
}

int velox_hip_fill_kv(VeloxHipArena* a, uint32_t layer, uint32_t n_pos, uint64_t seed, float sigma, hipStream_t st) {
    const VeloxHipModel* M = vx_model(a);
    if (!M) return VELOX_HIP_EINVAL;
    const VeloxHipModelConfig& c = M->cfg;
    if (layer >= c.num_layers || n_pos > c.max_seq_len) return VELOX_HIP_EINVAL;
    uint16_t* base = vx_kv(M, a, layer, 0);
    hipError_t e = vx_launch_fill_kv(base, c.num_kv_heads, M->s_cap, c.head_dim, n_pos,
                                     vx_stream(seed, vx_tag(layer, VX_TAG_KV_K)),
                                     vx_stream(seed, vx_tag(layer, VX_TAG_KV_V)), vx_normal_coef(sigma), st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return (int)e;
}

// ---------------------------------------------------------------------------------------------
// Decode state / prompt
// ---------------------------------------------------------------------------------------------
int velox_hip_set_prompt(VeloxHipArena* a, const uint32_t* tokens, uint32_t n, hipStream_t st) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || (n && !tokens)) return VELOX_HIP_EINVAL;
    if (n > M->cfg.max_seq_len) return VELOX_HIP_EINVAL;
    hipError_t e = hipSuccess;
    if (n) e = hipMemcpyAsync(a->activation_arena + M->a_prompt, tokens, (size_t)n * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(a->activation_arena + M->a_plen, &n, 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    if (e == hipSuccess) {
        std::lock_guard<std::mutex> lock(g_arena_mu);
        if (VxArenaRec* r = vx_rec_locked(a->weight_arena)) r->staged_plen = n;
    }
    return (int)e;
}

int velox_hip_set_state(VeloxHipArena* a, uint64_t step, uint32_t token, hipStream_t st) {
    const VeloxHipModel* M = vx_model(a);
    if (!M) return VELOX_HIP_EINVAL;
    return (int)vx_launch_set_state((VeloxDecodeState*)(a->activation_arena + M->a_state), step, token, st);
}

int velox_hip_get_state(const VeloxHipArena* a, VeloxDecodeState* out, hipStream_t st) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || !out) return VELOX_HIP_EINVAL;
    hipError_t e = hipMemcpyAsync(out, a->activation_arena + M->a_state, sizeof(*out), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return (int)e;
}

// ---------------------------------------------------------------------------------------------
// Batched decode of independent sequences (arena planned with max_batch > 1)
// ---------------------------------------------------------------------------------------------
int velox_hip_batch_set_prompt(VeloxHipArena* a, uint32_t seq, const uint32_t* tokens, uint32_t n, hipStream_t st) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || M->batch < 2 || seq >= M->batch || (n && !tokens)) return VELOX_HIP_EINVAL;
    if (n > M->cfg.max_seq_len) return VELOX_HIP_EINVAL;
    hipError_t e = hipSuccess;
    if (n)
        e = hipMemcpyAsync(a->activation_arena + M->a_bprompt + (size_t)seq * M->cfg.max_seq_len * 4, tokens,
                           (size_t)n * 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(a->activation_arena + M->a_bplen + (size_t)seq * 4, &n, 4, hipMemcpyHostToDevice, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return (int)e;
}

int velox_hip_batch_set_state(VeloxHipArena* a, uint32_t seq, uint64_t step, uint32_t token, hipStream_t st) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || M->batch < 2 || seq >= M->batch) return VELOX_HIP_EINVAL;
    VeloxDecodeState* s = (VeloxDecodeState*)(a->activation_arena + M->a_bstate) + seq;
    return (int)vx_launch_set_state(s, step, token, st);
}

int velox_hip_batch_get_state(const VeloxHipArena* a, uint32_t seq, VeloxDecodeState* out, hipStream_t st) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || M->batch < 2 || seq >= M->batch || !out) return VELOX_HIP_EINVAL;
    hipError_t e = hipMemcpyAsync(out, a->activation_arena + M->a_bstate + (size_t)seq * sizeof(*out),
                                  sizeof(*out), hipMemcpyDeviceToHost, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return (int)e;
}

int velox_hip_fill_kv_seq(VeloxHipArena* a, uint32_t layer, uint32_t seq, uint32_t n_pos, uint64_t seed, float sigma,
                          hipStream_t st) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || seq >= M->batch) return VELOX_HIP_EINVAL;
    const VeloxHipModelConfig& c = M->cfg;
    if (layer >= c.num_layers || n_pos > c.max_seq_len) return VELOX_HIP_EINVAL;
    // sequence 0 is velox_hip_fill_kv's context; others draw from streams of a sequence-tagged seed
    const uint64_t sseed = seed + (uint64_t)seq * 0x9E3779B97F4A7C15ULL;
    hipError_t e = vx_launch_fill_kv(vx_kv(M, a, layer, seq), c.num_kv_heads, M->s_cap, c.head_dim, n_pos,
                                     vx_stream(sseed, vx_tag(layer, VX_TAG_KV_K)),
                                     vx_stream(sseed, vx_tag(layer, VX_TAG_KV_V)), vx_normal_coef(sigma), st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    return (int)e;
}

int velox_hip_model_batch_layout(const VeloxHipModel* m, uint32_t* max_batch, uint64_t* logits_offset,
                                 uint64_t* hidden_offset) {
    if (!m) return VELOX_HIP_EINVAL;
    if (max_batch) *max_batch = m->batch;
    if (logits_offset) *logits_offset = m->a_blogits;
    if (hidden_offset) *hidden_offset = m->a_bh;
    return VELOX_HIP_OK;
}

uint64_t velox_hip_model_batch_step_bytes(const VeloxHipModel* m, uint32_t batch, uint64_t pos) {
    if (!m || batch == 0) return 0;
    const VeloxHipModelConfig& c = m->cfg;
    const uint64_t kvd = (uint64_t)c.num_kv_heads * c.head_dim;
    const uint64_t p = pos < c.max_seq_len ? pos : c.max_seq_len - 1;
    // weights and norms once; per further sequence its embedding row and its own KV read + write
    const uint64_t per_seq = (uint64_t)c.hidden_dim / 32 * 18 + (uint64_t)c.num_layers * 2 * kvd * 2 * (p + 2);
    return velox_hip_model_step_bytes(m, pos) + (uint64_t)(batch - 1) * per_seq;
}

namespace {

// One forward over rows 0 .. n-1 of the batched region through the LM head's argmax candidates;
// rows[r] holds row r's position and input token. Decode: row b is sequence b with its own KV
// cache, which the attention kernel appends the new position to. Prefill: the rows are
// consecutive positions of sequence 0, whose K/V rows all go into its cache before the attention,
// which then attends over [0, position] of every row. Launches: embed, L x [norm, QKV, (prefill:
// K/V rows,) attention, merge, o_proj + residual, norm, gate/up + SwiGLU, down + residual], norm,
// LM head.
void vx_rows_forward(const VeloxHipModel* M, VeloxHipArena* A, const VeloxDecodeState* rows, uint32_t n, uint64_t mask,
                     bool prefill, uint32_t max_len, hipStream_t st) {
    const VeloxHipModelConfig& c = M->cfg;
    uint8_t* act = A->activation_arena;
    const uint32_t H = c.hidden_dim, D = c.head_dim, qd = c.num_heads * D, kvd = c.num_kv_heads * D;
    const float* nrm = (const float*)A->norm_weight_arena;
    auto vecp = [&](uint64_t off) { return (const float*)((const uint8_t*)nrm + off); };
    float* h = (float*)(act + M->a_bh);
    uint16_t* xa = (uint16_t*)(act + M->a_bxa);
    uint16_t* xb = (uint16_t*)(act + M->a_bxb);
    float* qkv = (float*)(act + M->a_bqkv);
    float* part_r = (float*)(act + M->a_bpart_r);
    const uint64_t pstride = (uint64_t)M->rows * H;
    auto gemm = [&](const VxMatPlan& p, const VxBGemmArgs& ga, int epi) {
        return vx_launch_mgemm(vx_mview(A, p), ga, epi, st);
    };

    vx_record(vx_launch_bembed(vx_view(A, M->embed), rows, n, h, H, mask, st));
    VxAttnArgs at;
    std::memset(&at, 0, sizeof(at));
    at.qkv = qkv;
    at.rope = (const float2*)vecp(M->rope);
    at.state = rows;
    at.part_o = (float*)(act + M->a_bpart_o);
    at.part_ml = (float*)(act + M->a_bpart_ml);
    at.hq = c.num_heads;
    at.hkv = c.num_kv_heads;
    at.s_max = c.max_seq_len;
    at.s_cap = M->s_cap;
    // splits for about 256 attention workgroups over the rows' (row, kv head) pairs (measured at
    // Qwen2.5-7B ctx 2048: B = 32 best at 2, B = 8 at 8), at most the planned count the partial
    // buffers hold
    uint32_t bsplits = (256u + n * c.num_kv_heads / 2u) / (n * c.num_kv_heads);
    bsplits = bsplits < 1u ? 1u : bsplits > M->splits ? M->splits : bsplits;
    at.splits = bsplits;
    at.scale = 1.0f / sqrtf((float)D);
    at.active_mask = mask;
    at.partials_only = 1;
    at.batch = n;
    at.prefill = prefill ? 1u : 0u;
    at.max_len = max_len;
    // decode: consecutive sequences of one layer; prefill: every row reads sequence 0's cache
    at.kv_bstride = prefill ? 0 : M->kv_layer_bytes / 2;
    at.qkv_bstride = qd + 2 * kvd;
    if (bsplits == 1) {
        at.x16 = xa;
        at.x_ld = M->x_ld;
        at.x_bs = M->x_bs;
    }
    VxBGemmArgs g;
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        const VxLayerPlan& L = M->layers[l];
        // the previous layer's down projection left its K-split partials (none before layer 0)
        vx_record(vx_launch_bnorm(h, H, l && M->ksplit_down > 1 ? part_r : nullptr, M->ksplit_down, pstride,
                                  vecp(L.attn_norm), H, c.rms_norm_eps, xa, M->x_ld, M->x_bs, n, mask, st));
        std::memset(&g, 0, sizeof(g));
        g.batch = n;
        g.active_mask = mask;
        g.x16 = xa;
        g.ldx = M->x_ld;
        g.xbs = M->x_bs;
        g.bias = c.qkv_bias ? vecp(L.bias) : nullptr;
        g.y = qkv;
        g.ldy = qd + 2 * kvd;
        const uint32_t ks_qkv = n > 16u ? M->ksplit_qkv_wide : M->ksplit_qkv;
        if (ks_qkv > 1) {  // K-split partials, then their sum + bias
            g.ksplit = ks_qkv;
            g.part = part_r;
            g.pstride = (uint64_t)M->rows * g.ldy;
        }
        vx_record(gemm(L.qkv, g, VX_EPI_STORE));
        // QKV split over K: the K/V-row and attention kernels sum the partials (+ bias) themselves
        at.qkv_nparts = g.ksplit > 1 ? g.ksplit : 0u;
        at.qkv_part = part_r;
        at.qkv_pstride = g.pstride;
        at.qkv_bias = g.bias;
        at.kv = vx_kv(M, A, l, 0);
        if (prefill)
            vx_record(vx_launch_kv_append_rows(at.qkv_nparts ? part_r : qkv, qd + 2 * kvd, at.qkv_nparts, g.pstride,
                                               g.bias, c.num_heads, c.num_kv_heads, D, rows, n, at.rope,
                                               c.max_seq_len, M->s_cap, at.kv, mask, st));
        vx_record(vx_launch_attention(at, D, st));
        if (bsplits > 1)  // (one split: the attention wrote the o_proj operand itself)
            vx_record(vx_launch_bmerge(at.part_o, at.part_ml, c.num_heads, D, bsplits, xa, M->x_ld, M->x_bs, n, mask, st));
        std::memset(&g, 0, sizeof(g));
        g.batch = n;
        g.active_mask = mask;
        g.x16 = xa;
        g.ldx = M->x_ld;
        g.xbs = M->x_bs;
        g.y = h;
        g.ldy = H;
        g.ksplit = M->ksplit_o;
        g.part = part_r;
        g.pstride = pstride;
        vx_record(gemm(L.o, g, VX_EPI_RESID));
        vx_record(vx_launch_bnorm(h, H, M->ksplit_o > 1 ? part_r : nullptr, M->ksplit_o, pstride, vecp(L.mlp_norm), H,
                                  c.rms_norm_eps, xa, M->x_ld, M->x_bs, n, mask, st));
        std::memset(&g, 0, sizeof(g));
        g.batch = n;
        g.active_mask = mask;
        g.x16 = xa;
        g.ldx = M->x_ld;
        g.xbs = M->x_bs;
        g.out16 = xb;
        g.ldo = M->x_ld;
        g.obs = M->x_bs;
        vx_record(gemm(L.gate_up, g, VX_EPI_SWIGLU));
        std::memset(&g, 0, sizeof(g));
        g.batch = n;
        g.active_mask = mask;
        g.x16 = xb;
        g.ldx = M->x_ld;
        g.xbs = M->x_bs;
        g.y = h;
        g.ldy = H;
        g.ksplit = M->ksplit_down;
        g.part = part_r;
        g.pstride = pstride;
        vx_record(gemm(L.down, g, VX_EPI_RESID));
    }
    vx_record(vx_launch_bnorm(h, H, M->ksplit_down > 1 ? part_r : nullptr, M->ksplit_down, pstride,
                              vecp(M->final_norm), H, c.rms_norm_eps, xa, M->x_ld, M->x_bs, n, mask, st));
    std::memset(&g, 0, sizeof(g));
    g.batch = n;
    g.active_mask = mask;
    g.x16 = xa;
    g.ldx = M->x_ld;
        g.xbs = M->x_bs;
    g.y = (float*)(act + M->a_blogits);
    g.ldy = c.vocab_size;
    g.cand_v = (float*)(act + M->a_bcand_v);
    g.cand_i = (uint32_t*)(act + M->a_bcand_i);
    vx_record(gemm(M->head, g, VX_EPI_ARGMAX));
}

}  // namespace

// One decode step of sequences 0 .. batch-1, each at its own state (step, token): the weights are
// read once per step for all of them; then the argmax of every sequence.
void velox_hip_decode_batch_graph_step(VeloxHipArena* A, uint32_t batch, uint64_t mask, hipStream_t st) {
    const VeloxHipModel* M = vx_model(A);
    if (!M || M->batch < 2 || batch == 0 || batch > M->batch) {
        if (!g_last_error) g_last_error = VELOX_HIP_EINVAL;
        return;
    }
    uint8_t* act = A->activation_arena;
    VeloxDecodeState* states = (VeloxDecodeState*)(act + M->a_bstate);
    vx_rows_forward(M, A, states, batch, mask, false, 0u, st);
    vx_record(vx_launch_bfinalize((const float*)(act + M->a_bcand_v), (const uint32_t*)(act + M->a_bcand_i),
                                  M->head_bwgs, states, A->host_pinned_ring, (const uint32_t*)(act + M->a_bprompt),
                                  (const uint32_t*)(act + M->a_bplen), M->cfg.max_seq_len, batch, mask, st));
}

// Prompt positions [pos0, pos0 + n_tokens) of sequence 0 in chunks of up to prefill_chunk rows.
int velox_hip_prefill_batch(VeloxHipArena* A, uint64_t pos0, uint32_t n_tokens, uint64_t mask, hipStream_t st) {
    const VeloxHipModel* M = vx_model(A);
    if (!M) return VELOX_HIP_EINVAL;
    const uint32_t chunk = M->cfg.prefill_chunk;
    uint32_t plen = 0;
    {
        std::lock_guard<std::mutex> lock(g_arena_mu);
        if (const VxArenaRec* r = vx_rec_locked(A->weight_arena)) plen = r->staged_plen;
    }
    // every row reads its token from the staged prompt: positions must lie inside it
    if (chunk < 2 || n_tokens == 0 || pos0 + n_tokens > M->cfg.max_seq_len || pos0 + n_tokens > plen)
        return VELOX_HIP_EINVAL;
    uint8_t* act = A->activation_arena;
    VeloxDecodeState* rows = (VeloxDecodeState*)(act + M->a_prows);
    const uint32_t* prompt = (const uint32_t*)(act + M->a_prompt);
    // this call's first launch error, whatever an earlier unread one was (restored afterwards)
    const int before = g_last_error;
    g_last_error = 0;
    for (uint32_t done = 0; done < n_tokens;) {
        const uint32_t n = n_tokens - done < chunk ? n_tokens - done : chunk;
        vx_record(vx_launch_prefill_rows(rows, n, pos0 + done, prompt, mask, st));
        vx_rows_forward(M, A, rows, n, mask, true, (uint32_t)(pos0 + done + n), st);
        vx_record(vx_launch_prefill_finalize((const float*)(act + M->a_bcand_v), (const uint32_t*)(act + M->a_bcand_i),
                                             M->head_bwgs, rows, n, A->host_pinned_ring,
                                             (VeloxDecodeState*)(act + M->a_state), prompt,
                                             (const uint32_t*)(act + M->a_plen), mask, st));
        done += n;
    }
    const int mine = g_last_error;
    g_last_error = before;
    return mine;
}

// ---------------------------------------------------------------------------------------------
// The decode step: embed -> L x [QKV(+norm), attention, o_proj+res, gate/up(+norm)+SwiGLU,
// down+res] -> norm + LM head + argmax (+ ring + state advance). 2 + 5L launches.
// ---------------------------------------------------------------------------------------------
namespace {
// Grid cap of a single-sequence GEMV: one workgroup per CU (M->head_wgs) for matrices of more than
// 96 MB, as for the LM head, and for rows of 8192 or more weights (256+ blocks: every wave tile a long
// stream), else the default 512. Qwen2-72B's gate/up (272 MB) and down (136 MB): 48.3 -> 45.6 us and
// 31.1 -> 26.4 us per launch (kernel trace), 104.3-105.4 -> 108.2-111.2 tok/s (three alternating runs
// each); then its QKV and o_proj (K = 8192): 12.95 -> 12.23 and 9.77 -> 9.32 us, 107.1-110.0 ->
// 109.9-112.8 tok/s. Lowering the size bound to 60 MB (Llama-3-8B's and Qwen2.5-7B's gate/up, K 4096
// and 3584) lost: 773 -> 757 and 726 -> 712 tok/s. (Other grids of these models are already <= 256.)
constexpr uint64_t kVxOneRoundBytes = 96000000ull;
constexpr uint32_t kVxOneRoundK = 8192;
uint32_t vx_wgs_for(const VeloxHipModel* M, const VxMatPlan& p) {
    return p.code_bytes + p.scale_bytes > kVxOneRoundBytes || p.k >= kVxOneRoundK ? M->head_wgs : M->max_wgs;
}
}  // namespace

void velox_hip_decode_graph_step(VeloxHipArena* A, uint64_t mask, hipStream_t st) {
    bool xcd_rr = false;
    const VeloxHipModel* M = vx_model(A, &xcd_rr);
    if (!M) { if (!g_last_error) g_last_error = VELOX_HIP_EINVAL; return; }
    // QKV and attention in one launch per layer (vx_qkv_attn.hip)
    const bool fused = M->fused_splits && xcd_rr && g_fused_attention.load(std::memory_order_relaxed);
    const uint32_t att_splits = fused ? M->fused_splits : M->splits;
    const VeloxHipModelConfig& c = M->cfg;
    uint8_t* act = A->activation_arena;
    const float* nrm = (const float*)A->norm_weight_arena;
    VeloxDecodeState* state = (VeloxDecodeState*)(act + M->a_state);
    float* h = (float*)(act + M->a_h);
    float* qkv = (float*)(act + M->a_qkv);
    float* attn = (float*)(act + M->a_attn);
    float* ffn = (float*)(act + M->a_act);
    auto vecp = [&](uint64_t off) { return (const float*)((const uint8_t*)nrm + off); };

    float2* rope_cur = (float2*)(act + M->a_rope_cur);
    vx_record(vx_launch_embed(vx_view(A, M->embed), state, 0, h, mask, st, (const float2*)vecp(M->rope), rope_cur,
                              c.head_dim / 2, c.max_seq_len));
    VxAttnArgs at;
    std::memset(&at, 0, sizeof(at));
    at.qkv = qkv;
    at.rope = (const float2*)vecp(M->rope);
    at.rope_cur = rope_cur;
    at.state = state;
    at.part_o = (float*)(act + M->a_part_o);
    at.part_ml = (float*)(act + M->a_part_ml);
    at.counters = (uint32_t*)(act + M->a_counters);
    at.out = attn;
    at.hq = c.num_heads;
    at.hkv = c.num_kv_heads;
    at.s_max = c.max_seq_len;
    at.s_cap = M->s_cap;
    at.splits = att_splits;
    at.scale = 1.0f / sqrtf((float)c.head_dim);
    at.active_mask = mask;
    at.partials_only = M->fused_merge ? 1u : 0u;
    uint32_t tl_n = 0;
    for (uint32_t l = 0; l < c.num_layers; ++l) {
        const VxLayerPlan& L = M->layers[l];
        VxGemvArgs g;
        std::memset(&g, 0, sizeof(g));
        g.active_mask = mask;
        g.eps = c.rms_norm_eps;
        g.x = h;
        g.gain = vecp(L.attn_norm);
        g.bias = c.qkv_bias ? vecp(L.bias) : nullptr;
        g.y = qkv;
        at.kv = vx_kv(M, A, l, 0);
        if (fused) {
            VxQkvAttnArgs f;
            std::memset(&f, 0, sizeof(f));
            f.g = g;
            f.at = at;
            f.sync = (uint32_t*)(act + M->a_fsync);
            vx_tl_slot(f.g, tl_n);
            vx_record(vx_launch_qkv_attn(vx_view(A, L.qkv), f, M->fused_p, st));
        } else {
            vx_tl_slot(g, tl_n);
            vx_record(vx_launch_gemv(vx_view(A, L.qkv), g, VX_EPI_STORE, vx_wgs_for(M, L.qkv), st));
            vx_tl_slot(at, tl_n);
            vx_record(vx_launch_attention(at, c.head_dim, st));
        }

        std::memset(&g, 0, sizeof(g));
        g.active_mask = mask;
        g.x = attn;
        if (fused || M->fused_merge) {
            g.part_o = at.part_o;
            g.part_ml = at.part_ml;
            g.att_splits = att_splits;
            g.att_d = c.head_dim;
        }
        g.res = h;
        g.y = h;
        vx_tl_slot(g, tl_n);
        vx_record(vx_launch_gemv(vx_view(A, L.o), g, VX_EPI_RESID, vx_wgs_for(M, L.o), st));

        std::memset(&g, 0, sizeof(g));
        g.active_mask = mask;
        g.eps = c.rms_norm_eps;
        g.x = h;
        g.gain = vecp(L.mlp_norm);
        g.y = ffn;
        vx_tl_slot(g, tl_n);
        vx_record(vx_launch_gemv(vx_view(A, L.gate_up), g, VX_EPI_SWIGLU, vx_wgs_for(M, L.gate_up), st));

        std::memset(&g, 0, sizeof(g));
        g.active_mask = mask;
        g.x = ffn;
        g.res = h;
        g.y = h;
        vx_tl_slot(g, tl_n);
        vx_record(vx_launch_gemv(vx_view(A, L.down), g, VX_EPI_RESID, vx_wgs_for(M, L.down), st));
    }
    VxGemvArgs g;
    std::memset(&g, 0, sizeof(g));
    g.active_mask = mask;
    g.eps = c.rms_norm_eps;
    g.x = h;
    g.gain = vecp(M->final_norm);
    g.y = (float*)(act + M->a_logits);
    g.cand_v = (float*)(act + M->a_cand_v);
    g.cand_i = (uint32_t*)(act + M->a_cand_i);
    vx_tl_slot(g, tl_n);
    vx_record(vx_launch_gemv(vx_view(A, M->head), g, VX_EPI_ARGMAX, M->head_wgs, st));
    vx_record(vx_launch_argmax_finalize(g.cand_v, g.cand_i, vx_gemv_grid(M->head.n_tiles, M->head_wgs), state,
                                        A->host_pinned_ring, (const uint32_t*)(act + M->a_prompt),
                                        (const uint32_t*)(act + M->a_plen), (uint32_t*)(act + M->a_token), mask, st));
}

void velox_hip_decode(VeloxHipArena* A, uint32_t token_in, size_t step, uint64_t mask, hipStream_t st) {
    const VeloxHipModel* M = vx_model(A);
    if (!M) { if (!g_last_error) g_last_error = VELOX_HIP_EINVAL; return; }
    vx_record(vx_launch_set_state((VeloxDecodeState*)(A->activation_arena + M->a_state), step, token_in, st));
    velox_hip_decode_graph_step(A, mask, st);
}

// Prefill is the same single-token step (the reference runner prefills token by token,
// velox_cuda_runner.cu:504-506); the staged prompt forces the next token.
void velox_hip_prefill_graph_step(VeloxHipArena* A, uint64_t mask, hipStream_t st) {
    velox_hip_decode_graph_step(A, mask, st);
}
void velox_hip_prefill(VeloxHipArena* A, uint32_t token_in, size_t step, uint64_t mask, hipStream_t st) {
    velox_hip_decode(A, token_in, step, mask, st);
}

int velox_hip_arena_check(const VeloxHipArena* a, const VeloxHipModelConfig* want) {
    const VeloxHipModel* M = vx_model(a);
    if (!M || !want) return VELOX_HIP_EINVAL;
    const VeloxHipModelConfig& c = M->cfg;
    const bool same = c.vocab_size == want->vocab_size && c.hidden_dim == want->hidden_dim &&
                      c.intermediate_dim == want->intermediate_dim && c.num_heads == want->num_heads &&
                      c.num_kv_heads == want->num_kv_heads && c.head_dim == want->head_dim &&
                      c.qkv_bias == want->qkv_bias && c.tied_lm_head == want->tied_lm_head &&
                      c.rms_norm_eps == want->rms_norm_eps && c.rope_theta == want->rope_theta &&
                      (want->num_layers == 0 || c.num_layers == want->num_layers);
    return same ? VELOX_HIP_OK : VELOX_HIP_EINVAL;
}

// The builtin models' entry points take an arena whose plan has the model's dimensions (any depth:
// the parity tests run them on fewer layers), whatever the plan is named.
#define VX_MODEL_ENTRY(NAME, KEY)                                                                   \
    static bool vx_is_##NAME(const VeloxHipArena* a) {                                              \
        VeloxHipModelConfig want;                                                                   \
        if (velox_hip_builtin_config(KEY, 0, &want) == VELOX_HIP_OK) {                              \
            want.num_layers = 0;                                                                    \
            if (velox_hip_arena_check(a, &want) == VELOX_HIP_OK) return true;                      \
        }                                                                                           \
        if (!g_last_error) g_last_error = VELOX_HIP_EINVAL;                                         \
        return false;                                                                               \
    }                                                                                               \
    void velox_##NAME##_decode_graph_step_hip(VeloxHipArena* ctx, uint64_t m, hipStream_t s) {      \
        if (vx_is_##NAME(ctx)) velox_hip_decode_graph_step(ctx, m, s);                              \
    }                                                                                               \
    void velox_##NAME##_decode_hip(VeloxHipArena* ctx, uint32_t t, size_t st, uint64_t m, hipStream_t s) { \
        if (vx_is_##NAME(ctx)) velox_hip_decode(ctx, t, st, m, s);                                  \
    }

VX_MODEL_ENTRY(SmolLM_135M, "smollm_135m")
VX_MODEL_ENTRY(Llama3_8B, "llama3_8b")
VX_MODEL_ENTRY(Qwen2_5_7B, "qwen2_5_7b")
VX_MODEL_ENTRY(Qwen2_72B, "qwen2_72b")

void velox_SmolLM_135M_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t m, hipStream_t s) {
    if (vx_is_SmolLM_135M(ctx)) velox_hip_prefill_graph_step(ctx, m, s);
}
void velox_SmolLM_135M_prefill_hip(VeloxHipArena* ctx, uint32_t t, size_t st, uint64_t m, hipStream_t s) {
    if (vx_is_SmolLM_135M(ctx)) velox_hip_prefill(ctx, t, st, m, s);
}
void velox_Llama3_8B_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t m, hipStream_t s) {
    if (vx_is_Llama3_8B(ctx)) velox_hip_prefill_graph_step(ctx, m, s);
}
void velox_Llama3_8B_prefill_hip(VeloxHipArena* ctx, uint32_t t, size_t st, uint64_t m, hipStream_t s) {
    if (vx_is_Llama3_8B(ctx)) velox_hip_prefill(ctx, t, st, m, s);
}
void velox_Qwen2_5_7B_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t m, hipStream_t s) {
    if (vx_is_Qwen2_5_7B(ctx)) velox_hip_prefill_graph_step(ctx, m, s);
}
void velox_Qwen2_5_7B_prefill_hip(VeloxHipArena* ctx, uint32_t t, size_t st, uint64_t m, hipStream_t s) {
    if (vx_is_Qwen2_5_7B(ctx)) velox_hip_prefill(ctx, t, st, m, s);
}
void velox_Qwen2_72B_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t m, hipStream_t s) {
    if (vx_is_Qwen2_72B(ctx)) velox_hip_prefill_graph_step(ctx, m, s);
}
void velox_Qwen2_72B_prefill_hip(VeloxHipArena* ctx, uint32_t t, size_t st, uint64_t m, hipStream_t s) {
    if (vx_is_Qwen2_72B(ctx)) velox_hip_prefill(ctx, t, st, m, s);
}

// ---------------------------------------------------------------------------------------------
// Per-kernel entry points
// ---------------------------------------------------------------------------------------------
int velox_hip_q4_0_repack(const void* d_blocks, uint32_t rows, uint32_t row0, uint32_t pair_part,
                          const VeloxHipQ4Matrix* m, hipStream_t st) {
    if (!d_blocks || !m || m->format != 0) return VELOX_HIP_EINVAL;  // GGML Q4_0 blocks only
    const uint32_t logical = m->n;
    if (row0 + rows > logical || pair_part > (m->paired ? 1u : 0u)) return VELOX_HIP_EINVAL;
    return (int)vx_launch_repack(d_blocks, rows, row0, pair_part, vx_view_public(m), st);
}

int velox_hip_q4_0_dequant(const VeloxHipQ4Matrix* m, float* d_out, hipStream_t st) {
    if (!m || !d_out || (m->format != 0 && m->format != VELOX_QUANT_Q4_GROUP64)) return VELOX_HIP_EINVAL;
    return (int)vx_launch_dequant(vx_view_public(m), d_out, st);
}

int velox_hip_q4_0_quantize(const float* d_x, uint32_t rows, uint32_t k, void* d_blocks, hipStream_t st) {
    if (!d_x || !d_blocks || k % 32) return VELOX_HIP_EINVAL;
    return (int)vx_launch_quantize(d_x, rows, k, d_blocks, st);
}

int velox_hip_g64_quantize(const float* d_x, uint64_t n_groups, uint32_t* d_packed, uint16_t* d_scale_min,
                           hipStream_t st) {
    if (!d_x || !d_packed || !d_scale_min) return VELOX_HIP_EINVAL;
    return (int)vx_launch_g64_quantize_ref(d_x, n_groups, d_packed, d_scale_min, st);
}

int velox_hip_g64_pack(const float* d_rows, uint32_t rows, uint32_t row0, uint32_t pair_part,
                       const VeloxHipQ4Matrix* m, hipStream_t st) {
    if (!d_rows || !m || m->format != VELOX_QUANT_Q4_GROUP64 || m->k % 64 || (m->s_lanes & 1u)) return VELOX_HIP_EINVAL;
    if (row0 + rows > m->n || pair_part > (m->paired ? 1u : 0u)) return VELOX_HIP_EINVAL;
    return (int)vx_launch_g64_from_rows(d_rows, rows, row0, pair_part, vx_view_public(m), st);
}

int velox_hip_fill_normal(float* d_out, uint64_t n, uint64_t seed, uint64_t tag, float sigma, float mean,
                          hipStream_t st) {
    if (!d_out) return VELOX_HIP_EINVAL;
    return (int)vx_launch_fill_normal(d_out, n, vx_stream(seed, tag), sigma == 0.0f ? 0.0f : vx_normal_coef(sigma),
                                      mean, st);
}

int velox_hip_gemv_q4_0(const VeloxHipQ4Matrix* m, const float* d_x, const float* d_gain, float eps,
                        const float* d_bias, const float* d_res, float* d_y, int mode, hipStream_t st) {
    if (!m || !d_x || !d_y || mode < 0 || mode > 2) return VELOX_HIP_EINVAL;
    if (mode == VELOX_GEMV_RESIDUAL && !d_res) return VELOX_HIP_EINVAL;
    if ((mode == VELOX_GEMV_SWIGLU) != (m->paired != 0)) return VELOX_HIP_EINVAL;
    VxGemvArgs g;
    std::memset(&g, 0, sizeof(g));
    g.x = d_x;
    g.gain = d_gain;
    g.eps = eps;
    g.bias = d_bias;
    g.res = d_res;
    g.y = d_y;
    g.active_mask = 1;
    const int epi = mode == VELOX_GEMV_STORE ? VX_EPI_STORE : mode == VELOX_GEMV_RESIDUAL ? VX_EPI_RESID : VX_EPI_SWIGLU;
    return (int)vx_launch_gemv(vx_view_public(m), g, epi, vx_gemv_max_wgs_default(), st);
}

int velox_hip_gemm_q4_0_batch(const VeloxHipQ4Matrix* m, const uint16_t* d_x16, uint32_t batch, uint32_t ldx,
                              const float* d_bias, float* d_y, uint32_t ldy, uint16_t* d_out16, uint32_t ldo,
                              int mode, hipStream_t st) {
    if (!m || m->format != 0 || !d_x16 || batch == 0 || batch > 32 || ldx < m->k || (ldx & 7u) || mode < 0 ||
        mode > 2)
        return VELOX_HIP_EINVAL;
    if ((mode == VELOX_GEMV_SWIGLU) != (m->paired != 0)) return VELOX_HIP_EINVAL;
    if (mode == VELOX_GEMV_SWIGLU ? (!d_out16 || ldo < m->n) : (!d_y || ldy < m->n))
        return VELOX_HIP_EINVAL;
    // the batched steps' GEMM over a per-call MFMA-layout copy of the tiled matrix (built on the
    // device, released after a stream synchronization)
    VxMMat mm;
    vx_mmat_shape(m->n, m->k, m->paired, mm);
    const uint64_t cb = vx_mmat_code_bytes(mm), sb = vx_mmat_scale_bytes(mm);
    uint8_t* buf = nullptr;
    hipError_t e = hipMalloc((void**)&buf, cb + sb);
    if (e != hipSuccess) return (int)e;
    mm.codes = (const uint4*)buf;
    mm.scales = (const uint2*)(buf + cb);
    e = vx_launch_mlayout(vx_view_public(m), mm, st);
    VxBGemmArgs g;
    std::memset(&g, 0, sizeof(g));
    g.batch = batch;
    g.x16 = d_x16;
    g.ldx = ldx;
    g.xbs = 32;
    g.bias = d_bias;
    g.y = d_y;
    g.ldy = ldy;
    g.out16 = d_out16;
    g.ldo = ldo;
    g.obs = 32;
    g.active_mask = 1;
    g.ksplit = 1;
    const int epi = mode == VELOX_GEMV_STORE ? VX_EPI_STORE : mode == VELOX_GEMV_RESIDUAL ? VX_EPI_RESID : VX_EPI_SWIGLU;
    if (e == hipSuccess) e = vx_launch_mgemm(mm, g, epi, st);
    const hipError_t es = hipStreamSynchronize(st);
    if (e == hipSuccess) e = es;
    hipFree(buf);
    return (int)e;
}

namespace {
bool vx_mmat_public(const VeloxHipQ4Matrix* m, const void* codes, const void* scales, VxMMat& out) {
    if (!m || m->format != 0 || m->k == 0 || (m->k & 31u) || m->n == 0) return false;  // GGML Q4_0 only
    vx_mmat_shape(m->n, m->k, m->paired, out);
    out.codes = (const uint4*)codes;
    out.scales = (const uint2*)scales;
    return true;
}
}  // namespace

int velox_hip_q4_mlayout_bytes(const VeloxHipQ4Matrix* m, uint64_t* code_bytes, uint64_t* scale_bytes) {
    VxMMat mm;
    if (!vx_mmat_public(m, nullptr, nullptr, mm)) return VELOX_HIP_EINVAL;
    if (code_bytes) *code_bytes = vx_mmat_code_bytes(mm);
    if (scale_bytes) *scale_bytes = vx_mmat_scale_bytes(mm);
    return VELOX_HIP_OK;
}

int velox_hip_q4_mlayout(const VeloxHipQ4Matrix* m, void* d_codes, void* d_scales, hipStream_t st) {
    VxMMat mm;
    if (!d_codes || !d_scales || !vx_mmat_public(m, d_codes, d_scales, mm)) return VELOX_HIP_EINVAL;
    return (int)vx_launch_mlayout(vx_view_public(m), mm, st);
}

int velox_hip_gemm_q4_0_batch_m(const VeloxHipQ4Matrix* m, const void* d_mcodes, const void* d_mscales,
                                const uint16_t* d_x16, uint32_t batch, uint32_t ldx, uint32_t xbs, const float* d_bias,
                                float* d_y, uint32_t ldy, uint16_t* d_out16, uint32_t ldo, uint32_t obs, int mode,
                                uint32_t ksplit, float* d_part, hipStream_t st) {
    VxMMat mm;
    if (!d_mcodes || !d_mscales || !vx_mmat_public(m, d_mcodes, d_mscales, mm)) return VELOX_HIP_EINVAL;
    if (xbs == 0) xbs = 32;
    if (obs == 0) obs = 32;
    if (!d_x16 || batch == 0 || batch > 128 || (ldx & 7u) || (xbs & 7u) || !vx_x_layout_ok(m->k, ldx, xbs, batch) ||
        mode < 0 || mode > 2)
        return VELOX_HIP_EINVAL;
    if ((mode == VELOX_GEMV_SWIGLU) != (m->paired != 0)) return VELOX_HIP_EINVAL;
    if (mode == VELOX_GEMV_SWIGLU ? (!d_out16 || !vx_x_layout_ok(m->n, ldo, obs, batch)) : (!d_y || ldy < m->n))
        return VELOX_HIP_EINVAL;
    if (ksplit == 0 || ksplit > 8 || ksplit > mm.n_grp || (ksplit > 1 && (mode == VELOX_GEMV_SWIGLU || !d_part)))
        return VELOX_HIP_EINVAL;
    VxBGemmArgs g;
    std::memset(&g, 0, sizeof(g));
    g.batch = batch;
    g.x16 = d_x16;
    g.ldx = ldx;
    g.xbs = xbs;
    g.bias = d_bias;
    g.y = d_y;
    g.ldy = ldy;
    g.out16 = d_out16;
    g.ldo = ldo;
    g.obs = obs;
    g.active_mask = 1;
    g.ksplit = ksplit;
    g.part = d_part;
    g.pstride = (uint64_t)batch * ldy;
    const int epi = mode == VELOX_GEMV_STORE ? VX_EPI_STORE : mode == VELOX_GEMV_RESIDUAL ? VX_EPI_RESID : VX_EPI_SWIGLU;
    hipError_t e = vx_launch_mgemm(mm, g, epi, st);
    if (e == hipSuccess && ksplit > 1)
        e = vx_launch_msum(d_part, ksplit, g.pstride, epi == VX_EPI_STORE ? d_bias : nullptr, d_y, m->n, ldy, batch,
                           epi == VX_EPI_RESID ? 1u : 0u, 1ULL, st);
    return (int)e;
}

int velox_hip_lm_head_argmax(const VeloxHipQ4Matrix* m, const float* d_x, const float* d_gain, float eps,
                             float* d_logits, uint32_t* d_token, hipStream_t st) {
    if (!m || !d_x || !d_logits || !d_token || m->paired) return VELOX_HIP_EINVAL;
    // per-call candidate buffer (one (value, index) per GEMV workgroup), released once the call's
    // work has finished: this entry point returns after a stream synchronization
    const uint32_t wgs = vx_gemv_max_wgs_default(), n = vx_gemv_grid(m->n_tiles, wgs);
    void* cand = nullptr;
    hipError_t e = hipMalloc(&cand, (size_t)n * 8u);
    if (e != hipSuccess) return (int)e;
    VxGemvArgs g;
    std::memset(&g, 0, sizeof(g));
    g.x = d_x;
    g.gain = d_gain;
    g.eps = eps;
    g.y = d_logits;
    g.cand_v = (float*)cand;
    g.cand_i = (uint32_t*)((uint8_t*)cand + (size_t)n * 4u);
    g.active_mask = 1;
    e = vx_launch_gemv(vx_view_public(m), g, VX_EPI_ARGMAX, wgs, st);
    if (e == hipSuccess)
        e = vx_launch_argmax_finalize(g.cand_v, g.cand_i, n, nullptr, nullptr, nullptr, nullptr, d_token, 1, st);
    const hipError_t es = hipStreamSynchronize(st);
    if (e == hipSuccess) e = es;
    hipFree(cand);
    return (int)e;
}

int velox_hip_argmax_f32(const float* d_x, uint32_t n, uint32_t* d_out, hipStream_t st) {
    if (!d_x || !d_out || n == 0) return VELOX_HIP_EINVAL;
    return (int)vx_launch_argmax(d_x, n, d_out, st);
}

int velox_hip_rmsnorm(const float* d_x, const float* d_w, uint32_t n, float eps, float* d_y, hipStream_t st) {
    if (!d_x || !d_w || !d_y || n == 0) return VELOX_HIP_EINVAL;
    return (int)vx_launch_rmsnorm(d_x, d_w, n, eps, d_y, st);
}

int velox_hip_attention_decode(const float* d_qkv, uint16_t* d_kv_layer, uint32_t hq, uint32_t hkv, uint32_t d,
                               uint32_t s_max, uint32_t pos, float theta, uint32_t splits, float* d_out,
                               hipStream_t st) {
    if (!d_qkv || !d_kv_layer || !d_out || hkv == 0 || hkv > 64 || hq % hkv || pos >= s_max || splits == 0 ||
        splits > 64)
        return VELOX_HIP_EINVAL;
    // rope row for `pos`, partials and counters: per-call scratch (test entry point)
    const uint32_t half = d / 2;
    std::vector<float> rope((size_t)half * 2);
    for (uint32_t j = 0; j < half; ++j) {
        const float freq = 1.0f / powf(theta, (float)(2 * j) / (float)d);
        const float angle = (float)pos * freq;
        rope[2 * j] = cosf(angle);
        rope[2 * j + 1] = sinf(angle);
    }
    const size_t rope_b = vx_align((size_t)(pos + 1) * half * 8);
    const size_t po_b = vx_align((size_t)hq * splits * d * 4), pml_b = vx_align((size_t)hq * splits * 8);
    uint8_t* scratch = nullptr;
    hipError_t e = hipMalloc((void**)&scratch, rope_b + po_b + pml_b + 256);
    if (e != hipSuccess) return (int)e;
    e = hipMemsetAsync(scratch + rope_b + po_b + pml_b, 0, 256, st);
    if (e == hipSuccess)
        e = hipMemcpyAsync(scratch + (size_t)pos * half * 8, rope.data(), (size_t)half * 8, hipMemcpyHostToDevice, st);
    VxAttnArgs at;
    std::memset(&at, 0, sizeof(at));
    at.qkv = d_qkv;
    at.kv = d_kv_layer;
    at.rope = (const float2*)scratch;
    at.state = nullptr;
    at.fixed_pos = pos;
    at.part_o = (float*)(scratch + rope_b);
    at.part_ml = (float*)(scratch + rope_b + po_b);
    at.counters = (uint32_t*)(scratch + rope_b + po_b + pml_b);
    at.out = d_out;
    at.hq = hq;
    at.hkv = hkv;
    at.s_max = s_max;
    at.s_cap = (s_max + 31u) & ~31u;
    at.splits = splits;
    at.scale = 1.0f / sqrtf((float)d);
    at.active_mask = 1;
    if (e == hipSuccess) e = vx_launch_attention(at, d, st);
    if (e == hipSuccess) e = hipStreamSynchronize(st);
    hipFree(scratch);
    return (int)e;
}

// ---------------------------------------------------------------------------------------------
// Runner: the flow of velox_cuda_runner.cu main (:327-726) -- plan, alloc, load (synthesize),
// graph capture (:474-481), prefill (:493-512), timed decode replays (:535-563).
// ---------------------------------------------------------------------------------------------
// GGUF files start with the magic "GGUF"; any other checkpoint is read as safetensors.
static bool vx_is_gguf(const char* path) {
    FILE* f = std::fopen(path, "rb");
    if (!f) return false;
    char m[4] = {0, 0, 0, 0};
    const size_t n = std::fread(m, 1, 4, f);
    std::fclose(f);
    return n == 4 && !std::memcmp(m, "GGUF", 4);
}

int velox_hip_run(const VeloxHipRunOptions* opt, uint32_t* tokens, uint32_t max_tokens, VeloxHipRunReport* rep) {
    if (!opt || !rep || (!opt->model && !opt->weights_path && !opt->model_file && !opt->model_config) ||
        opt->prompt_len == 0)
        return VELOX_HIP_EINVAL;
    if (opt->context_len && opt->prompt_len != 1) return VELOX_HIP_EINVAL;  // context + one seed token
    std::memset(rep, 0, sizeof(*rep));
    const uint32_t base = opt->context_len;  // first decoded position
    const uint32_t total = base + opt->prompt_len + opt->warmup + opt->steps;
    VeloxHipModelConfig cfg;
    VeloxHipGguf* gguf = nullptr;
    VeloxHipSafetensors* stf = nullptr;
    int rc;
    const uint32_t msl = opt->max_seq_len ? opt->max_seq_len : total + 1;
    if (opt->weights_path && vx_is_gguf(opt->weights_path)) {
        rc = velox_hip_gguf_open(opt->weights_path, &gguf);
        if (!rc) rc = velox_hip_gguf_config(gguf, msl, &cfg);
        if (rc) { velox_hip_gguf_close(gguf); return rc; }
    } else {
        // a safetensors checkpoint (the reference runner's --weights) runs on the model the caller
        // names, or on the builtin configuration its tensor shapes match
        if (opt->weights_path) {
            rc = velox_hip_st_open(opt->weights_path, &stf);
            if (rc) return rc;
        }
        if (opt->model_config) {
            cfg = *opt->model_config;
            cfg.max_seq_len = msl;
            rc = VELOX_HIP_OK;
        } else if (opt->model_file) rc = velox_hip_vlx_load(opt->model_file, msl, &cfg, nullptr);
        else if (opt->model) rc = velox_hip_builtin_config(opt->model, msl, &cfg);
        else rc = velox_hip_st_config(stf, msl, &cfg);
        if (rc) { velox_hip_st_close(stf); return rc; }
    }
    // the arena's model stays alive until the end of the run; the file is closed once loaded
    struct Closer {
        VeloxHipGguf*& g;
        VeloxHipSafetensors*& s;
        ~Closer() { velox_hip_gguf_close(g); velox_hip_st_close(s); }
    } closer{gguf, stf};
    if (opt->num_layers && !gguf) cfg.num_layers = opt->num_layers;
    if (opt->attn_splits) cfg.attn_splits = opt->attn_splits;
    if (opt->unquantized > 3 || (opt->unquantized && gguf)) return VELOX_HIP_EINVAL;
    if (opt->unquantized)
        cfg.quant_mode = opt->unquantized == 1   ? VELOX_QUANT_F32
                         : opt->unquantized == 2 ? VELOX_QUANT_F16
                                                 : VELOX_QUANT_Q4_GROUP64;
    const uint32_t B = opt->batch > 1 ? opt->batch : 1u;
    if (B > 32 || (B > 1 && opt->prompt_tokens)) return VELOX_HIP_EINVAL;
    if (B > 1) cfg.max_batch = B;
    const bool batched_prefill = opt->prefill_chunk > 1;
    // (the batched prefill reads its tokens from the staged prompt at their positions: no context)
    if (batched_prefill && (B > 1 || opt->prefill_chunk > 128 || base)) return VELOX_HIP_EINVAL;
    if (batched_prefill) cfg.prefill_chunk = opt->prefill_chunk;
    if (cfg.max_seq_len < total) return VELOX_HIP_EINVAL;
    if (stf && (rc = velox_hip_st_check(stf, &cfg)) != 0) return rc;  // before any device allocation
    VeloxHipModel* M = nullptr;
    rc = velox_hip_model_create(&cfg, &M);
    if (rc) return rc;
    VeloxHipArena A;
    rc = velox_hip_arena_create(M, &A);
    if (rc) { velox_hip_model_destroy(M); return rc; }
    hipStream_t st;
    hipStreamCreateWithFlags(&st, hipStreamNonBlocking);
    hipEvent_t e0, e1, e2, e3;
    hipEventCreate(&e0); hipEventCreate(&e1); hipEventCreate(&e2); hipEventCreate(&e3);
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;

    const auto t_load = std::chrono::steady_clock::now();
    rc = gguf  ? velox_hip_gguf_load(&A, gguf, st)
         : stf ? velox_hip_st_load(&A, stf, st)
               : velox_hip_synthesize_model(&A, opt->seed, opt->sigma, opt->norm_sigma, st);
    rep->load_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t_load).count();

    // sequence b's prompt: seeded ids (sequence 0: the single-sequence prompt) or explicit ones
    std::vector<uint32_t> prompt((size_t)opt->prompt_len * B);
    for (uint32_t b = 0; b < B; ++b) {
        const uint64_t pst = vx_stream(opt->seed + (uint64_t)b * 0x9E3779B97F4A7C15ULL, vx_tag(0, VX_TAG_PROMPT));
        for (uint32_t i = 0; i < opt->prompt_len; ++i) {
            uint32_t& t = prompt[(size_t)b * opt->prompt_len + i];
            t = opt->prompt_tokens ? opt->prompt_tokens[i] : vx_uniform_u32(pst, i, cfg.vocab_size);
            if (t >= cfg.vocab_size && !rc) rc = VELOX_HIP_EINVAL;
        }
    }
    for (uint32_t l = 0; l < cfg.num_layers && !rc && base; ++l)
        for (uint32_t b = 0; b < B && !rc; ++b)
            rc = B > 1 ? velox_hip_fill_kv_seq(&A, l, b, base, opt->seed, 1.0f, st)
                       : velox_hip_fill_kv(&A, l, base, opt->seed, 1.0f, st);
    if (B > 1) {
        for (uint32_t b = 0; b < B && !rc; ++b) {
            rc = velox_hip_batch_set_prompt(&A, b, prompt.data() + (size_t)b * opt->prompt_len, opt->prompt_len, st);
            if (!rc) rc = velox_hip_batch_set_state(&A, b, base, prompt[(size_t)b * opt->prompt_len], st);
        }
    } else {
        if (!rc) rc = velox_hip_set_prompt(&A, prompt.data(), opt->prompt_len, st);
        if (!rc) rc = velox_hip_set_state(&A, base, prompt[0], st);
    }
    velox_hip_last_error();
    auto launch_step = [&]() {
        if (B > 1) velox_hip_decode_batch_graph_step(&A, B, 1ULL, st);
        else if (opt->decode_step) opt->decode_step(&A, 1ULL, st);
        else velox_hip_decode_graph_step(&A, 1ULL, st);
    };
    if (!rc && opt->use_graph) {
        hipError_t e = hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            launch_step();
            e = hipStreamEndCapture(st, &graph);
        }
        if (e == hipSuccess) e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
        if (e != hipSuccess) {  // fall back to eager launches (velox_cuda_runner.cu:483-486)
            if (opt->verbose) std::fprintf(stderr, "[velox-hip] graph capture failed (%d): eager launches\n", (int)e);
            exec = nullptr;
            (void)hipGetLastError();
        }
        rc = velox_hip_last_error();
    }
    // ring[pos & 1023] holds the argmax after position pos (velox_cuda_runner.cu:541-546). The host
    // copies entries out before the device can overwrite them. Single steps: an event marks the end
    // of every 512th position, and before launching the position that would overwrite an uncopied
    // entry the host waits for the event 1024 positions back and copies those 512 entries: the
    // stream keeps the ~512 steps queued behind it, so no drain stalls the device. Batched prefill
    // pieces and the end synchronize the stream and copy what is left.
    constexpr uint32_t kDrainChunk = VELOX_HIP_RING_SIZE / 2;
    uint32_t drained = base, next_pos = base, n_out = 0;
    bool first_seen = false;
    std::vector<std::pair<uint32_t, hipEvent_t>> marks;  // (position the event follows, event)
    auto copy_out = [&](uint32_t upto) {
        for (uint32_t p = drained; p < upto; ++p) {
            const uint32_t t = A.host_pinned_ring[p & (VELOX_HIP_RING_SIZE - 1)];
            if (p == base + opt->prompt_len - 1) { rep->first_token = t; first_seen = true; }
            if (tokens && n_out < max_tokens) tokens[n_out++] = t;
        }
        drained = upto;
    };
    auto drain = [&](uint32_t upto) {
        if (upto <= drained) return;
        const int e = (int)hipStreamSynchronize(st);
        if (!rc) rc = e;
        copy_out(upto);
    };
    auto one_step = [&]() {
        if (next_pos - drained >= VELOX_HIP_RING_SIZE) {
            // positions [drained, drained + kDrainChunk) ended at the mark recorded after them
            const uint32_t upto = drained + kDrainChunk;
            auto it = std::find_if(marks.begin(), marks.end(), [&](const auto& m) { return m.first == upto; });
            if (it == marks.end()) {
                drain(next_pos);
            } else {
                const int e = (int)hipEventSynchronize(it->second);
                if (!rc) rc = e;
                copy_out(upto);
                (void)hipEventDestroy(it->second);
                marks.erase(it);
            }
        }
        if (exec) vx_record(hipGraphLaunch(exec, st));
        else launch_step();
        ++next_pos;
        if ((next_pos - drained) % kDrainChunk == 0) {
            hipEvent_t ev = nullptr;
            if (hipEventCreateWithFlags(&ev, hipEventDisableTiming) == hipSuccess) {
                if (hipEventRecord(ev, st) == hipSuccess) marks.emplace_back(next_pos, ev);
                else (void)hipEventDestroy(ev);
            }
        }
    };
    if (!rc) {
        hipEventRecord(e0, st);
        if (batched_prefill) {
            // pieces of at most one ring of positions, drained in between
            for (uint32_t done = 0; done < opt->prompt_len && !rc;) {
                const uint32_t n = opt->prompt_len - done < VELOX_HIP_RING_SIZE ? opt->prompt_len - done
                                                                                : VELOX_HIP_RING_SIZE;
                drain(next_pos);
                rc = velox_hip_prefill_batch(&A, next_pos, n, 1ULL, st);
                next_pos += n;
                done += n;
            }
        } else {
            for (uint32_t p = 0; p < opt->prompt_len; ++p) one_step();
        }
        hipEventRecord(e1, st);
        for (uint32_t w = 0; w < opt->warmup && !rc; ++w) one_step();
        const int e = (int)hipStreamSynchronize(st);
        if (!rc) rc = e;
    }
    // one timing event after every timed step, for the per-step distribution (created before the
    // timed region; a record is one marker packet between two graph launches)
    std::vector<hipEvent_t> step_ev;
    if (!rc) {
        step_ev.reserve(opt->steps);
        for (uint32_t s = 0; s < opt->steps; ++s) {
            hipEvent_t ev = nullptr;
            if (hipEventCreate(&ev) != hipSuccess) break;
            step_ev.push_back(ev);
        }
    }
    if (!rc) {
        // timed region: synchronized on both sides, device time from events on the same stream
        const auto w0 = std::chrono::steady_clock::now();
        hipEventRecord(e2, st);
        for (uint32_t s = 0; s < opt->steps; ++s) {
            one_step();
            if (s < step_ev.size()) hipEventRecord(step_ev[s], st);
        }
        hipEventRecord(e3, st);
        rc = (int)hipStreamSynchronize(st);
        rep->wall_ms = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - w0).count();
        if (!rc) rc = velox_hip_last_error();
    }
    for (auto& m : marks) (void)hipEventDestroy(m.second);
    marks.clear();
    if (!rc) {
        drain(next_pos);
        float ms_p = 0.f, ms_d = 0.f;
        hipEventElapsedTime(&ms_p, e0, e1);
        hipEventElapsedTime(&ms_d, e2, e3);
        rep->prefill_ms = ms_p;
        rep->decode_ms = ms_d;
        if (!step_ev.empty() && step_ev.size() == opt->steps) {
            std::vector<double> t(step_ev.size());
            for (size_t s = 0; s < step_ev.size(); ++s) {
                float ms = 0.f;
                hipEventElapsedTime(&ms, s ? step_ev[s - 1] : e2, step_ev[s]);
                t[s] = ms;
            }
            std::sort(t.begin(), t.end());
            auto rank = [&](double q) { return t[std::min(t.size() - 1, (size_t)std::ceil(q * (double)t.size()) - 1)]; };
            rep->step_p50_ms = rank(0.50);
            rep->step_p99_ms = rank(0.99);
            rep->step_max_ms = t.back();
        }
        rep->tok_per_s = opt->steps && ms_d > 0 ? (double)B * opt->steps / (ms_d * 1e-3) : 0.0;
        double bytes = 0.0;
        const uint32_t first = base + opt->prompt_len + opt->warmup;
        for (uint32_t s = 0; s < opt->steps; ++s)
            bytes += (double)(B > 1 ? velox_hip_model_batch_step_bytes(M, B, first + s)
                                    : velox_hip_model_step_bytes(M, first + s));
        rep->bytes_per_step = opt->steps ? bytes / opt->steps : 0.0;
        rep->hbm_gbps = rep->bytes_per_step * rep->tok_per_s / B / 1e9;
        rep->n_tokens = n_out;
        rep->first_position = base;
        if (!first_seen) rep->first_token = 0;
    }
    if (!rc && opt->kernel_passes) {
        // The dominant kernel alone: the fused RMSNorm + gate/up + SwiGLU GEMV of every layer in
        // turn (each layer's weights are new to the caches), timed by events on this stream.
        uint8_t* act = A.activation_arena;
        VxGemvArgs g;
        std::memset(&g, 0, sizeof(g));
        g.active_mask = 1;
        g.eps = cfg.rms_norm_eps;
        g.x = (const float*)(act + M->a_h);
        g.y = (float*)(act + M->a_act);
        // batched: the MFMA GEMM of the gate/up + SwiGLU over all B sequences' fp16 activations
        VxBGemmArgs bg;
        std::memset(&bg, 0, sizeof(bg));
        bg.batch = B;
        bg.active_mask = 1;
        bg.x16 = (const uint16_t*)(act + M->a_bxa);
        bg.ldx = M->x_ld;
        bg.xbs = M->x_bs;
        bg.out16 = (uint16_t*)(act + M->a_bxb);
        bg.ldo = M->x_ld;
        bg.obs = M->x_bs;
        auto launch_all = [&]() {
            for (uint32_t l = 0; l < cfg.num_layers; ++l) {
                if (B > 1) {
                    const VxMatPlan& gu = M->layers[l].gate_up;
                    vx_record(vx_launch_mgemm(vx_mview(&A, gu), bg, VX_EPI_SWIGLU, st));
                } else {
                    g.gain = (const float*)(A.norm_weight_arena + M->layers[l].mlp_norm);
                    vx_record(vx_launch_gemv(vx_view(&A, M->layers[l].gate_up), g, VX_EPI_SWIGLU, M->max_wgs, st));
                }
            }
        };
        launch_all();  // warm
        hipEventRecord(e0, st);
        for (uint32_t r = 0; r < opt->kernel_passes; ++r) launch_all();
        hipEventRecord(e1, st);
        rc = (int)hipStreamSynchronize(st);
        if (!rc) rc = velox_hip_last_error();
        float ms = 0.f;
        hipEventElapsedTime(&ms, e0, e1);
        rep->kernel_launches = opt->kernel_passes * cfg.num_layers;
        rep->kernel_us = rep->kernel_launches ? ms * 1e3 / rep->kernel_launches : 0.0;
        rep->kernel_bytes = (double)cfg.intermediate_dim * 2.0 * cfg.hidden_dim / 32.0 * 18.0 +
                            (B > 1 ? (double)B * (cfg.hidden_dim * 2.0 + cfg.intermediate_dim * 2.0)
                                   : (double)cfg.hidden_dim * 4.0 * 2.0 + (double)cfg.intermediate_dim * 4.0);
    }
    rep->status = rc;
    if (exec) hipGraphExecDestroy(exec);
    if (graph) hipGraphDestroy(graph);
    for (hipEvent_t ev : step_ev) (void)hipEventDestroy(ev);
    hipEventDestroy(e0); hipEventDestroy(e1); hipEventDestroy(e2); hipEventDestroy(e3);
    hipStreamDestroy(st);
    velox_hip_arena_destroy(&A);
    velox_hip_model_destroy(M);
    return rc;
}

}  // extern "C"
