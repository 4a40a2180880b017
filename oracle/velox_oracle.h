/*
 * velox_oracle.h -- CPU restatement of Velox's fp32 decode path (TEST INFRASTRUCTURE ONLY).
 *
 * This library is the parity checker for the HIP decode step. Only tests/, the smoke()
 * entry point and bench.py's cpu_baseline leg may load it; the product path never does.
 *
 * Every function cites the reference file:line whose behaviour it restates. Formats that
 * the reference does not contain (GGML Q4_0, the synthetic-weight RNG, bf16 KV rounding,
 * QKV bias) are marked as such and are pinned by closed forms and properties in tests/.
 */
#ifndef VELOX_ORACLE_H
#define VELOX_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- counter-based synthetic RNG (shared bit-for-bit with the device synthesizer) ---- */
uint64_t vxo_mix64(uint64_t z);
uint64_t vxo_stream(uint64_t seed, uint64_t tag);
/* Irwin-Hall(8) normal approximation: (float)m * c, m an exact integer; c from vxo_normal_coef. */
float vxo_normal(uint64_t stream, uint64_t idx, float coef);
float vxo_normal_coef(float sigma);
uint32_t vxo_uniform_u32(uint64_t stream, uint64_t idx, uint32_t n);
void vxo_fill_normal(float* out, uint64_t n, uint64_t seed, uint64_t tag, float sigma, float mean);

/* Tensor tags for the synthetic model: tag = layer * 256 + kind. */
enum {
    VXO_T_EMBED = 1, VXO_T_Q = 2, VXO_T_K = 3, VXO_T_V = 4, VXO_T_O = 5, VXO_T_GATE = 6,
    VXO_T_UP = 7, VXO_T_DOWN = 8, VXO_T_ATTN_NORM = 9, VXO_T_MLP_NORM = 10,
    VXO_T_FINAL_NORM = 11, VXO_T_HEAD = 12, VXO_T_BQ = 13, VXO_T_BK = 14, VXO_T_BV = 15,
    VXO_T_PROMPT = 16,
    /* MLA layer tensors (benchmark configuration 4) */
    VXO_T_MLA_NORM = 32, VXO_T_MLA_QA = 33, VXO_T_MLA_QA_NORM = 34, VXO_T_MLA_QB = 35, VXO_T_MLA_KVA = 36,
    VXO_T_MLA_KVA_NORM = 37, VXO_T_MLA_KVB = 38, VXO_T_MLA_O = 39, VXO_T_MLA_HIDDEN = 40, VXO_T_MLA_CACHE = 41
};
uint64_t vxo_tag(uint32_t layer, uint32_t kind);

/* ---- scalar conversions (IEEE round-to-nearest-even, integer implementations) ---- */
uint16_t vxo_f32_to_f16(float f);
float vxo_f16_to_f32(uint16_t h);
uint16_t vxo_f32_to_bf16(float f);
float vxo_bf16_to_f32(uint16_t h);

/* ---- GGML Q4_0 block codec (not in the reference; GGML's published block format) ---- */
#define VXO_Q4_0_BLOCK 32
#define VXO_Q4_0_BYTES 18
void vxo_q4_0_quantize_row(const float* x, uint64_t k, uint8_t* out);
void vxo_q4_0_dequant_row(const uint8_t* blocks, uint64_t k, float* out);

/* ---- the reference's asymmetric group-64 "Q4" codec (src/codegen.rs:2337-2370, :2248-2265) ---- */
void vxo_g64_quantize(const float* src, uint64_t n_groups, uint32_t* packed, uint16_t* scale_min);
void vxo_g64_dequant(const uint32_t* packed, const uint16_t* scale_min, uint64_t n_groups, float* out);

/* ---- fp32 primitives (src/runtime.rs:588-1088) ---- */
void vxo_rmsnorm(float* dst, const float* x, const float* w, uint64_t dim, float eps);
void vxo_matmul_transposed(float* dst, const float* x, const float* w, uint64_t in_dim, uint64_t out_dim);
void vxo_matmul_q4_0(float* dst, const float* x, const uint8_t* w_blocks, uint64_t in_dim, uint64_t out_dim,
                     int threads);
void vxo_rope_rotate_half(float* t, uint64_t num_heads, uint64_t head_dim, uint64_t pos, float theta);
void vxo_gqa_attention_step(float* out, float* scores, const float* q, const float* k_layer,
                            const float* v_layer, uint64_t n_q, uint64_t n_kv, uint64_t head_dim,
                            uint64_t pos);
void vxo_swiglu_act(float* gate, const float* up, uint64_t n);
uint32_t vxo_argmax(const float* logits, uint64_t n);
void vxo_mla_absorbed_step(float* dst_hidden, const float* input_hidden, const float* w_norm,
                           const float* w_dkv, const float* w_abs_q, const float* w_abs_o,
                           float* kv_latent_pool, uint64_t hidden_dim, uint64_t latent_dim,
                           uint64_t max_seq_len, uint64_t step, float eps);

/* ---- fp8 e4m3fn (OCP) with 128x128 block scales (not in the reference: benchmark configuration 4's
 * DeepSeek-V3 weight format). scale = amax / 448 per block; code = e4m3(w / scale), round to
 * nearest even, saturating at +-448. Scales are [ceil(rows/128)][ceil(cols/128)] floats. ---- */
uint8_t vxo_f32_to_e4m3(float f);
float vxo_e4m3_to_f32(uint8_t b);
void vxo_fp8_quantize(const float* w, uint64_t rows, uint64_t cols, uint8_t* codes, float* scales);
void vxo_fp8_dequant(const uint8_t* codes, const float* scales, uint64_t rows, uint64_t cols, float* out);

/* ---- absorbed multi-head latent attention layer (DeepSeek-V3 form of src/runtime.rs:845-1044) ----
 * h_out = h + W_o concat_h(W_uv[h] ctx_h), ctx_h = softmax_t(s_ht) . c_t over t <= pos, with
 * s_ht = scale * (q_abs_h . c_t + rope(q_rope_h) . kr_t), q_abs_h = W_uk[h]^T q_nope_h,
 * q = W_qb rmsnorm(W_qa x) (q_lora > 0) or W_qb x (q_lora == 0), x = rmsnorm(h),
 * [c_t | kr_t] = [rmsnorm(c) (kv_norm) | rope(kr)] of W_kva x, written to cache row pos.
 * W_kvb rows: head h's d_nope k rows (W_uk[h]) then its d_v v rows (W_uv[h]).
 * With n_heads 1, q_lora 0, d_rope 0, kv_norm 0, d_nope = d_v = kv_lora and W_kvb = [I; I] this
 * is the reference's simplified step (vxo_mla_absorbed_step). */
typedef struct VxoMlaConfig {
    uint32_t hidden, n_heads, q_lora, kv_lora, d_nope, d_rope, d_v, kv_norm, max_seq;
    float eps, rope_theta, scale;
} VxoMlaConfig;

typedef struct VxoMlaWeights {
    const float *norm, *q_a, *q_a_norm, *q_b, *kv_a, *kv_a_norm, *kv_b, *o;  /* fp32 row-major [out][in] */
} VxoMlaWeights;

/* cache: [max_seq][kv_lora + d_rope]; cache_bf16: round the written row to bf16 (the device cache). */
void vxo_mla_layer_step(const VxoMlaConfig* c, const VxoMlaWeights* w, float* cache, int cache_bf16,
                        const float* h, float* h_out, uint64_t pos);

/* Seeded N(0, sigma) matrix (index r * cols + col of stream(seed, tag)) quantized to fp8 blocks;
 * codes [rows][cols], scales as above, dequant [rows][cols] fp32 (any output may be NULL). */
void vxo_fp8_synth_matrix(uint64_t seed, uint64_t tag, uint64_t rows, uint64_t cols, float sigma, uint8_t* codes,
                          float* scales, float* dequant);

/* ---- whole-model engine (src/runtime.rs:1160-1490) ---- */
typedef struct VxoConfig {
    uint32_t vocab_size, hidden_dim, intermediate_dim, num_layers;
    uint32_t num_heads, num_kv_heads, head_dim, max_seq_len;
    float rms_norm_eps, rope_theta;
    uint32_t qkv_bias;     /* 1: add b_q/b_k/b_v after the projections (HF Qwen semantics) */
    uint32_t tied_lm_head; /* 1: logits use the embedding table */
    uint32_t q4_0;         /* 1: linear weights + embedding are Q4_0 blocks; 0: fp32 */
    uint32_t kv_bf16;      /* 1: round K/V to bf16 when written to the cache */
    uint32_t w_f16;        /* 1 (with q4_0 = 0): linear weights and embedding rounded to fp16 (quant_mode 1) */
    uint32_t w_g64;        /* 1 (with q4_0 = 0): linear weights and embedding through the reference's
                              group-64 codec, quantized and dequantized (quant_mode 2) */
} VxoConfig;

typedef struct VxoEngine VxoEngine;

/* Synthesizes the seeded model of the benchmark recipe: linear weights N(0, sigma) (quantized to
 * Q4_0 when cfg->q4_0), norm gains 1.0 (norm_sigma == 0) or N(1, norm_sigma), biases N(0, sigma).
 * layers_to_build < num_layers builds only the first layers (bounded CPU samples). */
VxoEngine* vxo_engine_create(const VxoConfig* cfg, uint64_t seed, float sigma, float norm_sigma,
                             uint32_t layers_to_build, int threads);
void vxo_engine_destroy(VxoEngine* e);
/* One forward step at position pos; writes logits (vocab floats) and returns the argmax. */
uint32_t vxo_engine_forward(VxoEngine* e, uint32_t token, uint64_t pos, float* logits);
/* Same, stopping after `layers` layers (then final norm + head); used for bounded timing. */
uint32_t vxo_engine_forward_layers(VxoEngine* e, uint32_t token, uint64_t pos, uint32_t layers,
                                   float* logits);
void vxo_engine_reset(VxoEngine* e);
void vxo_engine_set_threads(VxoEngine* e, int threads);
/* Direct access to a synthesized tensor (for tests): returns bytes and pointer. */
const void* vxo_engine_tensor(const VxoEngine* e, uint32_t kind, uint32_t layer, uint64_t* nbytes);
const float* vxo_engine_hidden(const VxoEngine* e);

/* Emulated hand-off used by tests to fill KV caches for context configs. */
float* vxo_engine_k_cache(VxoEngine* e);
float* vxo_engine_v_cache(VxoEngine* e);
/* Test harness, not part of the reference's algorithm: for the next forward only, every layer writes
 * its own (bf16-rounded) K and V rows of that position to seen_k / seen_v ([layers][kv_heads * D]) and
 * attends with k_rows / v_rows in their place, so a step can be recomputed on another engine's cache
 * rows, the current position's included. */
void vxo_engine_force_kv(VxoEngine* e, const float* k_rows, const float* v_rows, float* seen_k, float* seen_v);

#ifdef __cplusplus
}
#endif
#endif
