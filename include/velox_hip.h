/*
 * velox_hip.h -- C ABI of the MI355X (gfx950) decode backend for Velox's generated LLM runners.
 *
 * The emitted-runner ABI of the reference is kept: the arena struct, the device-resident decode
 * state, and the per-model `velox_<Model>_{decode,prefill}{_graph_step,}` entry points, now with a
 * hipStream_t. Behind it every kernel is hand-written HIP for gfx950. No torch types appear here:
 * plain pointers, sizes and hipStream_t only.
 *
 * Errors: the step entry points return void like the reference's (src/codegen.rs:2803-2808) and
 * record the first launch error, readable with velox_hip_last_error(); every other entry point
 * returns an int status (0 = success, >0 = hipError_t, <0 = VELOX_HIP_E* argument errors).
 */
#ifndef VELOX_HIP_H
#define VELOX_HIP_H

#include <stddef.h>
#include <stdint.h>
#include <hip/hip_runtime_api.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status codes (negative: argument/plan errors; positive: hipError_t) ---- */
#define VELOX_HIP_OK 0
#define VELOX_HIP_EINVAL (-1)    /* bad argument / unsupported shape */
#define VELOX_HIP_ENOMEM (-2)    /* plan exceeds the VRAM budget (reference diagnostic E002) */
#define VELOX_HIP_ESHAPE (-3)    /* tensor size does not match the plan */
#define VELOX_HIP_ENOTLOADED (-4)
#define VELOX_HIP_ETENSOR (-5)   /* checkpoint tensor missing, or its data_offsets outside the file
                                    (reference diagnostic E013, src/runtime.rs:260-330) */
#define VELOX_HIP_EDTYPE (-6)    /* checkpoint tensor of a dtype the load cannot take (E014) */

/* ---- quant_mode values (src/codegen.rs:1024-1028 defines 0 fp32, 1 fp16, 2 group-64 "Q4",
 *      3/4 fp8). GGML Q4_0 is new to this backend and gets its own value. ---- */
#define VELOX_QUANT_F32 0u
#define VELOX_QUANT_F16 1u
#define VELOX_QUANT_Q4_GROUP64 2u
#define VELOX_QUANT_FP8_E4M3 3u  /* the MLA arena's fp8 weights (the reference's value) */
#define VELOX_QUANT_GGML_Q4_0 5u

/* Tensor kinds for the loaders (one per HF safetensors name the reference resolves,
 * src/runtime.rs:1273-1300). */
enum VeloxHipTensor {
    VELOX_T_EMBED = 1, VELOX_T_Q = 2, VELOX_T_K = 3, VELOX_T_V = 4, VELOX_T_O = 5,
    VELOX_T_GATE = 6, VELOX_T_UP = 7, VELOX_T_DOWN = 8, VELOX_T_ATTN_NORM = 9,
    VELOX_T_MLP_NORM = 10, VELOX_T_FINAL_NORM = 11, VELOX_T_HEAD = 12,
    VELOX_T_BQ = 13, VELOX_T_BK = 14, VELOX_T_BV = 15
};

/* Model constants. Replaces the compile-time VELOX_MODEL_* macros of the emitted module
 * (src/codegen.rs:993-1029) and runtime.rs TransformerConfig (src/runtime.rs:1160-1210); eps,
 * theta and the QKV bias come from the config instead of the reference's hard-coded values. */
typedef struct VeloxHipModelConfig {
    char name[32];
    uint32_t vocab_size, hidden_dim, intermediate_dim, num_layers;
    uint32_t num_heads, num_kv_heads, head_dim, max_seq_len;
    float rms_norm_eps, rope_theta;
    uint32_t qkv_bias;          /* 1: q/k/v biases (Qwen) */
    uint32_t tied_lm_head;      /* 1: LM head reads the embedding table */
    uint32_t quant_mode;        /* VELOX_QUANT_GGML_Q4_0; or the reference's formats (single-sequence decode
                                   only: max_batch and prefill_chunk <= 1): VELOX_QUANT_F32 / _F16 rows
                                   (widths <= 32768), VELOX_QUANT_Q4_GROUP64 (widths multiples of 64) */
    uint32_t attn_splits;       /* split-K partitions over the sequence (<= 64); 0 = automatic */
    uint64_t vram_budget_bytes; /* 0 = 288 GB of HBM3E */
    uint32_t max_batch;         /* sequences of the batched decode step (<= 32; 0 or 1 = single);
                                   sizes the KV pool like B_MAX in src/memory_planner.rs:282-488 */
    uint32_t prefill_chunk;     /* >1: positions of one prompt that velox_hip_prefill_batch runs as the
                                   rows of one batched step (<= 128); 0 or 1 = token-by-token only */
} VeloxHipModelConfig;

typedef struct VeloxHipModel VeloxHipModel; /* opaque: the static memory plan */

/* Layout-identical to VeloxCudaArena (src/codegen.rs:1032-1041): the same eight fields in the same
 * order, so emitted code and runners that fill the struct themselves (velox_cuda_runner.cu:417-431)
 * work unchanged. weight_arena holds the packed Q4_0 nibbles of every linear/embedding matrix,
 * weight_scales their fp16 block scales (codes and scales are split so that both stream with
 * 128-bit loads), norm_weight_arena the fp32 norm gains, biases and the RoPE cos/sin table. The
 * plan an arena belongs to is not a field: the library records it against weight_arena when the
 * arena is created (velox_hip_arena_create) or bound (velox_hip_arena_bind). */
typedef struct VeloxHipArena {
    const uint8_t* weight_arena;
    uint8_t* kv_cache_pool;
    uint8_t* activation_arena;
    uint32_t* host_pinned_ring;
    const uint8_t* norm_weight_arena;
    const uint8_t* weight_scales;
    uint32_t quant_mode;
    uint32_t tied_lm_head;
} VeloxHipArena;

/* Device-resident decode state (src/codegen.rs:1046-1050): one captured graph replays every step. */
typedef struct VeloxDecodeState {
    uint64_t step;
    uint32_t token;
    uint32_t reserved;
} VeloxDecodeState;

#define VELOX_HIP_RING_SIZE 1024u

/* ---- .vlx model sources (the reference's DSL; `velox build model.vlx`, src/cli.rs:1214-1388) ----
 * The model the decode step runs is read from the source's `model Name< const ... >` header
 * (VOCAB, HIDDEN_DIM, INTERMEDIATE_DIM, NUM_LAYERS, NUM_HEADS, NUM_KV_HEADS, HEAD_DIM, S_MAX, B_MAX,
 * ROPE_THETA), its weight declarations (b_q/b_k/b_v: QKV bias; no w_head/w_lm_head: tied head) and
 * its first weight binding's file; eps follows the model name as the reference's lowering sets it
 * (src/ir.rs:549-553), theta falls back on its name rule (src/codegen.rs:962-975). Header
 * constants must be whole numbers in 0..2^32-1. The `target hardware` block gives the planner's
 * budget: floor(vram_capacity * safety_factor) less the driver reserve (src/memory_planner.rs:372-
 * 488) -> vram_budget_bytes (0 without a target block: the default 288 GB). max_seq_len 0 takes
 * S_MAX. The config's max_batch and prefill_chunk stay 0: B_MAX is reported in the target info and
 * the caller chooses the batched rows. quant_mode is GGML Q4_0, this backend's weight format.
 * EINVAL for a malformed source, a missing dimension, or an MLA model (LATENT_KV_DIM), which
 * velox_hip_vlx_mla_config reads. _load reads a file (ENOTLOADED if it cannot be read). */
typedef struct VeloxHipVlxTarget {
    char device[64];
    uint64_t vram_capacity_bytes;
    double safety_factor;
    uint64_t safe_budget_bytes;     /* floor(vram_capacity * safety_factor) */
    uint64_t system_reserve_bytes;  /* driver + stream ring reserve */
    uint32_t b_max, s_max;          /* the model header's B_MAX and S_MAX (0 if absent) */
    char weights_file[256];         /* the first safetensors("file", ...) binding ("" if none): the
                                       checkpoint the CLI runs the model on (src/cli.rs:1400-1414) */
} VeloxHipVlxTarget;
int velox_hip_vlx_config(const char* source, uint32_t max_seq_len, VeloxHipModelConfig* out,
                         VeloxHipVlxTarget* target);
int velox_hip_vlx_load(const char* path, uint32_t max_seq_len, VeloxHipModelConfig* out, VeloxHipVlxTarget* target);

/* Built-in benchmark configurations (1, 2, 3, 5), each declared as a .vlx source targeting one
 * MI355X and read by velox_hip_vlx_config. which: "smollm_135m", "llama3_8b", "qwen2_5_7b",
 * "qwen2_72b" (also the config's name). max_seq_len 0 keeps the source's S_MAX. */
int velox_hip_builtin_config(const char* which, uint32_t max_seq_len, VeloxHipModelConfig* out);

/* ---- plan (memory_planner, src/memory_planner.rs:282-488) ---- */
int velox_hip_model_create(const VeloxHipModelConfig* cfg, VeloxHipModel** out);
void velox_hip_model_destroy(VeloxHipModel* m);
/* The planned configuration: the input, with attn_splits = the split count the planner chose when
 * the input left it 0. */
int velox_hip_model_config(const VeloxHipModel* m, VeloxHipModelConfig* out);
int velox_hip_model_arena_bytes(const VeloxHipModel* m, uint64_t* weight_bytes, uint64_t* scale_bytes,
                                uint64_t* norm_bytes, uint64_t* kv_bytes, uint64_t* act_bytes);
/* HBM bytes one decode step must move at position pos (weights once + KV read/write). */
uint64_t velox_hip_model_step_bytes(const VeloxHipModel* m, uint64_t pos);
/* Byte offset of the fp32 logits / hidden state inside activation_arena. */
uint64_t velox_hip_model_logits_offset(const VeloxHipModel* m);
uint64_t velox_hip_model_hidden_offset(const VeloxHipModel* m);

/* ---- arena (velox_cuda_runner.cu:417-431: cudaMalloc x3 + mapped host ring) ----
 * create: one hipMalloc holding every device region (256-byte aligned) plus the mapped host ring,
 * initialized (zeroed, RoPE table) and recorded against its weight_arena.
 * bind: the reference runner's pattern -- the caller allocated the buffers itself, each at least
 * the size velox_hip_model_arena_bytes gives (weights, scales, norms, KV pool, activations; a
 * mapped ring of VELOX_HIP_RING_SIZE * max(1, max_batch) entries), and filled the eight fields with
 * quant_mode and tied_lm_head equal to the plan's. bind initializes those buffers as create does
 * and records the plan; EINVAL for a missing buffer, mismatching flags or a weight_arena already
 * recorded.
 * destroy: forgets the arena; frees the buffers only if create allocated them.
 * model: the plan an arena was created or bound with (NULL for an unknown arena). */
int velox_hip_arena_create(const VeloxHipModel* m, VeloxHipArena* out);
int velox_hip_arena_bind(const VeloxHipModel* m, VeloxHipArena* a);
int velox_hip_arena_destroy(VeloxHipArena* a);
const VeloxHipModel* velox_hip_arena_model(const VeloxHipArena* a);

/* ---- loaders (velox_cuda_runner.cu:154-199 stream_tensor_converted) ----
 * q4_0: host GGML Q4_0 blocks, row-major [rows][in/32] x 18 B, for a matrix kind of `layer`.
 * rows: host fp32 (quant_mode VELOX_QUANT_F32) or fp16 (VELOX_QUANT_F16) rows [rows][in] of a
 *   matrix kind, stored as the reference's weight arena holds them (src/codegen.rs:1024-1028); or
 *   host fp32 rows of a VELOX_QUANT_Q4_GROUP64 arena, quantized on the device by the reference's
 *   group-64 rule (velox_cuda_runner.cu:174-197, src/codegen.rs:2337-2370) into the tiled layout;
 *   EINVAL on a Q4_0 arena, as q4_0 is on any other arena.
 * f32: host fp32 vector (norm gains, biases). All upload (and repack) on `stream`. */
int velox_hip_load_q4_0(VeloxHipArena* a, int kind, uint32_t layer, const void* blocks, uint64_t nbytes,
                        hipStream_t stream);
int velox_hip_load_rows(VeloxHipArena* a, int kind, uint32_t layer, const void* rows, uint64_t nbytes,
                        hipStream_t stream);
int velox_hip_load_f32(VeloxHipArena* a, int kind, uint32_t layer, const float* data, uint64_t count,
                       hipStream_t stream);
/* Element types of checkpoint tensors (safetensors "F32", "F16", "BF16"). */
#define VELOX_DT_F32 0u
#define VELOX_DT_F16 1u
#define VELOX_DT_BF16 2u
/* Any tensor kind from host data as a checkpoint stores it (row-major [rows][in] fp32, fp16 or bf16;
 * vectors [n]), converted on the device into the arena's format, as the reference runner's
 * stream_tensor_converted does (velox_cuda_runner.cu:154-199): fp32 or fp16 rows (fp16 rounded to
 * nearest even), the reference's group-64 format, or GGML Q4_0 (quantized on the device, bit-exact
 * with velox_hip_q4_0_quantize). Matrices go through the device in chunks of at most 64 MiB of
 * fp32; norm gains and biases are widened to fp32. ESHAPE when nbytes is not the kind's size,
 * EDTYPE for another dtype; the tied head takes no separate load (EINVAL). */
int velox_hip_load_tensor(VeloxHipArena* a, int kind, uint32_t layer, const void* data, uint64_t nbytes,
                          uint32_t dtype, hipStream_t stream);
/* Synthesizes the whole seeded model on the device (linear weights N(0,sigma) quantized to Q4_0,
 * as fp32 / fp16 rows, or quantized to group-64, per quant_mode; norm gains 1 or N(1,norm_sigma), biases
 * N(0,sigma)), bit-identical to the oracle's recipe. */
int velox_hip_synthesize_model(VeloxHipArena* a, uint64_t seed, float sigma, float norm_sigma,
                               hipStream_t stream);
/* Fills layer `layer`'s KV cache positions [0, n_pos) with bf16 values seed-generated N(0, sigma). */
int velox_hip_fill_kv(VeloxHipArena* a, uint32_t layer, uint32_t n_pos, uint64_t seed, float sigma,
                      hipStream_t stream);

/* ---- decode state / prompt ---- */
/* Stages a prompt for teacher-forced prefill through the decode graph: while step+1 < n, the
 * step's next token is prompt[step+1] instead of the argmax. */
int velox_hip_set_prompt(VeloxHipArena* a, const uint32_t* tokens, uint32_t n, hipStream_t stream);
int velox_hip_set_state(VeloxHipArena* a, uint64_t step, uint32_t token, hipStream_t stream);
int velox_hip_get_state(const VeloxHipArena* a, VeloxDecodeState* out, hipStream_t stream);

/* ---- the decode step (src/codegen.rs:2803-3253) ----
 * graph_step reads (step, token) from the device state, runs embed -> L x [QKV, attention,
 * o_proj+res, gate/up+SwiGLU, down+res] -> norm+LM head+argmax, writes ring[step & 1023] and
 * advances the state. decode/prefill set the state first. active_mask bit 0 predicates every
 * kernel. Capturable into a hipGraph; no allocation, no host sync. */
void velox_hip_decode_graph_step(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_hip_decode(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                      hipStream_t stream);
void velox_hip_prefill_graph_step(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_hip_prefill(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                       hipStream_t stream);
int velox_hip_last_error(void);

/* The single-sequence step runs QKV and attention as one launch per layer where the plan allows it
 * (Q4_0, head size 128, KV heads a multiple of 8, 4 or 8 q heads per KV head, up to 2048 positions,
 * the planner's own split count) and the device deals workgroup b of a launch to XCD (b + o) % 8, o
 * fixed per launch (checked when the arena is created or bound). No counterpart in the reference (whose step always launches
 * the two apart): set_fused_attention(0) makes steps recorded afterwards use the two launches
 * (process-wide; 1 restores the default). fused_attention_status reports the splits per KV head
 * the arena's steps use fused (0: two launches) and the fused launches' error bits (1: a KV head's
 * workgroups ran on two XCDs, 2: a wait expired; 0 after correct steps; synchronous). */
void velox_hip_set_fused_attention(int enable);
int velox_hip_fused_attention_status(const VeloxHipArena* a, uint32_t* splits_used, uint32_t* errors);

/* 0 when the arena's plan has `want`'s dimensions -- vocabulary, hidden, FFN, heads, KV heads, head
 * size, QKV bias, head tying, eps, theta, and depth unless want->num_layers is 0 -- else EINVAL
 * (the plan's name, context, batch rows and weight format are not compared). */
int velox_hip_arena_check(const VeloxHipArena* a, const VeloxHipModelConfig* want);

/* Per-model entry points with the reference's names (src/runners/tinystories_smollm.cu:1520,
 * 2383, 2388, 3251) for the builtin configurations; each runs only on an arena whose plan has that
 * model's dimensions (velox_hip_arena_check, at any depth), else records EINVAL. `velox_amd.build
 * --model X.vlx` generates the same four for the model any source declares. */
void velox_SmolLM_135M_decode_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_SmolLM_135M_decode_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                                  hipStream_t stream);
void velox_SmolLM_135M_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_SmolLM_135M_prefill_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                                   hipStream_t stream);
void velox_Llama3_8B_decode_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_Llama3_8B_decode_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                                hipStream_t stream);
void velox_Llama3_8B_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_Llama3_8B_prefill_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                                 hipStream_t stream);
void velox_Qwen2_5_7B_decode_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_Qwen2_5_7B_decode_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                                 hipStream_t stream);
void velox_Qwen2_72B_decode_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_Qwen2_72B_decode_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                                hipStream_t stream);
void velox_Qwen2_5_7B_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_Qwen2_5_7B_prefill_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                                  hipStream_t stream);
void velox_Qwen2_72B_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_Qwen2_72B_prefill_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                                 hipStream_t stream);

/* ---- per-kernel entry points (device pointers; for parity tests and benchmarks) ---- */

/* ---- batched decode of independent sequences (src/runners/velox_cuda_runner_k2.cu:553-1088 batched
 *      kernels; arena planned with max_batch > 1, src/memory_planner.rs:282-488 B_MAX) ----
 * Sequence b owns KV caches, a decode state, a prompt for teacher forcing and ring
 * host_pinned_ring[b * VELOX_HIP_RING_SIZE ...]; its logits are at logits_offset + b * vocab * 4 of
 * the activation arena and its hidden state at hidden_offset + b * hidden_dim * 4. */
int velox_hip_model_batch_layout(const VeloxHipModel* m, uint32_t* max_batch, uint64_t* logits_offset,
                                 uint64_t* hidden_offset);
/* Algorithmic HBM bytes of one batched step with every sequence at position pos. */
uint64_t velox_hip_model_batch_step_bytes(const VeloxHipModel* m, uint32_t batch, uint64_t pos);
int velox_hip_batch_set_prompt(VeloxHipArena* a, uint32_t seq, const uint32_t* tokens, uint32_t n, hipStream_t stream);
int velox_hip_batch_set_state(VeloxHipArena* a, uint32_t seq, uint64_t step, uint32_t token, hipStream_t stream);
int velox_hip_batch_get_state(const VeloxHipArena* a, uint32_t seq, VeloxDecodeState* out, hipStream_t stream);
/* Seeded N(0, sigma) bf16 context of sequence seq (seq 0: the same values as velox_hip_fill_kv). */
int velox_hip_fill_kv_seq(VeloxHipArena* a, uint32_t layer, uint32_t seq, uint32_t n_pos, uint64_t seed, float sigma,
                          hipStream_t stream);
/* One decode step of sequences 0 .. batch-1 (batch <= max_batch), each at its own state; capturable
 * like velox_hip_decode_graph_step. Weights are read once per step for all sequences (MFMA GEMMs). */
void velox_hip_decode_batch_graph_step(VeloxHipArena* ctx, uint32_t batch, uint64_t active_mask, hipStream_t stream);

/* ---- batched prefill (replaces the token-by-token prefill loop of velox_cuda_runner.cu:493-512
 *      and the K2 runner's velox_batched_prefill_q4, velox_cuda_runner_k2.cu:1614-1711, which takes
 *      at most 16 tokens in one pass and falls back to sequential decode beyond; the runtime form of
 *      the DSL's chunked_prefill scope and its chunk_size, src/ast.rs:632-654; arena planned with
 *      prefill_chunk > 1) ----
 * Positions [pos0, pos0 + n_tokens) of the staged prompt run in chunks of up to prefill_chunk
 * positions, each chunk as the rows of one batched step (the weights are read once per chunk):
 * every row's K/V row goes into the single-sequence KV cache, then each row attends over
 * [0, its position]. Afterwards the decode state is {pos0 + n_tokens, the next prompt token, or
 * the last row's argmax past the prompt} -- what n_tokens token-by-token prefill steps leave --,
 * ring[p % VELOX_HIP_RING_SIZE] holds each position's argmax and the last chunk's logits are at
 * the batch layout's logits_offset (row r = position of the chunk's r-th row). Positions must lie
 * inside the prompt last staged with velox_hip_set_prompt and below max_seq_len (else EINVAL).
 * Returns this call's first launch error (an earlier unread error stays for velox_hip_last_error). */
int velox_hip_prefill_batch(VeloxHipArena* ctx, uint64_t pos0, uint32_t n_tokens, uint64_t active_mask,
                            hipStream_t stream);

/* Q4_0 matrix in the tiled device layout. Row r, block b of an [n][k] matrix lives in lane
 * (r % (64/s_lanes)) * s_lanes + b % s_lanes of iteration b / s_lanes of tile r / (64/s_lanes):
 * codes uint4 [n_tiles][n_iter][64], scales fp16 [n_tiles][n_iter][64]. */
typedef struct VeloxHipQ4Matrix {
    void* codes;
    void* scales;
    uint32_t n, k;         /* rows, columns (k % 32 == 0) */
    uint32_t s_lanes;      /* lanes per row: 4, 8, 16, 32 or 64 */
    uint32_t n_tiles, n_iter;
    uint32_t paired;       /* 1: tiles interleave gate/up rows for the fused SwiGLU epilogue */
    uint32_t format;       /* 0: GGML Q4_0 (slot = fp16 d, w = d (q - 8)); VELOX_QUANT_Q4_GROUP64: the
                              reference's group-64 format (k % 64 == 0; the slot of block 2g holds the
                              group's fp16 scale s, of block 2g + 1 its fp16 minimum m; w = fmaf(q, s, m)) */
} VeloxHipQ4Matrix;

/* Descriptor of a weight matrix inside an arena (kind VELOX_T_Q/K/V return the fused QKV matrix
 * and GATE/UP the paired gate/up matrix; row0 receives the kind's first logical row). */
int velox_hip_arena_matrix(const VeloxHipArena* a, int kind, uint32_t layer, VeloxHipQ4Matrix* out,
                           uint32_t* row0);
/* Device pointer of a norm gain / bias vector inside an arena and its element count. */
int velox_hip_arena_vector(const VeloxHipArena* a, int kind, uint32_t layer, const float** out, uint64_t* count);

/* Fills n_tiles/n_iter and returns the byte sizes for a matrix (s_lanes 0 = automatic). */
int velox_hip_q4_layout(uint32_t n, uint32_t k, uint32_t s_lanes, uint32_t paired, VeloxHipQ4Matrix* m,
                        uint64_t* code_bytes, uint64_t* scale_bytes);
/* GGML Q4_0 blocks (device) of `rows` rows -> tiled layout rows [row0, row0+rows) (paired: pair_part
 * 0 = gate rows, 1 = up rows). Zero padding is the caller's (the arena loaders clear it). */
int velox_hip_q4_0_repack(const void* d_blocks, uint32_t rows, uint32_t row0, uint32_t pair_part,
                          const VeloxHipQ4Matrix* m, hipStream_t stream);
/* Tiled layout -> dense fp32 [n][k] (paired: logical rows gate 0..n/2-1 then up). Bit-exact d*(q-8)
 * (format 0) or fmaf(q, s, m) (group-64). */
int velox_hip_q4_0_dequant(const VeloxHipQ4Matrix* m, float* d_out, hipStream_t stream);
/* fp32 [rows][k] -> GGML Q4_0 blocks, the GGML rounding rule restated (bit-exact with the oracle). */
int velox_hip_q4_0_quantize(const float* d_x, uint32_t rows, uint32_t k, void* d_blocks, hipStream_t stream);
/* The reference's group-64 quantizer, velox_cuda_quantize_q4_group64_kernel (src/codegen.rs:2337-2370):
 * fp32 [n_groups][64] -> d_packed [n_groups][8] words (q0|q2<<4|q4<<8|q6<<12|q1<<16|q3<<20|q5<<24|q7<<28
 * of elements 8w..8w+7) and d_scale_min [n_groups][2] fp16 (s, m), in the reference's own layout. */
int velox_hip_g64_quantize(const float* d_x, uint64_t n_groups, uint32_t* d_packed, uint16_t* d_scale_min,
                           hipStream_t stream);
/* fp32 rows [rows][k] (device) -> group-64 codes of a tiled matrix (format VELOX_QUANT_Q4_GROUP64) at
 * logical rows [row0, row0+rows) (paired: pair_part 0 = gate rows, 1 = up rows); the same codes and
 * scales as velox_hip_g64_quantize. */
int velox_hip_g64_pack(const float* d_rows, uint32_t rows, uint32_t row0, uint32_t pair_part,
                       const VeloxHipQ4Matrix* m, hipStream_t stream);
/* Seeded N(mean, sigma) fill identical to the oracle's vxo_fill_normal. */
int velox_hip_fill_normal(float* d_out, uint64_t n, uint64_t seed, uint64_t tag, float sigma, float mean,
                          hipStream_t stream);

/* Fused GEMV y = W x with epilogues. mode 0: y = Wx (+bias); 1: y = res + Wx; 2: paired SwiGLU
 * y[j] = silu(g_j) * u_j; gain != NULL applies RMSNorm(x) * gain first (eps). */
#define VELOX_GEMV_STORE 0
#define VELOX_GEMV_RESIDUAL 1
#define VELOX_GEMV_SWIGLU 2
int velox_hip_gemv_q4_0(const VeloxHipQ4Matrix* m, const float* d_x, const float* d_gain, float eps,
                        const float* d_bias, const float* d_res, float* d_y, int mode, hipStream_t stream);
/* Fused RMSNorm + LM head + greedy argmax: logits and the winning index (lowest index on ties).
 * Allocates its candidate buffer per call and returns after synchronizing the stream. */
int velox_hip_lm_head_argmax(const VeloxHipQ4Matrix* m, const float* d_x, const float* d_gain, float eps,
                             float* d_logits, uint32_t* d_token, hipStream_t stream);
/* velox_hip_lm_head_argmax for callers that cannot allocate device memory (code under hipGraph
 * capture, serving loops, harnesses that forbid hipMalloc). No counterpart in the reference: its
 * emitted step never allocates because the runner sizes every buffer up front. Same arguments and
 * results as velox_hip_lm_head_argmax, but the per-workgroup candidates live in a fixed device
 * array of the library (512 candidates, 4 KiB per GPU, held until the process ends; EINVAL if a
 * matrix needed more), so the call allocates nothing and does not synchronize. Calls that overlap
 * on one GPU (concurrent streams or threads) share that array and race. The first call on a device
 * looks the array's address up (hipGetSymbolAddress, no stream work): make that first call eagerly,
 * then the call can be captured into a HIP graph (it records kernel launches only) and replayed. */
int velox_hip_lm_head_argmax_noalloc(const VeloxHipQ4Matrix* m, const float* d_x, const float* d_gain, float eps,
                                     float* d_logits, uint32_t* d_token, hipStream_t stream);
/* Standalone two-stage argmax over n fp32 values (strict '>' lowest-index rule). */
int velox_hip_argmax_f32(const float* d_x, uint32_t n, uint32_t* d_out, hipStream_t stream);
/* Batched GEMM of `batch` <= 32 sequences (src/runners/velox_cuda_runner_k2.cu:553-997, batched
 * Q4 kernels), on MFMA: d_x16 is [batch][ldx] fp16. mode VELOX_GEMV_STORE: y[m][n] = W x_m (+ bias);
 * VELOX_GEMV_RESIDUAL: y[m][n] += W x_m; VELOX_GEMV_SWIGLU (paired layout): d_out16[m][j] =
 * fp16(silu(gate) * up). Row strides ldx, ldy, ldo in elements. */
int velox_hip_gemm_q4_0_batch(const VeloxHipQ4Matrix* m, const uint16_t* d_x16, uint32_t batch, uint32_t ldx,
                              const float* d_bias, float* d_y, uint32_t ldy, uint16_t* d_out16, uint32_t ldo,
                              int mode, hipStream_t stream);
/* The batched GEMM's MFMA operand layout ("M-layout"), a second copy of a tiled matrix that arenas
 * planned for more than one batched row keep for every matrix: 16-row tiles (paired: gate tile u at
 * 2u, up tile u at 2u + 1) x groups of four blocks; per (tile, group) 64 words of 16 bytes, lane l
 * holding dword l / 16 (elements 8(l/16) .. +7, element e at bit 16 (e & 1) + 4 (e >> 1)) of blocks
 * 4j .. 4j+3 of row l % 16; fp16 scales [tile][group][row][4]. _bytes gives the sizes, _mlayout
 * builds the copy from the tiled matrix. */
int velox_hip_q4_mlayout_bytes(const VeloxHipQ4Matrix* m, uint64_t* code_bytes, uint64_t* scale_bytes);
int velox_hip_q4_mlayout(const VeloxHipQ4Matrix* m, void* d_codes, void* d_scales, hipStream_t stream);
/* velox_hip_gemm_q4_0_batch over an M-layout copy (the batched decode and prefill steps' GEMM).
 * Activations: element k of row m at d_x16[m * ldx + (k / 32) * xbs + k % 32] -- row-major with
 * xbs = 32 (0 means 32), or block-major [k / 32][rows][32] with ldx = 32, xbs = 32 * rows, the layout
 * the batched steps use (one operand load is 1 KiB contiguous); d_out16 (SWIGLU) likewise with
 * (ldo, obs). batch <= 128; ksplit 1..8 splits K over workgroup rows (STORE and RESIDUAL), the
 * partials going through d_part [ksplit][batch][ldy] and summed in split order (+ bias for STORE)
 * into y. */
int velox_hip_gemm_q4_0_batch_m(const VeloxHipQ4Matrix* m, const void* d_mcodes, const void* d_mscales,
                                const uint16_t* d_x16, uint32_t batch, uint32_t ldx, uint32_t xbs, const float* d_bias,
                                float* d_y, uint32_t ldy, uint16_t* d_out16, uint32_t ldo, uint32_t obs, int mode,
                                uint32_t ksplit, float* d_part, hipStream_t stream);
/* y = rmsnorm(x) * w (src/runtime.rs:588-601). */
int velox_hip_rmsnorm(const float* d_x, const float* d_w, uint32_t n, float eps, float* d_y, hipStream_t stream);
/* Decode attention for one layer at position pos: RoPE on q and the new k (table cos/sin of
 * pos*theta^(-2j/D)), bf16 K/V append at pos, split-K online softmax with an LSE merge.
 * qkv: fp32 [hq*d | hkv*d | hkv*d]; out: fp32 [hq*d]. kv_layer: bf16, s_cap = s_max rounded up to
 * a multiple of 32 positions; the K plane [hkv][s_cap][d] row-major, then the V plane
 * [hkv][s_cap/32][d][32]: per block of 32 positions, dimension-major, position r (0..31) of a block
 * in slot 8*((r%16)/4) + 4*(r/16) + r%4 (the order the P.V MFMA consumes). The arenas' KV pools use
 * this layout per layer (and sequence). */
int velox_hip_attention_decode(const float* d_qkv, uint16_t* d_kv_layer, uint32_t hq, uint32_t hkv,
                               uint32_t d, uint32_t s_max, uint32_t pos, float theta, uint32_t splits,
                               float* d_out, hipStream_t stream);

/* ---- runner (velox_cuda_runner.cu:327-726 flow: plan, alloc, load, capture, prefill, decode) ---- */
typedef struct VeloxHipRunOptions {
    const char* model;       /* builtin config name (unless model_file or weights_path is given) */
    uint32_t max_seq_len;    /* 0 = prompt_len + warmup + steps + 1 */
    uint32_t prompt_len;     /* random prompt tokens (seeded) */
    uint32_t warmup;         /* untimed decode steps */
    uint32_t steps;          /* timed decode steps */
    uint64_t seed;
    float sigma, norm_sigma;
    uint32_t use_graph;      /* 1: hipGraph capture + replay (reference default) */
    uint32_t num_layers;     /* 0 = config value (fewer layers for parity runs) */
    uint32_t kernel_passes;  /* >0: afterwards time the gate/up GEMV alone over all layers this often */
    uint32_t verbose;
    const uint32_t* prompt_tokens; /* NULL: prompt_len seeded random ids; else prompt_len explicit ids
                                      (the runner's --tokens, src/cli.rs:655-661) */
    uint32_t context_len;    /* >0: positions [0, context_len) of every layer's KV cache hold a seeded
                                N(0,1) bf16 context (velox_hip_fill_kv) and decoding starts at
                                position context_len with the first prompt token
                                (src/runners/velox_cuda_runner_k2.cu:1789 --context-len) */
    uint32_t batch;          /* >1: decode `batch` independent sequences per step (own seeded prompt and
                                context each); tokens/report cover sequence 0, tok_per_s all of them */
    const char* weights_path;/* NULL: synthetic weights of `model`; else a checkpoint (the runner's
                                --weights): a GGUF Q4_0 file (by its magic), whose metadata defines
                                the model, or a safetensors file, run on model_file's or model's
                                configuration, or with both NULL on the builtin one its tensor shapes
                                match (velox_hip_st_config), converted to the quant_mode
                                `unquantized` selects */
    uint32_t prefill_chunk;  /* >1 (single sequence, no context_len): the prompt runs through
                                velox_hip_prefill_batch in chunks of this many positions (<= 128)
                                instead of one decode step each */
    const char* model_file;  /* non-NULL: the model is read from this .vlx source (velox_hip_vlx_load),
                                its target block setting the VRAM budget; `model` is then ignored */
    uint32_t unquantized;    /* 0: GGML Q4_0 weights; else the reference's fp32 weights (single sequence
                                only): 1 as fp32 rows (a build without --quantize, src/cli.rs:1214-1388),
                                2 converted to fp16 rows (--quantize f16), 3 quantized to group-64
                                (--quantize q4_0, velox_cuda_runner.cu:356-372). A safetensors
                                checkpoint is converted on the device to the format chosen (0:
                                quantized to GGML Q4_0 there) */
    const VeloxHipModelConfig* model_config; /* non-NULL: run this configuration (a generated runner's
                                model) instead of model_file / model; a checkpoint must fit it */
    void (*decode_step)(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
                             /* non-NULL: the single-sequence step the run captures and replays (a
                                generated runner's velox_<Model>_decode_graph_step_hip); NULL:
                                velox_hip_decode_graph_step */
    uint32_t attn_splits;    /* >0: the configuration's attn_splits (split-K attention with that many
                                splits, never the fused QKV + attention launch); 0: the planner's */
} VeloxHipRunOptions;

typedef struct VeloxHipRunReport {
    double load_ms, prefill_ms, decode_ms;  /* decode_ms over `steps` timed steps */
    double tok_per_s;                       /* steps / decode seconds */
    double bytes_per_step;                  /* mean algorithmic HBM bytes per timed step */
    double hbm_gbps;
    double wall_ms;                         /* host clock around the timed steps (synced both sides) */
    double kernel_us;                       /* mean duration of one fused gate/up GEMV launch */
    double kernel_bytes;                    /* algorithmic bytes of that launch */
    uint32_t kernel_launches;               /* launches averaged over (all layers, several passes) */
    uint32_t n_tokens;                      /* tokens written to `tokens` */
    uint32_t first_token;                   /* the argmax after the last prompt position */
    int status;
    uint32_t first_position;                /* position whose argmax is tokens[0] (the first decoded
                                               position: context_len) */
    /* per-step device time of the timed steps (an event after every step on the step's stream):
       median, 99th percentile (nearest rank) and maximum; the mean is decode_ms / steps */
    double step_p50_ms, step_p99_ms, step_max_ms;
} VeloxHipRunReport;

/* Runs the whole flow; tokens (capacity max_tokens) receives, from position first_position on, the
 * argmax after every position (prompt-forced positions included), drained from the 1024-entry ring
 * at least once per 1024 positions. */
int velox_hip_run(const VeloxHipRunOptions* opt, uint32_t* tokens, uint32_t max_tokens, VeloxHipRunReport* rep);

/* The runner program (argv and stdout report of the reference's runner, velox_cuda_runner.cu:327-726,
 * parsed by src/cli.rs:706-733): the generic velox_hip_runner passes NULL, NULL; a runner generated
 * for one model (velox_amd.build --model X.vlx) passes its configuration and its named graph step.
 * Returns the process exit code (0, or 1 with a message on stderr). */
int velox_hip_runner_main(int argc, char** argv, const VeloxHipModelConfig* model,
                          void (*decode_step)(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream));
/* Records `status` as the step error velox_hip_last_error() returns, unless one is recorded already
 * (generated entry points report an arena of another model through it). */
void velox_hip_record_error(int status);

/* ---- GGUF checkpoints (GGML's container, read by the reference's K2 runner,
 * src/runners/velox_cuda_runner_k2.cu:48-196; llama.cpp tensor names as at :1918-1963) ----
 * Memory-maps the file and parses header, metadata and tensor directory (bounds checked).
 * velox_hip_gguf_config derives the model from the {arch}.* metadata (vocab from token_embd,
 * QKV bias from blk.0.attn_q.bias, tied head when output.weight is absent); velox_hip_gguf_load
 * loads every Q4_0 matrix and fp32/fp16 vector into an arena planned with that config. For arch
 * "llama" the q/k rows (and biases) return from llama.cpp's pairwise order to rotate-half order. */
typedef struct VeloxHipGguf VeloxHipGguf;
int velox_hip_gguf_open(const char* path, VeloxHipGguf** out);
void velox_hip_gguf_close(VeloxHipGguf* g);
uint64_t velox_hip_gguf_tensor_count(const VeloxHipGguf* g);
/* dims: 4 entries, GGML order (dims[0] is the contiguous one); nbytes 0 for unknown types */
int velox_hip_gguf_tensor_info(const VeloxHipGguf* g, uint64_t i, char* name, uint32_t name_cap, uint32_t* type,
                               uint32_t* n_dims, uint64_t* dims, uint64_t* nbytes);
int velox_hip_gguf_config(const VeloxHipGguf* g, uint32_t max_seq_len, VeloxHipModelConfig* out);
int velox_hip_gguf_load(VeloxHipArena* arena, const VeloxHipGguf* g, hipStream_t stream);

/* ---- safetensors checkpoints (the reference runner's --weights file: velox_cuda_runner.cu:60-199,
 * 390-393; its CPU engine's MmapSafetensors, src/runtime.rs:200-520; Hugging Face tensor names as
 * load_safetensors resolves them, src/runtime.rs:1258-1300) ----
 * open: memory-maps the file and parses the 8-byte header length and the UTF-8 JSON header;
 *   ENOTLOADED when the file cannot be opened, EINVAL for a file under 8 bytes, a header length
 *   past the end of the file, invalid UTF-8 or JSON that is not an object of {dtype, shape,
 *   data_offsets} entries ("__metadata__" is skipped).
 * find / tensor_data: "lm_head.weight" falls back on "model.embed_tokens.weight" when absent (the
 *   tied head); ETENSOR (E013) for a missing name or data_offsets inverted or past the end of the
 *   file, EDTYPE (E014) when the stored dtype is not `dtype`, ESHAPE when the byte count is not the
 *   shape's.
 * config: the model of a file (vocabulary, depth, QKV bias and head tying from its tensors; head
 *   count and size from the builtin configuration with the same layer shapes, which also gives eps
 *   and theta); EINVAL when none matches. quant_mode is VELOX_QUANT_F32, the reference runner's
 *   default.
 * check: every tensor the configuration needs is present, F32/F16/BF16, in the file and shaped
 *   [out][in] ([n] for vectors).
 * load: check, then every tensor through velox_hip_load_tensor into an arena planned with the
 *   configuration (converted to its quant_mode on the device). */
typedef struct VeloxHipSafetensors VeloxHipSafetensors;
int velox_hip_st_open(const char* path, VeloxHipSafetensors** out);
void velox_hip_st_close(VeloxHipSafetensors* st);
uint64_t velox_hip_st_tensor_count(const VeloxHipSafetensors* st);
/* dtype: 16 bytes; shape: up to 8 entries; begin/end: data_offsets as written */
int velox_hip_st_tensor_info(const VeloxHipSafetensors* st, uint64_t i, char* name, uint32_t name_cap, char* dtype,
                             uint64_t* shape, uint32_t* n_dims, uint64_t* begin, uint64_t* end);
int velox_hip_st_find(const VeloxHipSafetensors* st, const char* name, uint64_t* index);
int velox_hip_st_tensor_data(const VeloxHipSafetensors* st, const char* name, const char* dtype, const void** data,
                             uint64_t* nbytes);
int velox_hip_st_config(const VeloxHipSafetensors* st, uint32_t max_seq_len, VeloxHipModelConfig* out);
int velox_hip_st_check(const VeloxHipSafetensors* st, const VeloxHipModelConfig* cfg);
int velox_hip_st_load(VeloxHipArena* arena, const VeloxHipSafetensors* st, hipStream_t stream);

/* ---- Absorbed multi-head latent attention layer (benchmark configuration 4, DeepSeek-V3 form) ----
 * Replaces the reference's MLA step: the emitted velox_cuda_fused_mla_absorbed_attn
 * (src/codegen.rs:2001-2109, launched 1x256 at :2993) and the CPU mla_absorbed_step_f32
 * (src/runtime.rs:845-1044) with its absorbed weights (MlaAbsorptionPass, src/optimizer.rs:138-184).
 * Per head h: q_abs_h = W_uk[h]^T q_nope_h; s_ht = softmax_scale * (q_abs_h . c_t + rope(q_rope_h) .
 * kr_t); ctx_h = softmax_t(s) . c_t; o_h = W_uv[h] ctx_h; hidden += W_o [o_h]. q = W_qb rmsnorm(W_qa x)
 * (q_lora_rank > 0) or W_qb x; [c_t | kr_t] = [rmsnorm(c) | rope(kr)] of W_kva x, appended to the
 * bf16 latent cache. Weights are fp8 e4m3fn with fp32 scales per 128x128 block. The device step
 * takes num_heads a multiple of 16 and a 64-wide rope part; the reduction to the reference's
 * simplified single-head step (one head, no q LoRA, no rope part, kv_norm 0, identity W_kvb) holds
 * in the CPU oracle only, which is how the DeepSeek-V3 form is tied to the reference. */
typedef struct VeloxHipMlaConfig {
    uint32_t hidden_dim, num_heads, q_lora_rank, kv_lora_rank, qk_nope_dim, qk_rope_dim, v_head_dim;
    uint32_t num_layers, max_seq_len, max_batch; /* max_batch <= 32 */
    uint32_t kv_norm;                            /* 1: RMSNorm on the latent (kv_a_layernorm) */
    uint32_t attn_splits;                        /* 0: planner's choice */
    float rms_norm_eps, rope_theta, softmax_scale; /* softmax_scale 0: 1/sqrt(qk_nope_dim + qk_rope_dim) */
    uint32_t reserved;
    uint64_t vram_budget_bytes;                  /* 0: 288e9 */
} VeloxHipMlaConfig;

typedef struct VeloxHipMla VeloxHipMla;

/* An MLA model's .vlx source (LATENT_KV_DIM, Q_LATENT_DIM, ROPE_DIM, HEAD_DIM as nope and v width,
 * as examples/deepseek_v3_mla.vlx declares them) -> the MLA layer configuration; budget as
 * velox_hip_vlx_config. max_seq_len / max_batch 0 take S_MAX / B_MAX (at most 32). */
int velox_hip_vlx_mla_config(const char* source, uint32_t max_seq_len, uint32_t max_batch, VeloxHipMlaConfig* out,
                             VeloxHipVlxTarget* target);

/* weight kinds: fp8 matrices (row-major [rows][cols] as in the checkpoint) and fp32 gains */
enum {
    VELOX_MLA_Q_A = 1,       /* [q_lora_rank][hidden_dim] */
    VELOX_MLA_Q_B = 2,       /* [num_heads * (nope + rope)][q_lora_rank or hidden_dim] */
    VELOX_MLA_KV_A = 3,      /* [kv_lora_rank + rope][hidden_dim] */
    VELOX_MLA_KV_B = 4,      /* [num_heads * (nope + v)][kv_lora_rank]: per head its nope k rows, then v rows */
    VELOX_MLA_O = 5,         /* [hidden_dim][num_heads * v] */
    VELOX_MLA_NORM = 6,      /* [hidden_dim] */
    VELOX_MLA_Q_A_NORM = 7,  /* [q_lora_rank] */
    VELOX_MLA_KV_A_NORM = 8  /* [kv_lora_rank] */
};

typedef struct VeloxHipMlaBuffers {
    float* hidden;           /* [max_batch][hidden_dim] fp32: input and output of a layer step */
    uint16_t* latent_cache;  /* bf16 [num_layers][max_batch][s_cap][kv_lora_rank + rope] */
    VeloxDecodeState* states;/* [max_batch]: step = the sequence's position */
    uint32_t s_cap, splits;
    uint64_t weight_bytes, cache_bytes, act_bytes;
} VeloxHipMlaBuffers;

/* "deepseek_v3_mla": hidden 7168, 128 heads, q LoRA 1536, kv LoRA 512, nope 128 + rope 64, v 128. */
int velox_hip_mla_builtin_config(const char* which, uint32_t max_seq_len, uint32_t max_batch,
                                 VeloxHipMlaConfig* out);
/* plan: the static memory plan only (no device memory; ENOMEM past the budget, E002); create: plan
 * plus one hipMalloc holding every region, initialized. destroy forgets its arenas too. */
int velox_hip_mla_plan(const VeloxHipMlaConfig* cfg, VeloxHipMla** out);
int velox_hip_mla_create(const VeloxHipMlaConfig* cfg, VeloxHipMla** out);
void velox_hip_mla_destroy(VeloxHipMla* m);
int velox_hip_mla_buffers(const VeloxHipMla* m, VeloxHipMlaBuffers* out);
/* fp8 matrix of `kind` for `layer`: codes [rows][cols], scales [ceil(rows/128)][ceil(cols/128)]. */
int velox_hip_mla_load_fp8(VeloxHipMla* m, int kind, uint32_t layer, const uint8_t* codes, const float* scales,
                           hipStream_t stream);
int velox_hip_mla_load_f32(VeloxHipMla* m, int kind, uint32_t layer, const float* data, uint64_t count,
                           hipStream_t stream);
/* Every weight seeded N(0, sigma) and quantized on the device (the oracle's vxo_fp8_synth_matrix);
 * gains 1 (norm_sigma 0) or N(1, norm_sigma). */
int velox_hip_mla_synthesize(VeloxHipMla* m, uint64_t seed, float sigma, float norm_sigma, hipStream_t stream);
/* Latent rows [0, n_pos) of sequence `seq` in `layer` := bf16 of seeded N(0, sigma). */
int velox_hip_mla_fill_cache(VeloxHipMla* m, uint32_t layer, uint32_t seq, uint32_t n_pos, uint64_t seed,
                             float sigma, hipStream_t stream);
int velox_hip_mla_set_position(VeloxHipMla* m, uint32_t seq, uint64_t pos, hipStream_t stream);
/* hidden[b] += MLA(hidden[b]) for b < batch at each sequence's position; appends the latent row.
 * Capturable; errors through velox_hip_last_error(). */
void velox_hip_mla_layer_step(VeloxHipMla* m, uint32_t layer, uint32_t batch, uint64_t active_mask,
                              hipStream_t stream);
/* The attention stack of a decode step: the layer step of layers 0 .. num_layers - 1 in order, as the
 * reference's graph step launches its MLA kernel per layer (src/codegen.rs:2980-3003), with each
 * layer's W_o partials folded into the next layer's RMSNorm instead of a residual launch (hidden
 * ends equal to num_layers successive layer steps, bit for bit). The MoE FFN the reference model
 * places between the attention layers is outside this backend (not in the benchmark configurations).
 * Capturable; errors through velox_hip_last_error(). */
void velox_hip_mla_decode_step(VeloxHipMla* m, uint32_t batch, uint64_t active_mask, hipStream_t stream);
/* Algorithmic HBM bytes of one layer step (weights + scales + latent rows 0..pos + activations). */
double velox_hip_mla_step_bytes(const VeloxHipMla* m, uint32_t batch, uint64_t pos);

/* ---- the MLA model on the emitted-runner arena (src/codegen.rs:2980-3003: the MLA kernel reads its
 * weights from weight_arena and its latent cache from kv_cache_pool) ----
 * The regions of a plan as the eight VeloxHipArena fields: weight_arena = fp8 codes (tiled),
 * weight_scales = fp32 block scales, norm_weight_arena = fp32 gains then the RoPE table,
 * kv_cache_pool = the bf16 latent cache [layer][sequence][s_cap][kv_lora_rank + rope],
 * activation_arena = the sequences' VeloxDecodeState, then activations; host_pinned_ring NULL (the
 * attention stack emits no token), quant_mode VELOX_QUANT_FP8_E4M3, tied_lm_head 0.
 * arena_bytes: the region sizes of a plan (for caller-owned buffers, as the reference runner
 *   cudaMallocs its own, velox_cuda_runner.cu:417-431).
 * arena: fills the fields over a created handle's buffers and records the arena.
 * arena_bind: a planned handle (velox_hip_mla_plan) takes the caller's buffers from the fields
 *   (each at least its arena_bytes size, quant_mode VELOX_QUANT_FP8_E4M3), initializes them as
 *   create does and records the arena; EINVAL for a handle with buffers or a recorded weight_arena.
 * arena_mla: the handle an arena was recorded with (NULL if none).
 * arena_check: 0 when the arena's plan has `want`'s per-layer dimensions, norm, eps, theta and
 *   softmax scale (depth, context and batch are the plan's own), else EINVAL.
 * graph_step: velox_hip_mla_decode_step over all max_batch sequences, then every active sequence's
 *   position advances by one (capturable; one graph replays every step). decode: sets sequence 0's
 *   state to (step, token_in) first. Errors through velox_hip_last_error(). */
int velox_hip_mla_arena_bytes(const VeloxHipMla* m, uint64_t* weight_bytes, uint64_t* scale_bytes,
                              uint64_t* norm_bytes, uint64_t* kv_bytes, uint64_t* act_bytes);
int velox_hip_mla_arena(VeloxHipMla* m, VeloxHipArena* out);
int velox_hip_mla_arena_bind(VeloxHipMla* m, VeloxHipArena* a);
VeloxHipMla* velox_hip_mla_arena_mla(const VeloxHipArena* a);
int velox_hip_mla_arena_check(const VeloxHipArena* a, const VeloxHipMlaConfig* want);
void velox_hip_mla_graph_step(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_hip_mla_decode(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                          hipStream_t stream);
/* DeepSeek-V3's MLA model (examples/deepseek_v3_mla.vlx) under the reference's emitted names, for an
 * arena whose plan has DeepSeek-V3's dimensions (velox_hip_mla_arena_check against
 * velox_hip_mla_builtin_config("deepseek_v3_mla")); prefill is the same single-token step. */
void velox_DeepSeek_V3_MLA_decode_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_DeepSeek_V3_MLA_decode_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                                      hipStream_t stream);
void velox_DeepSeek_V3_MLA_prefill_graph_step_hip(VeloxHipArena* ctx, uint64_t active_mask, hipStream_t stream);
void velox_DeepSeek_V3_MLA_prefill_hip(VeloxHipArena* ctx, uint32_t token_in, size_t step, uint64_t active_mask,
                                       hipStream_t stream);

typedef struct VeloxHipMlaRunReport {
    double us_per_layer;     /* mean device time per layer (hipGraph replays of the step / layers) */
    double bytes_per_layer, hbm_gbps;
    double attn_us;          /* mean attention-kernel time (event-timed passes) */
    double attn_bytes;       /* its algorithmic bytes (latent rows read) */
    double wall_ms;
    int status;
} VeloxHipMlaRunReport;
/* Synthesize `which` with num_layers layers, seed a context_len-position latent context per
 * sequence and layer, time `steps` steps of `batch` sequences at position context_len after
 * `warmup` untimed ones: velox_hip_mla_decode_step over the stack (num_layers > 1; every layer's
 * weights then stream from HBM once per step) or one layer step (num_layers 0 or 1). */
int velox_hip_mla_run(const char* which, uint32_t batch, uint32_t context_len, uint32_t num_layers, uint32_t warmup,
                      uint32_t steps, uint64_t seed, VeloxHipMlaRunReport* rep);

#ifdef __cplusplus
}
#endif
#endif
