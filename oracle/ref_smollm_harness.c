/*
 * ref_smollm_harness.c -- drives the reference's emitted C99 SmolLM module (TEST INFRASTRUCTURE).
 *
 * Built only where /root/reference exists, by oracle/Makefile, into oracle/_ref/. It compiles
 * /root/reference/src/runners/tinystories_smollm.c in place (#include of the file where it lies;
 * nothing is copied) and lays the build's seeded synthetic fp32 weights out at that module's own
 * VELOX_W_OFFSET_* offsets, so that the reference's velox_SmolLM_135M_prefill (a complete
 * single-token forward step, tinystories_smollm.c:532) can be compared with the oracle's
 * restatement of src/runtime.rs. The emitted decode entry point (:602) skips the transformer
 * layers and is therefore not used.
 */
#include <stdlib.h>
#include <string.h>

#include "tinystories_smollm.c"
#include "velox_oracle.h"

static VeloxArenaContext g_ctx;
static uint8_t *g_w, *g_kv, *g_act;

static void fill(uint64_t off, uint64_t n, uint64_t seed, uint64_t tag, float sigma, float mean) {
    float* dst = (float*)(g_w + off);
    if (sigma == 0.0f) {
        for (uint64_t i = 0; i < n; ++i) dst[i] = mean;
    } else {
        vxo_fill_normal(dst, n, seed, tag, sigma, mean);
    }
}

/* Same tensor tags and element order as vxo_engine_create (velox_oracle.c). */
int vxr_smollm_init(uint64_t seed, float sigma, float norm_sigma) {
    const uint64_t H = VELOX_MODEL_HIDDEN_DIM, F = VELOX_MODEL_INTERMEDIATE_DIM;
    const uint64_t QD = VELOX_MODEL_NUM_HEADS * VELOX_MODEL_HEAD_DIM;
    const uint64_t KVD = VELOX_MODEL_NUM_KV_HEADS * VELOX_MODEL_HEAD_DIM;
    const uint64_t V = VELOX_MODEL_VOCAB_SIZE, L = VELOX_MODEL_NUM_LAYERS;
    g_w = (uint8_t*)calloc(1, VELOX_WEIGHT_ARENA_BYTES);
    g_kv = (uint8_t*)calloc(1, VELOX_KV_CACHE_POOL_BYTES);
    g_act = (uint8_t*)calloc(1, VELOX_ACTIVATION_ARENA_BYTES);
    if (!g_w || !g_kv || !g_act) return -1;
    fill(VELOX_W_OFFSET_W_EMBED, V * H, seed, vxo_tag(0, VXO_T_EMBED), sigma, 0.0f);
    memcpy(g_w + VELOX_W_OFFSET_W_HEAD, g_w + VELOX_W_OFFSET_W_EMBED, V * H * sizeof(float)); /* tied */
    fill(VELOX_W_OFFSET_W_FINAL_NORM, H, seed, vxo_tag(0, VXO_T_FINAL_NORM), norm_sigma, 1.0f);
    for (uint64_t l = 0; l < L; ++l) {
        const uint32_t li = (uint32_t)l;
        fill(VELOX_W_OFFSET_W_Q + l * QD * H * 4, QD * H, seed, vxo_tag(li, VXO_T_Q), sigma, 0.0f);
        fill(VELOX_W_OFFSET_W_K + l * KVD * H * 4, KVD * H, seed, vxo_tag(li, VXO_T_K), sigma, 0.0f);
        fill(VELOX_W_OFFSET_W_V + l * KVD * H * 4, KVD * H, seed, vxo_tag(li, VXO_T_V), sigma, 0.0f);
        fill(VELOX_W_OFFSET_W_OUT + l * H * QD * 4, H * QD, seed, vxo_tag(li, VXO_T_O), sigma, 0.0f);
        fill(VELOX_W_OFFSET_W_GATE + l * F * H * 4, F * H, seed, vxo_tag(li, VXO_T_GATE), sigma, 0.0f);
        fill(VELOX_W_OFFSET_W_UP + l * F * H * 4, F * H, seed, vxo_tag(li, VXO_T_UP), sigma, 0.0f);
        fill(VELOX_W_OFFSET_W_DOWN + l * H * F * 4, H * F, seed, vxo_tag(li, VXO_T_DOWN), sigma, 0.0f);
        fill(VELOX_W_OFFSET_W_ATTN_NORM + l * H * 4, H, seed, vxo_tag(li, VXO_T_ATTN_NORM), norm_sigma, 1.0f);
        fill(VELOX_W_OFFSET_W_MLP_NORM + l * H * 4, H, seed, vxo_tag(li, VXO_T_MLP_NORM), norm_sigma, 1.0f);
    }
    g_ctx.weight_arena = g_w;
    g_ctx.kv_cache_pool = g_kv;
    g_ctx.activation_arena = g_act;
    g_ctx.host_pinned_ring = NULL;
    return 0;
}

/* One full forward step at position pos through the reference module; copies the logits
 * (activation-arena offset 0 after the LM head, tinystories_smollm.c:598) to logits_out. */
uint32_t vxr_smollm_step(uint32_t token, uint64_t pos, float* logits_out) {
    const uint32_t tok = velox_SmolLM_135M_prefill(&g_ctx, token, (size_t)pos, 1ULL);
    if (logits_out) memcpy(logits_out, g_act, VELOX_MODEL_VOCAB_SIZE * sizeof(float));
    return tok;
}

void vxr_smollm_free(void) {
    free(g_w); free(g_kv); free(g_act);
    g_w = g_kv = g_act = NULL;
}
