/*
 * velox_oracle.c -- CPU restatement of Velox's decode path (TEST INFRASTRUCTURE ONLY).
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library,
 * and only as the checker or as the timed CPU baseline; the HIP product never calls it.
 *
 * Primary source: /root/reference/src/runtime.rs (the reference's CPU engine). Compile with
 * -ffp-contract=off: Rust never contracts a*b+c, so every fused multiply-add below is an
 * explicit fmaf() standing for an AVX2 _mm256_fmadd_ps of the reference.
 *
 * Pinning (see tests/test_oracle.py):
 *   - rmsnorm/matmul/rope/attention/swiglu/argmax/mla: the reference's own known answers
 *     (src/runtime.rs:1551-1613, tests/test_runtime_e2e.rs:38-201) plus bit-exact agreement
 *     with the reference's emitted C99 module compiled from /root/reference (oracle/_ref),
 *     captured in tests/golden/ for machines without the reference.
 *   - Q4_0: closed form d*(q-8) over all 16 nibbles, GGML round-trip bounds, fp16 rounding vs
 *     numpy.float16.  Parity of the GGML quantizer's tie-breaking is pinned by properties only.
 *   - group-64 codec: the reference test's nibble/scale constants
 *     (tests/empirical_challenge_phase2/test3_marlin_lop3_dequant.cu:109-206).
 */
#include "velox_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#if defined(_OPENMP)
#include <omp.h>
#endif

/* ------------------------------------------------------------------------------------------ */
/* RNG (not in the reference: the build's seeded synthetic-model recipe)                        */
/* ------------------------------------------------------------------------------------------ */
uint64_t vxo_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}

uint64_t vxo_stream(uint64_t seed, uint64_t tag) {
    return vxo_mix64(seed ^ vxo_mix64(tag + 0x632BE59BD9B4E019ULL));
}

static inline uint64_t vxo_hash(uint64_t stream, uint64_t idx) {
    return vxo_mix64(stream + (idx + 1ULL) * 0x9E3779B97F4A7C15ULL);
}

float vxo_normal(uint64_t stream, uint64_t idx, float coef) {
    const uint64_t a = vxo_hash(stream, 2ULL * idx);
    const uint64_t b = vxo_hash(stream, 2ULL * idx + 1ULL);
    int64_t s = 0;
    for (int i = 0; i < 4; ++i) s += (int64_t)((a >> (16 * i)) & 0xFFFFULL);
    for (int i = 0; i < 4; ++i) s += (int64_t)((b >> (16 * i)) & 0xFFFFULL);
    /* m = 2*sum(U) + 8 - 8*65536: an exact integer, |m| < 2^20 */
    const int32_t m = (int32_t)(2 * s - 524280);
    return (float)m * coef;
}

float vxo_normal_coef(float sigma) {
    return (float)((double)sigma / (131072.0 * sqrt(2.0 / 3.0)));
}

uint32_t vxo_uniform_u32(uint64_t stream, uint64_t idx, uint32_t n) {
    const uint64_t h = vxo_hash(stream, idx);
    return (uint32_t)(((h >> 32) * (uint64_t)n) >> 32);
}

void vxo_fill_normal(float* out, uint64_t n, uint64_t seed, uint64_t tag, float sigma, float mean) {
    const uint64_t st = vxo_stream(seed, tag);
    const float c = vxo_normal_coef(sigma);
    for (uint64_t i = 0; i < n; ++i) out[i] = mean + vxo_normal(st, i, c);
}

uint64_t vxo_tag(uint32_t layer, uint32_t kind) { return (uint64_t)layer * 256ULL + kind; }

/* ------------------------------------------------------------------------------------------ */
/* fp16 / bf16 conversions                                                                     */
/* ------------------------------------------------------------------------------------------ */
uint16_t vxo_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const uint32_t ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) {
        if (ax == 0x7F800000u) return (uint16_t)(sign | 0x7C00u);
        return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    }
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u); /* >= 65520 rounds to inf */
    if (ax < 0x38800000u) {                                 /* below 2^-14: subnormal or zero */
        if (ax < 0x33000000u) return (uint16_t)sign;        /* below 2^-25 */
        const uint32_t e = ax >> 23;
        const uint32_t mant = (ax & 0x7FFFFFu) | 0x800000u;
        const uint32_t sh = 126u - e;
        uint32_t q = mant >> sh;
        const uint32_t rem = mant & ((1u << sh) - 1u);
        const uint32_t half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    const uint32_t e = (ax >> 23) - 112u;
    const uint32_t mant = ax & 0x7FFFFFu;
    uint32_t h = (e << 10) | (mant >> 13);
    const uint32_t rem = mant & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}

float vxo_f16_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            uint32_t sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            m &= 0x3FFu;
            x = sign | ((113u - sh) << 23) | (m << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t vxo_f32_to_bf16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

float vxo_bf16_to_f32(uint16_t h) {
    const uint32_t x = (uint32_t)h << 16;
    float f;
    memcpy(&f, &x, 4);
    return f;
}

/* ------------------------------------------------------------------------------------------ */
/* GGML Q4_0 (third-party format, absent from the reference; ggml quantize_row_q4_0_ref /      */
/* dequantize_row_q4_0 as published in ggml-quants.c): 18-byte block {fp16 d; u8 qs[16]},      */
/* element j = (qs[j] & 15) - 8, element j+16 = (qs[j] >> 4) - 8, value = d * q.               */
/* ------------------------------------------------------------------------------------------ */
void vxo_q4_0_quantize_row(const float* x, uint64_t k, uint8_t* out) {
    const uint64_t nb = k / VXO_Q4_0_BLOCK;
    for (uint64_t b = 0; b < nb; ++b) {
        const float* xb = x + b * VXO_Q4_0_BLOCK;
        uint8_t* y = out + b * VXO_Q4_0_BYTES;
        float amax = 0.0f, vmax = 0.0f;
        for (int j = 0; j < 32; ++j) {
            const float v = xb[j];
            if (amax < fabsf(v)) { amax = fabsf(v); vmax = v; }
        }
        const float d = vmax / -8.0f;
        const float id = (d != 0.0f) ? 1.0f / d : 0.0f;
        const uint16_t dh = vxo_f32_to_f16(d);
        y[0] = (uint8_t)(dh & 0xFFu);
        y[1] = (uint8_t)(dh >> 8);
        for (int j = 0; j < 16; ++j) {
            const float x0 = xb[j] * id;
            const float x1 = xb[16 + j] * id;
            int8_t i0 = (int8_t)(x0 + 8.5f);
            int8_t i1 = (int8_t)(x1 + 8.5f);
            const uint8_t q0 = (uint8_t)(i0 < 15 ? i0 : 15);
            const uint8_t q1 = (uint8_t)(i1 < 15 ? i1 : 15);
            y[2 + j] = (uint8_t)(q0 | (q1 << 4));
        }
    }
}

void vxo_q4_0_dequant_row(const uint8_t* blocks, uint64_t k, float* out) {
    const uint64_t nb = k / VXO_Q4_0_BLOCK;
    for (uint64_t b = 0; b < nb; ++b) {
        const uint8_t* y = blocks + b * VXO_Q4_0_BYTES;
        const float d = vxo_f16_to_f32((uint16_t)(y[0] | (y[1] << 8)));
        for (int j = 0; j < 16; ++j) {
            const int q0 = (y[2 + j] & 0x0F) - 8;
            const int q1 = (y[2 + j] >> 4) - 8;
            out[b * 32 + j] = (float)q0 * d;
            out[b * 32 + 16 + j] = (float)q1 * d;
        }
    }
}

/* ------------------------------------------------------------------------------------------ */
/* Reference group-64 asymmetric codec: src/codegen.rs:2337-2370 (quantize),                  */
/* :2248-2265 / :2381-2410 (dequant w = fmaf(q, s, m)). scale_min[2g] = s, [2g+1] = m (fp16). */
/* ------------------------------------------------------------------------------------------ */
void vxo_g64_quantize(const float* src, uint64_t n_groups, uint32_t* packed, uint16_t* scale_min) {
    for (uint64_t g = 0; g < n_groups; ++g) {
        const float* grp = src + g * 64;
        float fmin = grp[0], fmax = grp[0];
        for (int i = 1; i < 64; ++i) {
            const float v = grp[i];
            if (v < fmin) fmin = v;
            if (v > fmax) fmax = v;
        }
        const float scale_f = (fmax > fmin) ? ((fmax - fmin) / 15.0f) : 0.0f;
        const uint16_t hs = vxo_f32_to_f16(scale_f);
        const uint16_t hm = vxo_f32_to_f16(fmin);
        scale_min[2 * g] = hs;
        scale_min[2 * g + 1] = hm;
        const float s_exact = vxo_f16_to_f32(hs);
        const float m_exact = vxo_f16_to_f32(hm);
        const float inv_s = (s_exact > 1.0e-12f) ? (1.0f / s_exact) : 0.0f;
        for (int w = 0; w < 8; ++w) {
            uint32_t q[8];
            for (int j = 0; j < 8; ++j) {
                long qi = lrintf((grp[w * 8 + j] - m_exact) * inv_s);
                if (qi < 0) qi = 0;
                if (qi > 15) qi = 15;
                q[j] = (uint32_t)qi;
            }
            packed[g * 8 + w] = (q[0] << 0) | (q[2] << 4) | (q[4] << 8) | (q[6] << 12) |
                                (q[1] << 16) | (q[3] << 20) | (q[5] << 24) | (q[7] << 28);
        }
    }
}

void vxo_g64_dequant(const uint32_t* packed, const uint16_t* scale_min, uint64_t n_groups, float* out) {
    for (uint64_t g = 0; g < n_groups; ++g) {
        const float s = vxo_f16_to_f32(scale_min[2 * g]);
        const float m = vxo_f16_to_f32(scale_min[2 * g + 1]);
        for (int w = 0; w < 8; ++w) {
            const uint32_t p = packed[g * 8 + w];
            /* nibble pairs (h2_0..h2_3) of velox_marlin_dot8_q4: bits 0/16, 4/20, 8/24, 12/28 */
            for (int pair = 0; pair < 4; ++pair) {
                const float lo = (float)((p >> (4 * pair)) & 0xFu);
                const float hi = (float)((p >> (16 + 4 * pair)) & 0xFu);
                out[g * 64 + w * 8 + 2 * pair] = fmaf(lo, s, m);
                out[g * 64 + w * 8 + 2 * pair + 1] = fmaf(hi, s, m);
            }
        }
    }
}

/* ------------------------------------------------------------------------------------------ */
/* fp32 primitives                                                                             */
/* ------------------------------------------------------------------------------------------ */

/* src/runtime.rs:588-601 */
void vxo_rmsnorm(float* dst, const float* x, const float* w, uint64_t dim, float eps) {
    float ss = 0.0f;
    for (uint64_t i = 0; i < dim; ++i) ss += x[i] * x[i];
    const float inv_rms = 1.0f / sqrtf((ss / (float)dim) + eps);
    for (uint64_t i = 0; i < dim; ++i) dst[i] = (x[i] * inv_rms) * w[i];
}

/* One row of src/runtime.rs:623-697 (AVX2 4-row inner): 8 lane accumulators fed by FMA over
 * k = 8c + lane, horizontal sum ((l0+l4)+(l1+l5)) + ((l2+l6)+(l3+l7)) as in hsum256_ps
 * (:605-616), then the scalar tail k >= 8*floor(in_dim/8) with separate multiply and add. */
static inline float vxo_row_dot(const float* x, const float* w, uint64_t in_dim) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    const uint64_t chunks = in_dim / 8;
    for (uint64_t c = 0; c < chunks; ++c) {
        const uint64_t k = c * 8;
        for (int l = 0; l < 8; ++l) acc[l] = fmaf(x[k + l], w[k + l], acc[l]);
    }
    float s = ((acc[0] + acc[4]) + (acc[1] + acc[5])) + ((acc[2] + acc[6]) + (acc[3] + acc[7]));
    for (uint64_t k = chunks * 8; k < in_dim; ++k) s += x[k] * w[k];
    return s;
}

/* src/runtime.rs:702-740 */
void vxo_matmul_transposed(float* dst, const float* x, const float* w, uint64_t in_dim, uint64_t out_dim) {
    for (uint64_t o = 0; o < out_dim; ++o) dst[o] = vxo_row_dot(x, w + o * in_dim, in_dim);
}

/* matmul_transposed_f32 over Q4_0 rows dequantized on the fly (exact in fp32); OpenMP over
 * rows leaves each row's arithmetic unchanged. */
void vxo_matmul_q4_0(float* dst, const float* x, const uint8_t* w_blocks, uint64_t in_dim,
                     uint64_t out_dim, int threads) {
    const uint64_t row_bytes = (in_dim / 32) * VXO_Q4_0_BYTES;
#if defined(_OPENMP)
    if (threads > 1) {
#pragma omp parallel num_threads(threads)
        {
            float* row = (float*)malloc(in_dim * sizeof(float));
#pragma omp for schedule(static)
            for (long o = 0; o < (long)out_dim; ++o) {
                vxo_q4_0_dequant_row(w_blocks + (uint64_t)o * row_bytes, in_dim, row);
                dst[o] = vxo_row_dot(x, row, in_dim);
            }
            free(row);
        }
        return;
    }
#else
    (void)threads;
#endif
    float* row = (float*)malloc(in_dim * sizeof(float));
    for (uint64_t o = 0; o < out_dim; ++o) {
        vxo_q4_0_dequant_row(w_blocks + o * row_bytes, in_dim, row);
        dst[o] = vxo_row_dot(x, row, in_dim);
    }
    free(row);
}

/* src/runtime.rs:745-768 */
void vxo_rope_rotate_half(float* t, uint64_t num_heads, uint64_t head_dim, uint64_t pos, float theta) {
    const uint64_t half = head_dim / 2;
    const float pos_f = (float)pos;
    for (uint64_t h = 0; h < num_heads; ++h) {
        float* hs = t + h * head_dim;
        for (uint64_t j = 0; j < half; ++j) {
            const float freq = 1.0f / powf(theta, (float)(2 * j) / (float)head_dim);
            const float angle = pos_f * freq;
            const float sin_a = sinf(angle);
            const float cos_a = cosf(angle);
            const float x1 = hs[j];
            const float x2 = hs[j + half];
            hs[j] = x1 * cos_a - x2 * sin_a;
            hs[j + half] = x2 * cos_a + x1 * sin_a;
        }
    }
}

/* src/runtime.rs:772-831 (two-pass softmax), with the -inf guards of the emitted C99 kernel
 * (src/codegen.rs:366,370), which change nothing for finite scores. */
void vxo_gqa_attention_step(float* out, float* scores, const float* q, const float* k_layer,
                            const float* v_layer, uint64_t n_q, uint64_t n_kv, uint64_t head_dim,
                            uint64_t pos) {
    const uint64_t group = n_q / n_kv;
    const uint64_t kv_stride = n_kv * head_dim;
    const float scale = 1.0f / sqrtf((float)head_dim);
    const uint64_t seq_len = pos + 1;
    for (uint64_t h = 0; h < n_q; ++h) {
        const uint64_t kv_h = h / group;
        const float* qh = q + h * head_dim;
        float max_score = -INFINITY;
        for (uint64_t t = 0; t < seq_len; ++t) {
            const float* kh = k_layer + t * kv_stride + kv_h * head_dim;
            float dot = 0.0f;
            for (uint64_t d = 0; d < head_dim; ++d) dot += qh[d] * kh[d];
            const float s = dot * scale;
            scores[t] = s;
            if (s > max_score) max_score = s;
        }
        float sum_exp = 0.0f;
        for (uint64_t t = 0; t < seq_len; ++t) {
            const float e = (max_score == -INFINITY) ? 0.0f : expf(scores[t] - max_score);
            scores[t] = e;
            sum_exp += e;
        }
        const float inv_sum = (sum_exp > 0.0f) ? (1.0f / sum_exp) : 0.0f;
        for (uint64_t t = 0; t < seq_len; ++t) scores[t] *= inv_sum;
        float* oh = out + h * head_dim;
        for (uint64_t d = 0; d < head_dim; ++d) oh[d] = 0.0f;
        for (uint64_t t = 0; t < seq_len; ++t) {
            const float p = scores[t];
            const float* vh = v_layer + t * kv_stride + kv_h * head_dim;
            for (uint64_t d = 0; d < head_dim; ++d) oh[d] += p * vh[d];
        }
    }
}

/* src/runtime.rs:1061-1067: gate <- silu(gate) * up */
void vxo_swiglu_act(float* gate, const float* up, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) {
        const float g = gate[i];
        const float silu = g / (1.0f + expf(-g));
        gate[i] = silu * up[i];
    }
}

/* src/runtime.rs:1078-1088: strict '>' from -inf, so ties resolve to the lowest index. */
uint32_t vxo_argmax(const float* logits, uint64_t n) {
    uint32_t best = 0;
    float bv = -INFINITY;
    for (uint64_t i = 0; i < n; ++i) {
        if (logits[i] > bv) { bv = logits[i]; best = (uint32_t)i; }
    }
    return best;
}

/* src/runtime.rs:944-1044 (single-layer slices; online softmax over latents, K = V = latent). */
void vxo_mla_absorbed_step(float* dst_hidden, const float* input_hidden, const float* w_norm,
                           const float* w_dkv, const float* w_abs_q, const float* w_abs_o,
                           float* kv_latent_pool, uint64_t hidden_dim, uint64_t latent_dim,
                           uint64_t max_seq_len, uint64_t step, float eps) {
    float* norm_x = (float*)malloc(hidden_dim * sizeof(float));
    float* q_abs = (float*)malloc(latent_dim * sizeof(float));
    float* ctx = (float*)malloc(latent_dim * sizeof(float));
    float* o_proj = (float*)malloc(hidden_dim * sizeof(float));
    vxo_rmsnorm(norm_x, input_hidden, w_norm, hidden_dim, eps);
    const uint64_t safe_step = step < max_seq_len ? step : (max_seq_len ? max_seq_len - 1 : 0);
    float* slot = kv_latent_pool + safe_step * latent_dim;
    vxo_matmul_transposed(slot, norm_x, w_dkv, hidden_dim, latent_dim);
    vxo_matmul_transposed(q_abs, norm_x, w_abs_q, hidden_dim, latent_dim);
    const float scale = latent_dim >= 128 ? 1.0f / sqrtf(128.0f) : 1.0f / sqrtf((float)latent_dim);
    float m = -INFINITY, l = 0.0f;
    for (uint64_t d = 0; d < latent_dim; ++d) ctx[d] = 0.0f;
    for (uint64_t t = 0; t <= safe_step; ++t) {
        const float* kv = kv_latent_pool + t * latent_dim;
        float dot = 0.0f;
        for (uint64_t d = 0; d < latent_dim; ++d) dot += q_abs[d] * kv[d];
        const float s = dot * scale;
        const float nm = s > m ? s : m;
        const float alpha = (m == -INFINITY) ? 0.0f : expf(m - nm);
        const float beta = expf(s - nm);
        l = l * alpha + beta;
        m = nm;
        for (uint64_t d = 0; d < latent_dim; ++d) ctx[d] = ctx[d] * alpha + beta * kv[d];
    }
    if (l > 0.0f) {
        const float inv_l = 1.0f / l;
        for (uint64_t d = 0; d < latent_dim; ++d) ctx[d] *= inv_l;
    }
    vxo_matmul_transposed(o_proj, ctx, w_abs_o, latent_dim, hidden_dim);
    for (uint64_t i = 0; i < hidden_dim; ++i) dst_hidden[i] = input_hidden[i] + o_proj[i];
    free(norm_x); free(q_abs); free(ctx); free(o_proj);
}

/* ------------------------------------------------------------------------------------------ */
/* fp8 e4m3fn (OCP) with 128x128 block scales: benchmark configuration 4's weight format (DeepSeek-V3),  */
/* not in the reference. Integer round-to-nearest-even so the device quantizer matches bit for  */
/* bit.                                                                                         */
/* ------------------------------------------------------------------------------------------ */
static inline uint32_t vxo_fbits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }

uint8_t vxo_f32_to_e4m3(float f) {
    const uint32_t u = vxo_fbits(f);
    const uint8_t sign = (uint8_t)((u >> 24) & 0x80u);
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7Fu;  /* NaN */
    if (a >= 0x43E00000u) return sign | 0x7Eu; /* |f| >= 448: saturate */
    const int e = (int)(a >> 23) - 127;
    if (e < -6) {
        /* subnormal range: q = rne(|f| * 2^9), q <= 8 (8 is the smallest normal, code 0x08) */
        if (a < 0x00800000u) return sign;      /* fp32 subnormals round to 0 */
        const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
        const int shift = 14 - e;              /* |f| * 2^9 = mant * 2^(e - 14) */
        if (shift > 25) return sign;
        uint32_t q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return sign | (uint8_t)q;
    }
    uint32_t m = (a & 0x7FFFFFu) >> 20, ex = (uint32_t)(e + 7);
    const uint32_t rem = a & 0xFFFFFu, half = 0x80000u;
    if (rem > half || (rem == half && (m & 1u))) ++m;
    if (m == 8u) { m = 0u; ++ex; }
    if (ex > 15u || (ex == 15u && m == 7u)) return sign | 0x7Eu;
    return sign | (uint8_t)((ex << 3) | m);
}

float vxo_e4m3_to_f32(uint8_t b) {
    const uint32_t e = (b >> 3) & 15u, m = b & 7u;
    if (e == 15u && m == 7u) return NAN;
    const float v = e ? ldexpf(1.0f + (float)m / 8.0f, (int)e - 7) : ldexpf((float)m / 8.0f, -6);
    return (b & 0x80u) ? -v : v;
}

void vxo_fp8_quantize(const float* w, uint64_t rows, uint64_t cols, uint8_t* codes, float* scales) {
    const uint64_t rb = (rows + 127) / 128, cb = (cols + 127) / 128;
    for (uint64_t i = 0; i < rb; ++i)
        for (uint64_t j = 0; j < cb; ++j) {
            float amax = 0.0f;
            for (uint64_t r = i * 128; r < rows && r < i * 128 + 128; ++r)
                for (uint64_t c = j * 128; c < cols && c < j * 128 + 128; ++c) {
                    const float v = fabsf(w[r * cols + c]);
                    if (v > amax) amax = v;
                }
            const float s = amax > 0.0f ? amax / 448.0f : 1.0f;
            scales[i * cb + j] = s;
            for (uint64_t r = i * 128; r < rows && r < i * 128 + 128; ++r)
                for (uint64_t c = j * 128; c < cols && c < j * 128 + 128; ++c)
                    codes[r * cols + c] = vxo_f32_to_e4m3(w[r * cols + c] / s);
        }
}

void vxo_fp8_dequant(const uint8_t* codes, const float* scales, uint64_t rows, uint64_t cols, float* out) {
    const uint64_t cb = (cols + 127) / 128;
    for (uint64_t r = 0; r < rows; ++r)
        for (uint64_t c = 0; c < cols; ++c)
            out[r * cols + c] = vxo_e4m3_to_f32(codes[r * cols + c]) * scales[(r / 128) * cb + c / 128];
}

void vxo_fp8_synth_matrix(uint64_t seed, uint64_t tag, uint64_t rows, uint64_t cols, float sigma, uint8_t* codes,
                          float* scales, float* dequant) {
    const uint64_t st = vxo_stream(seed, tag);
    const float coef = vxo_normal_coef(sigma);
    float* w = (float*)malloc(rows * cols * sizeof(float));
    for (uint64_t i = 0; i < rows * cols; ++i) w[i] = vxo_normal(st, i, coef);
    const uint64_t ns = ((rows + 127) / 128) * ((cols + 127) / 128);
    uint8_t* cd = codes ? codes : (uint8_t*)malloc(rows * cols);
    float* sc = scales ? scales : (float*)malloc(ns * sizeof(float));
    vxo_fp8_quantize(w, rows, cols, cd, sc);
    if (dequant) vxo_fp8_dequant(cd, sc, rows, cols, dequant);
    if (!codes) free(cd);
    if (!scales) free(sc);
    free(w);
}

/* DeepSeek-V3 absorbed MLA decode step. The attention loop is the reference's online softmax
 * (src/runtime.rs:995-1028) per head; the projections use the reference's matmul
 * (src/runtime.rs:702-740); RoPE is the reference's rotate-half (src/runtime.rs:745-768) over the
 * d_rope dimensions. */
void vxo_mla_layer_step(const VxoMlaConfig* c, const VxoMlaWeights* w, float* cache, int cache_bf16,
                        const float* h, float* h_out, uint64_t pos) {
    const uint64_t H = c->hidden, nh = c->n_heads, dn = c->d_nope, dr = c->d_rope, dv = c->d_v;
    const uint64_t lr = c->kv_lora, R = lr + dr, dq = dn + dr, kvb_rows = dn + dv;
    float* x = (float*)malloc(H * sizeof(float));
    float* q = (float*)malloc(nh * dq * sizeof(float));
    float* ckr = (float*)malloc(R * sizeof(float));
    float* o = (float*)malloc(nh * dv * sizeof(float));
    float* out = (float*)malloc(H * sizeof(float));
    vxo_rmsnorm(x, h, w->norm, H, c->eps);
    if (c->q_lora) {
        float* ql = (float*)malloc(c->q_lora * sizeof(float));
        float* qn = (float*)malloc(c->q_lora * sizeof(float));
        vxo_matmul_transposed(ql, x, w->q_a, H, c->q_lora);
        vxo_rmsnorm(qn, ql, w->q_a_norm, c->q_lora, c->eps);
        vxo_matmul_transposed(q, qn, w->q_b, c->q_lora, nh * dq);
        free(ql); free(qn);
    } else {
        vxo_matmul_transposed(q, x, w->q_b, H, nh * dq);
    }
    vxo_matmul_transposed(ckr, x, w->kv_a, H, R);
    float* row = cache + pos * R;
    if (c->kv_norm) vxo_rmsnorm(row, ckr, w->kv_a_norm, lr, c->eps);
    else memcpy(row, ckr, lr * sizeof(float));
    if (dr) {
        memcpy(row + lr, ckr + lr, dr * sizeof(float));
        vxo_rope_rotate_half(row + lr, 1, dr, pos, c->rope_theta);
    }
    if (cache_bf16)
        for (uint64_t i = 0; i < R; ++i) row[i] = vxo_bf16_to_f32(vxo_f32_to_bf16(row[i]));
    /* heads are independent; each is computed in order by one thread */
#if defined(_OPENMP)
#pragma omp parallel
#endif
    {
    float* qabs = (float*)malloc(lr * sizeof(float));
    float* qr = (float*)malloc((dr ? dr : 1) * sizeof(float));
    float* ctx = (float*)malloc(lr * sizeof(float));
#if defined(_OPENMP)
#pragma omp for schedule(static)
#endif
    for (long hl = 0; hl < (long)nh; ++hl) {
        const uint64_t hh = (uint64_t)hl;
        const float* qn = q + hh * dq;
        const float* wk = w->kv_b + hh * kvb_rows * lr;  /* W_uk[hh]: dn rows of lr */
        const float* wv = wk + dn * lr;                  /* W_uv[hh]: dv rows of lr */
        for (uint64_t cc = 0; cc < lr; ++cc) {
            float acc = 0.0f;
            for (uint64_t i = 0; i < dn; ++i) acc += qn[i] * wk[i * lr + cc];
            qabs[cc] = acc;
        }
        if (dr) {
            memcpy(qr, qn + dn, dr * sizeof(float));
            vxo_rope_rotate_half(qr, 1, dr, pos, c->rope_theta);
        }
        float m = -INFINITY, l = 0.0f;
        for (uint64_t cc = 0; cc < lr; ++cc) ctx[cc] = 0.0f;
        for (uint64_t t = 0; t <= pos; ++t) {
            const float* kv = cache + t * R;
            float dot = 0.0f;
            for (uint64_t cc = 0; cc < lr; ++cc) dot += qabs[cc] * kv[cc];
            for (uint64_t j = 0; j < dr; ++j) dot += qr[j] * kv[lr + j];
            const float s = dot * c->scale;
            const float nm = s > m ? s : m;
            const float alpha = (m == -INFINITY) ? 0.0f : expf(m - nm);
            const float beta = expf(s - nm);
            l = l * alpha + beta;
            m = nm;
            for (uint64_t cc = 0; cc < lr; ++cc) ctx[cc] = ctx[cc] * alpha + beta * kv[cc];
        }
        if (l > 0.0f) {
            const float inv_l = 1.0f / l;
            for (uint64_t cc = 0; cc < lr; ++cc) ctx[cc] *= inv_l;
        }
        for (uint64_t j = 0; j < dv; ++j) {
            float acc = 0.0f;
            for (uint64_t cc = 0; cc < lr; ++cc) acc += wv[j * lr + cc] * ctx[cc];
            o[hh * dv + j] = acc;
        }
    }
    free(qabs); free(qr); free(ctx);
    }
    vxo_matmul_transposed(out, o, w->o, nh * dv, H);
    for (uint64_t i = 0; i < H; ++i) h_out[i] = h[i] + out[i];
    free(x); free(q); free(ckr); free(o); free(out);
}

/* ------------------------------------------------------------------------------------------ */
/* Engine: src/runtime.rs:1229-1451 (VeloxStaticExecutionEngine::forward_step) with the        */
/* Benchmark extensions (config-driven eps/theta, Q4_0 weights, bf16 KV rounding, QKV bias,     */
/* tied head).                                                                                 */
/* ------------------------------------------------------------------------------------------ */
typedef struct {
    void* data;
    uint64_t nbytes;
} VxoTensor;

struct VxoEngine {
    VxoConfig cfg;
    uint32_t built_layers;
    int threads;
    VxoTensor embed, final_norm, head;
    VxoTensor* layer; /* [built_layers][16] indexed by kind */
    float *k_cache, *v_cache;
    /* one-step K/V forcing (vxo_engine_force_kv): rows to attend with at the next forward's position,
     * and where the rows it computed itself go */
    const float *force_k, *force_v;
    float *seen_k, *seen_v;
    float *hidden, *norm_x, *q_buf, *attn_out, *o_buf, *gate, *up, *down, *scores;
};

static void vxo_make_matrix(VxoTensor* t, const VxoConfig* c, uint64_t seed, uint64_t tag, uint64_t rows,
                            uint64_t cols, float sigma, int threads) {
    const uint64_t st = vxo_stream(seed, tag);
    const float coef = vxo_normal_coef(sigma);
    if (c->q4_0) {
        const uint64_t row_bytes = (cols / 32) * VXO_Q4_0_BYTES;
        t->nbytes = rows * row_bytes;
        t->data = malloc(t->nbytes);
        uint8_t* dst = (uint8_t*)t->data;
#if defined(_OPENMP)
#pragma omp parallel num_threads(threads > 0 ? threads : 1)
#endif
        {
            float* buf = (float*)malloc(cols * sizeof(float));
#if defined(_OPENMP)
#pragma omp for schedule(static)
#endif
            for (long r = 0; r < (long)rows; ++r) {
                for (uint64_t k = 0; k < cols; ++k) buf[k] = vxo_normal(st, (uint64_t)r * cols + k, coef);
                vxo_q4_0_quantize_row(buf, cols, dst + (uint64_t)r * row_bytes);
            }
            free(buf);
        }
    } else {
        t->nbytes = rows * cols * sizeof(float);
        t->data = malloc(t->nbytes);
        float* dst = (float*)t->data;
#if defined(_OPENMP)
#pragma omp parallel for num_threads(threads > 0 ? threads : 1) schedule(static)
#endif
        for (long r = 0; r < (long)rows; ++r) {
            float* row = dst + (uint64_t)r * cols;
            for (uint64_t k = 0; k < cols; ++k) {
                const float v = vxo_normal(st, (uint64_t)r * cols + k, coef);
                /* fp16 weights (the reference's quant_mode 1): the value rounded to fp16, exact in fp32 */
                row[k] = c->w_f16 ? vxo_f16_to_f32(vxo_f32_to_f16(v)) : v;
            }
            if (c->w_g64) {
                /* group-64 weights (quant_mode 2): the values the reference's GEMV dequantizes,
                 * fmaf(q, s, m), from its load-time quantizer */
                uint32_t packed[8];
                uint16_t sm[2];
                for (uint64_t g = 0; g < cols / 64; ++g) {
                    vxo_g64_quantize(row + g * 64, 1, packed, sm);
                    vxo_g64_dequant(packed, sm, 1, row + g * 64);
                }
            }
        }
    }
    (void)threads;
}

static void vxo_make_vector(VxoTensor* t, uint64_t seed, uint64_t tag, uint64_t n, float sigma, float mean) {
    t->nbytes = n * sizeof(float);
    t->data = malloc(t->nbytes);
    if (sigma == 0.0f) {
        for (uint64_t i = 0; i < n; ++i) ((float*)t->data)[i] = mean;
    } else {
        vxo_fill_normal((float*)t->data, n, seed, tag, sigma, mean);
    }
}

VxoEngine* vxo_engine_create(const VxoConfig* cfg, uint64_t seed, float sigma, float norm_sigma,
                             uint32_t layers_to_build, int threads) {
    VxoEngine* e = (VxoEngine*)calloc(1, sizeof(VxoEngine));
    e->cfg = *cfg;
    e->threads = threads;
    const VxoConfig* c = &e->cfg;
    const uint64_t H = c->hidden_dim, F = c->intermediate_dim, D = c->head_dim;
    const uint64_t qd = (uint64_t)c->num_heads * D, kvd = (uint64_t)c->num_kv_heads * D;
    e->built_layers = layers_to_build < c->num_layers ? layers_to_build : c->num_layers;
    vxo_make_matrix(&e->embed, c, seed, vxo_tag(0, VXO_T_EMBED), c->vocab_size, H, sigma, threads);
    vxo_make_vector(&e->final_norm, seed, vxo_tag(0, VXO_T_FINAL_NORM), H, norm_sigma, 1.0f);
    if (!c->tied_lm_head) vxo_make_matrix(&e->head, c, seed, vxo_tag(0, VXO_T_HEAD), c->vocab_size, H, sigma, threads);
    e->layer = (VxoTensor*)calloc((size_t)e->built_layers * 16, sizeof(VxoTensor));
    for (uint32_t l = 0; l < e->built_layers; ++l) {
        VxoTensor* L = e->layer + (size_t)l * 16;
        vxo_make_vector(&L[VXO_T_ATTN_NORM], seed, vxo_tag(l, VXO_T_ATTN_NORM), H, norm_sigma, 1.0f);
        vxo_make_vector(&L[VXO_T_MLP_NORM], seed, vxo_tag(l, VXO_T_MLP_NORM), H, norm_sigma, 1.0f);
        vxo_make_matrix(&L[VXO_T_Q], c, seed, vxo_tag(l, VXO_T_Q), qd, H, sigma, threads);
        vxo_make_matrix(&L[VXO_T_K], c, seed, vxo_tag(l, VXO_T_K), kvd, H, sigma, threads);
        vxo_make_matrix(&L[VXO_T_V], c, seed, vxo_tag(l, VXO_T_V), kvd, H, sigma, threads);
        vxo_make_matrix(&L[VXO_T_O], c, seed, vxo_tag(l, VXO_T_O), H, qd, sigma, threads);
        vxo_make_matrix(&L[VXO_T_GATE], c, seed, vxo_tag(l, VXO_T_GATE), F, H, sigma, threads);
        vxo_make_matrix(&L[VXO_T_UP], c, seed, vxo_tag(l, VXO_T_UP), F, H, sigma, threads);
        vxo_make_matrix(&L[VXO_T_DOWN], c, seed, vxo_tag(l, VXO_T_DOWN), H, F, sigma, threads);
        if (c->qkv_bias) {
            vxo_make_vector(&L[VXO_T_BQ], seed, vxo_tag(l, VXO_T_BQ), qd, sigma, 0.0f);
            vxo_make_vector(&L[VXO_T_BK], seed, vxo_tag(l, VXO_T_BK), kvd, sigma, 0.0f);
            vxo_make_vector(&L[VXO_T_BV], seed, vxo_tag(l, VXO_T_BV), kvd, sigma, 0.0f);
        }
    }
    const uint64_t kv_elems = (uint64_t)e->built_layers * c->max_seq_len * kvd;
    e->k_cache = (float*)calloc(kv_elems ? kv_elems : 1, sizeof(float));
    e->v_cache = (float*)calloc(kv_elems ? kv_elems : 1, sizeof(float));
    const uint64_t big = (H > qd ? H : qd);
    e->hidden = (float*)calloc(H, sizeof(float));
    e->norm_x = (float*)calloc(big, sizeof(float));
    e->q_buf = (float*)calloc(qd, sizeof(float));
    e->attn_out = (float*)calloc(qd, sizeof(float));
    e->o_buf = (float*)calloc(H, sizeof(float));
    e->gate = (float*)calloc(F, sizeof(float));
    e->up = (float*)calloc(F, sizeof(float));
    e->down = (float*)calloc(H, sizeof(float));
    e->scores = (float*)calloc(c->max_seq_len, sizeof(float));
    return e;
}

void vxo_engine_destroy(VxoEngine* e) {
    if (!e) return;
    free(e->embed.data); free(e->final_norm.data); free(e->head.data);
    for (uint32_t i = 0; i < e->built_layers * 16; ++i) free(e->layer[i].data);
    free(e->layer);
    free(e->k_cache); free(e->v_cache);
    free(e->hidden); free(e->norm_x); free(e->q_buf); free(e->attn_out); free(e->o_buf);
    free(e->gate); free(e->up); free(e->down); free(e->scores);
    free(e);
}

void vxo_engine_reset(VxoEngine* e) {
    const uint64_t kvd = (uint64_t)e->cfg.num_kv_heads * e->cfg.head_dim;
    const uint64_t n = (uint64_t)e->built_layers * e->cfg.max_seq_len * kvd;
    memset(e->k_cache, 0, n * sizeof(float));
    memset(e->v_cache, 0, n * sizeof(float));
}

const void* vxo_engine_tensor(const VxoEngine* e, uint32_t kind, uint32_t layer, uint64_t* nbytes) {
    const VxoTensor* t = NULL;
    if (kind == VXO_T_EMBED) t = &e->embed;
    else if (kind == VXO_T_FINAL_NORM) t = &e->final_norm;
    else if (kind == VXO_T_HEAD) t = e->cfg.tied_lm_head ? &e->embed : &e->head;
    else if (layer < e->built_layers && kind < 16) t = &e->layer[(size_t)layer * 16 + kind];
    if (!t || !t->data) { if (nbytes) *nbytes = 0; return NULL; }
    if (nbytes) *nbytes = t->nbytes;
    return t->data;
}

const float* vxo_engine_hidden(const VxoEngine* e) { return e->hidden; }
void vxo_engine_set_threads(VxoEngine* e, int threads) { e->threads = threads > 0 ? threads : 1; }
float* vxo_engine_k_cache(VxoEngine* e) { return e->k_cache; }
float* vxo_engine_v_cache(VxoEngine* e) { return e->v_cache; }

void vxo_engine_force_kv(VxoEngine* e, const float* k_rows, const float* v_rows, float* seen_k, float* seen_v) {
    e->force_k = k_rows;
    e->force_v = v_rows;
    e->seen_k = seen_k;
    e->seen_v = seen_v;
}

static void vxo_linear(const VxoEngine* e, float* dst, const float* x, const VxoTensor* w, uint64_t in_dim,
                       uint64_t out_dim) {
    if (e->cfg.q4_0) vxo_matmul_q4_0(dst, x, (const uint8_t*)w->data, in_dim, out_dim, e->threads);
    else vxo_matmul_transposed(dst, x, (const float*)w->data, in_dim, out_dim);
}

uint32_t vxo_engine_forward_layers(VxoEngine* e, uint32_t token, uint64_t pos, uint32_t layers, float* logits) {
    const VxoConfig* c = &e->cfg;
    const uint64_t H = c->hidden_dim, F = c->intermediate_dim, D = c->head_dim;
    const uint64_t qd = (uint64_t)c->num_heads * D, kvd = (uint64_t)c->num_kv_heads * D;
    const uint64_t layer_kv = (uint64_t)c->max_seq_len * kvd;
    if (layers > e->built_layers) layers = e->built_layers;

    /* 1. embedding row (dequantized when Q4_0) */
    if (c->q4_0) {
        const uint64_t row_bytes = (H / 32) * VXO_Q4_0_BYTES;
        vxo_q4_0_dequant_row((const uint8_t*)e->embed.data + (uint64_t)token * row_bytes, H, e->hidden);
    } else {
        memcpy(e->hidden, (const float*)e->embed.data + (uint64_t)token * H, H * sizeof(float));
    }

    for (uint32_t l = 0; l < layers; ++l) {
        const VxoTensor* L = e->layer + (size_t)l * 16;
        vxo_rmsnorm(e->norm_x, e->hidden, (const float*)L[VXO_T_ATTN_NORM].data, H, c->rms_norm_eps);
        float* k_slot = e->k_cache + (uint64_t)l * layer_kv + pos * kvd;
        float* v_slot = e->v_cache + (uint64_t)l * layer_kv + pos * kvd;
        vxo_linear(e, e->q_buf, e->norm_x, &L[VXO_T_Q], H, qd);
        vxo_linear(e, k_slot, e->norm_x, &L[VXO_T_K], H, kvd);
        vxo_linear(e, v_slot, e->norm_x, &L[VXO_T_V], H, kvd);
        if (c->qkv_bias) {
            const float* bq = (const float*)L[VXO_T_BQ].data;
            const float* bk = (const float*)L[VXO_T_BK].data;
            const float* bv = (const float*)L[VXO_T_BV].data;
            for (uint64_t i = 0; i < qd; ++i) e->q_buf[i] += bq[i];
            for (uint64_t i = 0; i < kvd; ++i) { k_slot[i] += bk[i]; v_slot[i] += bv[i]; }
        }
        vxo_rope_rotate_half(e->q_buf, c->num_heads, D, pos, c->rope_theta);
        vxo_rope_rotate_half(k_slot, c->num_kv_heads, D, pos, c->rope_theta);
        if (c->kv_bf16) {
            for (uint64_t i = 0; i < kvd; ++i) {
                k_slot[i] = vxo_bf16_to_f32(vxo_f32_to_bf16(k_slot[i]));
                v_slot[i] = vxo_bf16_to_f32(vxo_f32_to_bf16(v_slot[i]));
            }
        }
        if (e->force_k) {
            memcpy(e->seen_k + (uint64_t)l * kvd, k_slot, kvd * sizeof(float));
            memcpy(e->seen_v + (uint64_t)l * kvd, v_slot, kvd * sizeof(float));
            memcpy(k_slot, e->force_k + (uint64_t)l * kvd, kvd * sizeof(float));
            memcpy(v_slot, e->force_v + (uint64_t)l * kvd, kvd * sizeof(float));
        }
        vxo_gqa_attention_step(e->attn_out, e->scores, e->q_buf, e->k_cache + (uint64_t)l * layer_kv,
                               e->v_cache + (uint64_t)l * layer_kv, c->num_heads, c->num_kv_heads, D, pos);
        vxo_linear(e, e->o_buf, e->attn_out, &L[VXO_T_O], qd, H);
        for (uint64_t i = 0; i < H; ++i) e->hidden[i] += e->o_buf[i];
        vxo_rmsnorm(e->norm_x, e->hidden, (const float*)L[VXO_T_MLP_NORM].data, H, c->rms_norm_eps);
        /* src/runtime.rs:1048-1073 */
        vxo_linear(e, e->gate, e->norm_x, &L[VXO_T_GATE], H, F);
        vxo_linear(e, e->up, e->norm_x, &L[VXO_T_UP], H, F);
        vxo_swiglu_act(e->gate, e->up, F);
        vxo_linear(e, e->down, e->gate, &L[VXO_T_DOWN], F, H);
        for (uint64_t i = 0; i < H; ++i) e->hidden[i] += e->down[i];
    }

    e->force_k = e->force_v = NULL;
    vxo_rmsnorm(e->norm_x, e->hidden, (const float*)e->final_norm.data, H, c->rms_norm_eps);
    const VxoTensor* head = c->tied_lm_head ? &e->embed : &e->head;
    vxo_linear(e, logits, e->norm_x, head, H, c->vocab_size);
    return vxo_argmax(logits, c->vocab_size);
}

uint32_t vxo_engine_forward(VxoEngine* e, uint32_t token, uint64_t pos, float* logits) {
    return vxo_engine_forward_layers(e, token, pos, e->cfg.num_layers, logits);
}
