// vx_kernels.hip -- hand-written gfx950 (CDNA4) kernels of the batch-1 decode step.
//
// Replaces the emitted CUDA kernels of src/codegen.rs:1104-2582 (warp-per-row GEMV with
// 32-bit loads, single-block RMSNorm, separate RoPE, sequential-over-t attention, 2-stage argmax)
// with an MI355X design:
//   * Q4_0 GEMV: wave64 tiles of R = 64/S rows x S lanes per row; every lane streams one
//     16-byte code word (one 32-weight block) per iteration with fully coalesced 1 KiB wave loads
//     of a layout repacked at load time; x lives in LDS as 22-bit integers per power-of-two-scaled
//     32-element block, stored as six planes of signed base-16 digits, and each code word meets
//     them in v_dot8_i32_i4 (q - 8 is the code nibble xor 8): the block's dot product is exact
//     integer arithmetic, so x keeps 2^-22 of each block's largest magnitude (fp32-class).
//     RMSNorm's gain is applied while staging x and its 1/rms in the epilogue, with residual /
//     SwiGLU / argmax.
//   * Decode attention: split-K over the sequence, RoPE + bf16 KV append in the prologue,
//     online softmax per split, LSE merge by the last workgroup of each KV head.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "vx_common.h"
#include "vx_gemv_q4.h"

namespace {

// Places one GGML Q4_0 block (scale bits d, 16 bytes qs: element j low nibble of qs[j],
// element j+16 high nibble) into the tiled layout at physical row `phys`, block b.
__device__ __forceinline__ void vx_store_tiled_block(const VxMat& m, uint32_t phys, uint32_t b, uint16_t d,
                                                     const uint8_t* qs) {
    uint32_t dw[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t v = 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int el = 8 * w + e;
            const uint32_t q = el < 16 ? (qs[el] & 15u) : (qs[el - 16] >> 4);
            v |= q << (8 * (e & 3) + 4 * (e >> 2));
        }
        dw[w] = v;
    }
    const size_t off = vx_tiled_off(m, phys, b);
    ((uint4*)m.codes)[off] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
    ((uint16_t*)m.scales)[off] = d;
}


// GGML quantize_row_q4_0_ref restated with contraction-free IEEE ops (bit-exact with the oracle).
// HIP's __fmul_rn/__fadd_rn are plain * and + here, so contraction is switched off explicitly:
// x * id + 8.5f fused into one FMA rounds differently at level boundaries.
__device__ __forceinline__ void vx_quantize_block(const float* x, uint16_t* d_out, uint8_t* qs) {
#pragma clang fp contract(off)
    float amax = 0.0f, vmax = 0.0f;
    for (int j = 0; j < 32; ++j) {
        const float v = x[j];
        if (amax < fabsf(v)) { amax = fabsf(v); vmax = v; }
    }
    const float d = vmax / -8.0f;
    const float id = (d != 0.0f) ? 1.0f / d : 0.0f;  // IEEE division (HIP's default is correctly rounded)
    *d_out = vx_f32_to_f16_bits(d);
    for (int j = 0; j < 16; ++j) {
        const float x0 = x[j] * id + 8.5f;
        const float x1 = x[16 + j] * id + 8.5f;
        int i0 = (int)x0, i1 = (int)x1;  // truncation, as the C (int8_t) conversion
        i0 = i0 < 15 ? i0 : 15;
        i1 = i1 < 15 ? i1 : 15;
        qs[j] = (uint8_t)(i0 | (i1 << 4));
    }
}

// Rotate-half RoPE of one pair (src/runtime.rs:761-764), unfused like the reference's Rust.
__device__ __forceinline__ float2 vx_rope_pair(float x1, float x2, float2 cs) {
#pragma clang fp contract(off)
    return make_float2(x1 * cs.x - x2 * cs.y, x2 * cs.x + x1 * cs.y);
}


}  // namespace

// Greedy token from the LM head's per-workgroup candidates (strict '>' scan semantics, lowest
// index on ties), then the ring write and device-state advance of src/codegen.rs:1627-1677.
__global__ __launch_bounds__(256) void vx_argmax_finalize_kernel(const float* cand_v, const uint32_t* cand_i,
                                                                 uint32_t n, VeloxDecodeState* state, uint32_t* ring,
                                                                 const uint32_t* prompt, const uint32_t* prompt_len,
                                                                 uint32_t* token_out, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    __shared__ float s_v[4];
    __shared__ uint32_t s_i[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t j = tid; j < n; j += 256) {
        const float v = cand_v[j];
        const uint32_t ii = cand_i[j];
        if (vx_better(v, ii, bv, bi)) { bv = v; bi = ii; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        if (vx_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w)
            if (vx_better(s_v[w], s_i[w], s_v[0], s_i[0])) { s_v[0] = s_v[w]; s_i[0] = s_i[w]; }
        // all-NaN or empty logits: token 0, as the reference's scan from -inf
        const uint32_t win = s_i[0] == 0xFFFFFFFFu ? 0u : s_i[0];
        if (token_out) *token_out = win;
        if (state) {
            const uint64_t step = state->step;
            if (ring) {
                __atomic_store_n(ring + (step & (VELOX_HIP_RING_SIZE - 1u)), win, __ATOMIC_RELAXED);
                __threadfence_system();
            }
            const uint32_t plen = prompt_len ? *prompt_len : 0u;
            const uint32_t next = (step + 1u < (uint64_t)plen) ? prompt[step + 1u] : win;
            state->token = next;
            state->step = step + 1u;
        }
    }
}

// =============================================================================================
// Split-K decode attention on MFMA
// =============================================================================================

// KV cache of one layer (and sequence), bf16: the K plane [hkv][s_cap][D] row-major, and the V
// plane [hkv][s_cap / 32][D][32]: per block of 32 positions, dimension-major, the 32 positions of
// one dimension in the slot order vx_vslot (vx_common.h) gives, so one 16-byte load gives a P.V
// lane its 8 values. s_cap is the position capacity rounded up to 32.

typedef __bf16 vx_bf8 __attribute__((ext_vector_type(8)));
typedef float vx_af4 __attribute__((ext_vector_type(4)));
typedef uint32_t vx_au4 __attribute__((ext_vector_type(4)));

// 8 fp32 values as the sum of NS bf16 vectors, each the truncation of what the previous ones leave
// (exact differences): NS = 3 represents every fp32 exactly, NS = 2 to 2^-16 relative.
template <int NS>
__device__ __forceinline__ void vx_split_bf16(const float (&x)[8], vx_bf8 (&out)[NS]) {
    float r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) r[e] = x[e];
#pragma unroll
    for (int t = 0; t < NS; ++t) {
        vx_au4 w;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const uint32_t a = __float_as_uint(r[2 * e]) & 0xFFFF0000u, b = __float_as_uint(r[2 * e + 1]) & 0xFFFF0000u;
            w[e] = (a >> 16) | b;
            r[2 * e] -= __uint_as_float(a);
            r[2 * e + 1] -= __uint_as_float(b);
        }
        out[t] = __builtin_bit_cast(vx_bf8, w);
    }
}

// Decode attention for one (split, kv head, sequence): RoPE of q and the new k
// (src/runtime.rs:745-768), bf16 KV append, then softmax(q K^T / sqrt(D)) V over the positions
// (src/runtime.rs:772-831). Split sp owns positions [sp * chunk, (sp + 1) * chunk) of the capacity
// (chunk a multiple of 32 fixed by s_max and the split count, so the first K/V loads need no
// state); its waves take the 32-position chunks below the current position in turn, on
// v_mfma_f32_16x16x32_bf16:
//   scores S^T[pos][head] = K Q^T: A = K rows straight from HBM (16 positions x 32 dimensions per
//     instruction, one 16-byte load per lane), B = the G q heads (rows past G zero) as three bf16
//     terms whose sum is the fp32 q, so every product and sum is fp32;
//   online softmax per head in the log2 domain (q pre-scaled by log2(e) / sqrt(D)); each lane
//     holds 8 positions of one head, the chunk maximum takes two lane exchanges;
//   O[head][dim] += P V: A = the probabilities where the scores left them (two bf16 terms), B =
//     the V block (one 16-byte load per lane and 16 dimensions).
// The current position is never read from the cache (the append may not have landed): the split
// that owns it adds q . k_new and v_new from the RoPE'd registers as one more softmax term when it
// merges its waves' (m, l, O) into the split's partial (o unnormalized). The o_proj GEMV or
// vx_attn_merge_kernel merges the partials; with one split and no consumer merge, the output is
// normalized here.
// head rows of the per-wave O in LDS: the used MFMA columns (G heads of each of R rows) rounded up
template <int D, int G, int R>
constexpr int vx_attn_hrows() { return G * R <= 4 ? 4 : G * R <= 8 ? 8 : 16; }

template <int D, int G, int W, int R>
constexpr size_t vx_attn_lds_bytes() {
    return (size_t)3 * 16 * (D + 8) * 2 + (size_t)2 * D * 2 + (size_t)W * 16 * 2 * 4 + 16 * 4 +
           (size_t)W * vx_attn_hrows<D, G, R>() * D * 4;
}

// R > 1 (prefill chunks only: the rows' K/V are in the cache, no append, no new position): the
// workgroup takes R consecutive rows of the chunk, the MFMA columns r G + h holding head h of row
// r, each column masked at its own row's position, so R rows share every K/V chunk load and the
// q operand's 16 columns are used 16 / G times as fully (Llama-3-8B at 128 rows: 4 rows of 4 heads).
template <int D, int G, int W, bool PS, int R = 1, bool RC = false>
__global__ __launch_bounds__(64 * W) void vx_attn_kernel(VxAttnArgs a) {
    static_assert(!RC || (R == 1 && !PS), "the copied RoPE row serves the single-sequence decode step");
    VX_TL_BEGIN(a, blockIdx.x + gridDim.x * (blockIdx.y + gridDim.y * blockIdx.z));
    // (the active-mask test follows the first barrier: a branch here would wait for the kernel
    // arguments once for the mask and again for everything else)
    const bool active = (a.active_mask & 1ULL) != 0ULL;
    constexpr int HALF = D / 2, NT = 64 * W, NC = D / 32, NB = D / 16, HR = vx_attn_hrows<D, G, R>();
    constexpr int GC = G * R;  // used MFMA columns
    static_assert(GC <= 16 && (R == 1 || PS), "R rows of G heads in 16 columns; several rows only in prefill");
    constexpr int QP = D + 8;  // padded q row: the 16 rows one operand read touches sit 4 banks apart
    constexpr float kLog2e = 1.4426950408889634f;
    static_assert(G >= 1 && G <= 8, "q heads of a group: MFMA columns 0..G-1, O rows 4 grp + i < 8");
    extern __shared__ __align__(16) unsigned char vx_smem[];
    uint16_t* qt_s = (uint16_t*)vx_smem;                   // [3][16][QP] bf16 terms of the pre-scaled q
    uint16_t* kn_s = qt_s + 3 * 16 * QP;                   // new position's k (RoPE'd), v
    uint16_t* vn_s = kn_s + D;
    float* ml_s = (float*)(vn_s + D);                      // [W][2][16]: per wave m, l of each head
    float* sn_s = ml_s + W * 32;                           // [16]: q_h . k_new of the new position
    float* o_s = sn_s + 16;                                // [W][HR][D]: per wave O
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;            // MFMA column (head / dimension), K group
    const uint32_t g = blockIdx.y, sp = blockIdx.x, bq = blockIdx.z * (uint32_t)R;  // bq: sequence / first row
    const uint32_t chunk = a.chunk;
    const uint32_t t0 = sp * chunk;
    uint16_t* kvb = a.kv + (size_t)bq * a.kv_bstride;
    uint16_t* Kc = kvb + (size_t)g * a.s_cap * D;
    uint16_t* Vc = kvb + ((size_t)a.hkv + g) * a.s_cap * D;

    // RoPE pairs (q heads and the new k; R > 1: the q heads of R rows), pairs per thread
    constexpr int NP = R == 1 ? (G + 1) * HALF : GC * HALF, RP = (NP + NT - 1) / NT;
    // ---- the decode position first, as a vector load, then the RoPE row it selects; vector loads
    // return in order, so both arrive ahead of the q/k/v and K/V chunk loads issued after them (a
    // scalar state load issued after those waited behind every workgroup's whole burst: ~4 us at 256
    // workgroups) ----
    const uint32_t nrow = a.batch ? a.batch : 1u;
    // row bq + r's position (rows past the chunk repeat its last row; safe_step clamp)
    auto row_pos = [&](uint32_t r) {
        uint64_t step = (uint64_t)a.fixed_pos;
        if (a.state)
            step = __hip_atomic_load((uint64_t*)&a.state[min(bq + r, nrow - 1u)].step, __ATOMIC_RELAXED,
                                     __HIP_MEMORY_SCOPE_AGENT);
        return step < (uint64_t)a.s_max ? (uint32_t)step : a.s_max - 1u;
    };
    auto uniform = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane(v); };
    // the row (of R) a RoPE pair belongs to
    auto pair_row = [&](int p) { return R == 1 ? 0 : p / (G * HALF); };
    float2 rcs[RP];
    uint32_t pos = 0, posmax = 0;
    uint64_t step0 = (uint64_t)a.fixed_pos;
    if constexpr (RC) {
        // the step's RoPE row was copied to rope_cur: nothing waits for the position until the masks
        // below, so its load goes first and the RoPE row, q/k/v and first K/V chunk loads follow at once
        step0 = __hip_atomic_load((uint64_t*)&a.state[0].step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
        for (int i = 0; i < RP; ++i) rcs[i] = a.rope_cur[min(tid + i * NT, NP - 1) % HALF];
    } else {
        pos = uniform(row_pos(0u));
        posmax = pos;
#pragma unroll
        for (int r = 1; r < R; ++r) posmax = max(posmax, uniform(row_pos((uint32_t)r)));
#pragma unroll
        for (int i = 0; i < RP; ++i) {
            const int p = min(tid + i * NT, NP - 1);
            rcs[i] = a.rope[(size_t)(R == 1 ? pos : row_pos((uint32_t)pair_row(p))) * HALF + p % HALF];
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // ---- q, the new k/v into registers (clamped: no load under a branch) ----
    float r1[RP], r2[RP], vnew;
    if constexpr (!PS) {
        const float* q = a.qkv + (size_t)bq * a.qkv_bstride;
        const float* k = q + (size_t)a.hq * D;
        const float* v = k + (size_t)a.hkv * D;
#pragma unroll
        for (int i = 0; i < RP; ++i) {
            const int p = min(tid + i * NT, NP - 1);
            const int hh = p / HALF, j = p % HALF;
            const float* src = hh < G ? q + (size_t)(g * G + hh) * D : k + (size_t)g * D;
            r1[i] = src[j];
            r2[i] = src[j + HALF];
        }
        vnew = v[(size_t)g * D + min(tid, D - 1)];
    } else {
        const uint32_t vcol = (a.hq + a.hkv + g) * (uint32_t)D + (uint32_t)min(tid, D - 1);
        // K-split partials of the batched QKV GEMM: every partial of an element loaded before the
        // adds, summed in split order, then the bias
        const uint32_t np = a.qkv_nparts;
        auto qkv_at = [&](uint32_t row, uint32_t c) {
            const float* base = a.qkv_part + (size_t)row * a.qkv_bstride;
            float t[8];
#pragma unroll
            for (uint32_t s = 0; s < 8; ++s) t[s] = base[min(s, np - 1u) * a.qkv_pstride + c];
            float acc = 0.0f;
#pragma unroll
            for (uint32_t s = 0; s < 8; ++s)
                if (s < np) acc += t[s];
            return a.qkv_bias ? acc + a.qkv_bias[c] : acc;
        };
#pragma unroll
        for (int i = 0; i < RP; ++i) {
            const int p = min(tid + i * NT, NP - 1);
            const int r = pair_row(p), hh = (p / HALF) % (R == 1 ? G + 1 : G), j = p % HALF;
            const uint32_t c0 = (hh < G ? (g * G + hh) : (a.hq + g)) * (uint32_t)D + (uint32_t)j;
            const uint32_t row = min(bq + (uint32_t)r, nrow - 1u);
            r1[i] = qkv_at(row, c0);
            r2[i] = qkv_at(row, c0 + HALF);
        }
        vnew = R == 1 ? qkv_at(bq, vcol) : 0.0f;
    }

    // ---- one 32-position chunk into registers: K rows cb + 16 b + col, dimensions 32 c + 8 grp;
    // V block cb / 32, dimensions 16 nb + col (clamped to the capacity; positions at or past the
    // current one are masked) ----
    vx_bf8 kf[2][NC], vf[NB];
    auto load_chunk = [&](uint32_t cb) {
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            const uint32_t row = min(cb + 16u * b + (uint32_t)col, a.s_cap - 1u);
#pragma unroll
            for (int c = 0; c < NC; ++c) kf[b][c] = *(const vx_bf8*)(Kc + (size_t)row * D + 32 * c + 8 * grp);
        }
        const uint16_t* vb = Vc + (size_t)(min(cb, a.s_cap - 32u) >> 5) * D * 32;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) vf[nb] = *(const vx_bf8*)(vb + (16 * nb + col) * 32 + 8 * grp);
    };
    uint32_t ci = (uint32_t)wave;
    load_chunk(t0 + 32u * min(ci, chunk / 32u - 1u));
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (RC) {  // the position: its load, issued first, has returned first
        pos = uniform(step0 < (uint64_t)a.s_max ? (uint32_t)step0 : a.s_max - 1u);
        posmax = pos;
    }
    // cached positions [t0, t1): below pos, or up to pos when a prefill chunk appended its rows
    const uint32_t t1 = min(a.prefill ? posmax + 1u : pos, t0 + chunk);
    const uint32_t n_chunks = t1 > t0 ? (t1 - t0 + 31u) >> 5 : 0u;
    const bool has_new = !a.prefill && t0 <= pos && pos < t0 + chunk;  // this split folds in the new position

    // ---- RoPE on this group's q heads and the new k; bf16 K/V row ----
    const float qscale = a.scale * kLog2e;  // scores in the log2 domain
    for (int i = tid; i < 3 * (16 - GC) * QP / 2; i += NT) {  // q rows GC..15 of every term: zero
        const int t = i / ((16 - GC) * QP / 2), r = i % ((16 - GC) * QP / 2);
        ((uint32_t*)(qt_s + (t * 16 + GC) * QP))[r] = 0u;
    }
#pragma unroll
    for (int i = 0; i < RP; ++i) {
        const int p = tid + i * NT;
        const float2 o = vx_rope_pair(r1[i], r2[i], rcs[i]);
        if (p < NP) {
            const int hh = p / HALF, j = p % HALF;  // q column r G + h (R == 1: head h, or G for k)
            if (hh < GC) {
                // the pre-scaled q as three bf16 terms (truncations of the exact remainders)
                float x0 = o.x * qscale, x1 = o.y * qscale;
#pragma unroll
                for (int t = 0; t < 3; ++t) {
                    const uint32_t b0 = __float_as_uint(x0) & 0xFFFF0000u, b1 = __float_as_uint(x1) & 0xFFFF0000u;
                    qt_s[(t * 16 + hh) * QP + j] = (uint16_t)(b0 >> 16);
                    qt_s[(t * 16 + hh) * QP + j + HALF] = (uint16_t)(b1 >> 16);
                    x0 -= __uint_as_float(b0);
                    x1 -= __uint_as_float(b1);
                }
            } else {
                kn_s[j] = vx_f32_to_bf16_bits(o.x);
                kn_s[j + HALF] = vx_f32_to_bf16_bits(o.y);
            }
        }
    }
    if (tid < D) vn_s[tid] = vx_f32_to_bf16_bits(vnew);
    __syncthreads();
    VX_TL_MARK(1);
    // the step's mask (uniform) after the barrier: loads are not moved across it, so the kernel
    // arguments come in one batch and every load above is issued before the test
    if (!active) return;
    if (sp == 0 && !a.prefill) {
        const uint16_t* vblk = Vc + (size_t)(pos >> 5) * D * 32 + vx_vslot(pos & 31u);
        for (int d = tid; d < D; d += NT) {
            Kc[(size_t)pos * D + d] = kn_s[d];
            ((uint16_t*)vblk)[d * 32] = vn_s[d];
        }
    }
    if (has_new && wave == W - 1) {
        // q_h . k_new for the new position (q = the sum of its three exact terms)
        for (int h = 0; h < G; ++h) {
            float sn = 0.0f;
#pragma unroll
            for (int d = lane; d < D; d += 64) {
                float qv = 0.0f;
#pragma unroll
                for (int t = 0; t < 3; ++t) qv += __uint_as_float((uint32_t)qt_s[(t * 16 + h) * QP + d] << 16);
                sn += qv * __uint_as_float((uint32_t)kn_s[d] << 16);
            }
            sn = vx_wave_sum(sn);
            if (lane == 0) sn_s[h] = sn;
        }
    }
    // q operand: head col (rows past G are zero), dimensions 32 c + 8 grp .. + 7, three bf16 terms
    vx_bf8 qop[NC][3];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int t = 0; t < 3; ++t) qop[c][t] = *(const vx_bf8*)(qt_s + (t * 16 + col) * QP + 32 * c + 8 * grp);

    float m_run = -INFINITY, l_run = 0.0f;  // head col: running max, this lane's share of the sum
    vx_af4 o_acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) o_acc[nb] = vx_af4{0.f, 0.f, 0.f, 0.f};

    // positions this lane's column attends below: its row's (R > 1; columns past GC none)
    uint32_t t1c = t1;
    if constexpr (R > 1) t1c = col < GC ? min(row_pos((uint32_t)(col / G)) + 1u, t0 + chunk) : 0u;
    for (; ci < n_chunks; ci += W) {
        const uint32_t cb = t0 + 32u * ci;
        // scores: sc[b][i] = S[position cb + 16 b + 4 grp + i][head col]
        vx_af4 sc[2];
#pragma unroll
        for (int b = 0; b < 2; ++b) {
            sc[b] = vx_af4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c)
#pragma unroll
                for (int t = 0; t < 3; ++t) sc[b] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[b][c], qop[c][t], sc[b], 0, 0, 0);
        }
        float pr[8];
        float mx = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t p = cb + 16u * b + 4u * grp + i;
                pr[4 * b + i] = p < t1c ? sc[b][i] : -INFINITY;
                mx = fmaxf(mx, pr[4 * b + i]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = m_run == -INFINITY ? 0.0f : vx_exp2(m_run - m_new);
        float lt = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            pr[e] = pr[e] == -INFINITY ? 0.0f : vx_exp2(pr[e] - m_new);
            lt += pr[e];
        }
        l_run = l_run * alpha + lt;
        m_run = m_new;
        // rescale O: o_acc[nb][i] belongs to head 4 grp + i, whose alpha lane (4 grp + i) holds
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float ai = __shfl(alpha, 4 * grp + i);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) o_acc[nb][i] *= ai;
        }
        vx_bf8 pop[2];
        vx_split_bf16<2>(pr, pop);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int t = 0; t < 2; ++t) o_acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop[t], vf[nb], o_acc[nb], 0, 0, 0);
        if (ci + W < n_chunks) load_chunk(t0 + 32u * (ci + W));
    }

    VX_TL_MARK(3);
    // ---- merge the waves (and the new position): per head the max m, weights 2^(m_w - m) ----
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (lane < 16) {
        ml_s[wave * 32 + lane] = m_run;
        ml_s[wave * 32 + 16 + lane] = l_run;
    }
    if (grp < HR / 4) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int i = 0; i < 4; ++i) o_s[(wave * HR + 4 * grp + i) * D + 16 * nb + col] = o_acc[nb][i];
    }
    __syncthreads();
    VX_TL_MARK(4);
    for (int idx = tid; idx < GC * D; idx += NT) {
        const int h = idx / D, d = idx % D;  // column: head h % G of row h / G
        const uint32_t row = bq + (uint32_t)(h / G);
        if (R > 1 && row >= nrow) continue;  // past the chunk's last row
        const float sn = has_new ? sn_s[h] : -INFINITY;
        float M = sn;
#pragma unroll
        for (int w = 0; w < W; ++w) M = fmaxf(M, ml_s[w * 32 + h]);
        float o = 0.0f, l = 0.0f;
        if (has_new) {
            const float wt = vx_exp2(sn - M);
            o = wt * __uint_as_float((uint32_t)vn_s[d] << 16);
            l = wt;
        }
#pragma unroll
        for (int w = 0; w < W; ++w) {
            const float mw = ml_s[w * 32 + h];
            const float wt = mw == -INFINITY ? 0.0f : vx_exp2(mw - M);
            o += wt * o_s[(w * HR + h) * D + d];
            l += wt * ml_s[w * 32 + 16 + h];
        }
        const size_t hq_idx = (size_t)row * a.hq + (size_t)g * G + (size_t)(h % G);  // (sequence or row, q head)
        if (a.splits == 1 && !a.partials_only) {
            a.out[hq_idx * D + d] = l > 0.0f ? o / l : 0.0f;
        } else if (a.splits == 1 && a.x16) {
            const float w = l > 0.0f ? 1.0f / l : 0.0f;
            const size_t e = (size_t)(g * G + (uint32_t)(h % G)) * D + d;
            a.x16[(size_t)row * a.x_ld + (e >> 5) * a.x_bs + (e & 31u)] = __half_as_ushort(__float2half(w * o));
        } else {
            a.part_o[(hq_idx * a.splits + sp) * D + d] = o;
            if (d == 0) {
                a.part_ml[(hq_idx * a.splits + sp) * 2] = M;
                a.part_ml[(hq_idx * a.splits + sp) * 2 + 1] = l;
            }
        }
    }
}

// LSE merge of the split partials (m, l in the log2 domain) of one q head per workgroup.
template <int D>
__global__ __launch_bounds__(D) void vx_attn_merge_kernel(VxAttnArgs a) {
    if ((a.active_mask & 1ULL) == 0ULL) return;
    __shared__ float s_w[64];
    const int tid = threadIdx.x;
    const size_t h = blockIdx.x;
    if (tid < 64) {
        const float mj = tid < (int)a.splits ? a.part_ml[(h * a.splits + tid) * 2] : -INFINITY;
        const float lj = tid < (int)a.splits ? a.part_ml[(h * a.splits + tid) * 2 + 1] : 0.0f;
        const float M = vx_wave_max(mj);
        const float wj = (mj == -INFINITY) ? 0.0f : vx_exp2(mj - M);
        const float L = vx_wave_sum(lj * wj);
        s_w[tid] = L > 0.0f ? wj / L : 0.0f;
    }
    __syncthreads();
    float acc = 0.0f;
#pragma unroll 8
    for (uint32_t j = 0; j < a.splits; ++j) acc += s_w[j] * a.part_o[(h * a.splits + j) * D + tid];
    a.out[h * D + tid] = acc;
}

// =============================================================================================
// Small kernels: embedding gather, decode state, loaders, parity helpers
// =============================================================================================
// rope_cur (single-sequence step): the RoPE row of the state's position, copied here for the step's
// attention kernels, which then issue every load before they wait for the position.
__global__ __launch_bounds__(kWG) void vx_embed_kernel(VxMat m, const VeloxDecodeState* state, uint32_t fixed_token,
                                                       float* h, uint64_t mask, const float2* rope, float2* rope_cur,
                                                       uint32_t half, uint32_t s_max) {
    if ((mask & 1ULL) == 0ULL) return;
    if (rope_cur && state && blockIdx.x == 0 && threadIdx.x < half) {
        const uint64_t step = state->step;
        const uint32_t pos = step < (uint64_t)s_max ? (uint32_t)step : s_max - 1u;  // the attention's clamp
        rope_cur[threadIdx.x] = rope[(size_t)pos * half + threadIdx.x];
    }
    const uint32_t token = state ? state->token : fixed_token;
    const uint32_t b = blockIdx.x * kWG + threadIdx.x, nb = m.k >> 5;
    if (b >= nb || token >= m.n) return;  // src/codegen.rs:2386-2390 guard
    if (m.fmt == VX_FMT_F32 || m.fmt == VX_FMT_F16) {  // unquantized rows (src/codegen.rs:1108-1117, fp16 twin)
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const size_t i = (size_t)token * m.k + b * 32u + (uint32_t)e;
            h[b * 32 + e] = m.fmt == VX_FMT_F32 ? ((const float*)m.codes)[i]
                                                : __half2float(__ushort_as_half(((const uint16_t*)m.codes)[i]));
        }
        return;
    }
    const uint32_t phys = vx_phys_row(m, token, 0);
    const size_t off = vx_tiled_off(m, phys, b);
    const uint4 c = m.codes[off];
    const uint32_t dw[4] = {c.x, c.y, c.z, c.w};
    if (m.fmt == VX_FMT_G64) {  // src/codegen.rs:2381-2410: fmaf(q, s, m) per weight
        const float sc = vx_h2f(m.scales[vx_tiled_off(m, phys, b & ~1u)]);
        const float mn = vx_h2f(m.scales[vx_tiled_off(m, phys, b | 1u)]);
#pragma unroll
        for (int e = 0; e < 32; ++e) h[b * 32 + e] = vx_tiled_weight<VX_FMT_G64>(dw, e, sc, mn);
        return;
    }
    const float d = vx_h2f(m.scales[off]);
#pragma unroll
    for (int e = 0; e < 32; ++e) h[b * 32 + e] = vx_tiled_weight<VX_FMT_Q4>(dw, e, d, 0.0f);
}

__global__ void vx_set_state_kernel(VeloxDecodeState* s, uint64_t step, uint32_t token) {
    s->step = step;
    s->token = token;
}

__global__ __launch_bounds__(kWG) void vx_repack_kernel(const uint8_t* src, uint32_t rows, uint32_t row0,
                                                        uint32_t pair_part, VxMat m) {
    const uint32_t nb = m.k >> 5;
    const size_t idx = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (idx >= (size_t)rows * nb) return;
    const uint32_t r = (uint32_t)(idx / nb), b = (uint32_t)(idx % nb);
    const uint8_t* blk = src + idx * 18u;
    uint8_t qs[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) qs[j] = blk[2 + j];
    const uint16_t d = (uint16_t)(blk[0] | (blk[1] << 8));
    vx_store_tiled_block(m, vx_phys_row(m, row0 + r, pair_part), b, d, qs);
}

__global__ __launch_bounds__(kWG) void vx_synth_q4_kernel(VxMat m, uint32_t rows, uint32_t row0, uint32_t pair_part,
                                                          uint64_t stream, float coef) {
    const uint32_t nb = m.k >> 5;
    const size_t idx = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (idx >= (size_t)rows * nb) return;
    const uint32_t r = (uint32_t)(idx / nb), b = (uint32_t)(idx % nb);
    float x[32];
    const uint64_t e0 = (uint64_t)r * m.k + (uint64_t)b * 32u;
#pragma unroll 4
    for (int j = 0; j < 32; ++j) x[j] = vx_normal_value(stream, e0 + j, coef, 0.0f);
    uint16_t d;
    uint8_t qs[16];
    vx_quantize_block(x, &d, qs);
    vx_store_tiled_block(m, vx_phys_row(m, row0 + r, pair_part), b, d, qs);
}

__global__ __launch_bounds__(kWG) void vx_fill_normal_kernel(float* out, uint64_t n, uint64_t stream, float coef,
                                                             float mean) {
    for (uint64_t i = (uint64_t)blockIdx.x * kWG + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kWG)
        out[i] = vx_normal_value(stream, i, coef, mean);
}

// The same values rounded to fp16 (to nearest even): the synthetic weights of an fp16-row model.
__global__ __launch_bounds__(kWG) void vx_fill_normal_f16_kernel(uint16_t* out, uint64_t n, uint64_t stream, float coef,
                                                                 float mean) {
    for (uint64_t i = (uint64_t)blockIdx.x * kWG + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kWG)
        out[i] = vx_f32_to_f16_bits(vx_normal_value(stream, i, coef, mean));
}

__global__ __launch_bounds__(kWG) void vx_fill_kv_kernel(uint16_t* base, uint32_t hkv, uint32_t s_cap, uint32_t d,
                                                         uint32_t n_pos, uint64_t stream_k, uint64_t stream_v,
                                                         float coef) {
    const uint64_t per_plane = (uint64_t)hkv * n_pos * d, n = 2 * per_plane;
    for (uint64_t i = (uint64_t)blockIdx.x * kWG + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kWG) {
        const uint32_t kv = (uint32_t)(i / per_plane);
        const uint64_t r = i % per_plane;
        const uint32_t g = (uint32_t)(r / ((uint64_t)n_pos * d));
        const uint32_t t = (uint32_t)((r / d) % n_pos), dd = (uint32_t)(r % d);
        const uint64_t ref_idx = ((uint64_t)t * hkv + g) * d + dd;
        const float v = vx_normal_value(kv ? stream_v : stream_k, ref_idx, coef, 0.0f);
        const uint64_t plane = ((uint64_t)kv * hkv + g) * s_cap * d;
        const uint64_t off = kv ? ((uint64_t)(t >> 5) * d + dd) * 32u + vx_vslot(t & 31u) : (uint64_t)t * d + dd;
        base[plane + off] = vx_f32_to_bf16_bits(v);
    }
}

__global__ __launch_bounds__(kWG) void vx_dequant_kernel(VxMat m, float* out) {
    const uint32_t nb = m.k >> 5;
    const uint32_t logical_rows = m.paired ? 2u * m.n : m.n;
    const size_t idx = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (idx >= (size_t)logical_rows * nb) return;
    const uint32_t lr = (uint32_t)(idx / nb), b = (uint32_t)(idx % nb);
    const uint32_t phys = m.paired ? vx_phys_row(m, lr % m.n, lr / m.n) : lr;
    const size_t off = vx_tiled_off(m, phys, b);
    const uint4 c = m.codes[off];
    const uint32_t dw[4] = {c.x, c.y, c.z, c.w};
    float* o = out + (size_t)lr * m.k + (size_t)b * 32u;
    if (m.fmt == VX_FMT_G64) {
        const float sc = vx_h2f(m.scales[vx_tiled_off(m, phys, b & ~1u)]);
        const float mn = vx_h2f(m.scales[vx_tiled_off(m, phys, b | 1u)]);
#pragma unroll
        for (int e = 0; e < 32; ++e) o[e] = vx_tiled_weight<VX_FMT_G64>(dw, e, sc, mn);
        return;
    }
    const float d = vx_h2f(m.scales[off]);
#pragma unroll
    for (int e = 0; e < 32; ++e) o[e] = vx_tiled_weight<VX_FMT_Q4>(dw, e, d, 0.0f);
}

__global__ __launch_bounds__(kWG) void vx_quantize_kernel(const float* x, uint32_t rows, uint32_t k, uint8_t* blocks) {
    const uint32_t nb = k >> 5;
    const size_t idx = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (idx >= (size_t)rows * nb) return;
    float v[32];
    for (int j = 0; j < 32; ++j) v[j] = x[idx * 32u + j];
    uint16_t d;
    uint8_t qs[16];
    vx_quantize_block(v, &d, qs);
    uint8_t* o = blocks + idx * 18u;
    o[0] = (uint8_t)(d & 0xFF);
    o[1] = (uint8_t)(d >> 8);
    for (int j = 0; j < 16; ++j) o[2 + j] = qs[j];
}

// Checkpoint elements as stored (fp32, fp16 or bf16: VX_DT_*) widened to fp32, or rounded to fp16
// (nearest even), for the loaders (the reference converts on the device at load as well,
// velox_cuda_f32_to_f16_kernel in src/runners/velox_cuda_runner.cu:174-197).
__global__ __launch_bounds__(kWG) void vx_convert_kernel(const void* src, uint32_t src_dt, void* dst, uint32_t dst_dt,
                                                         uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * kWG + threadIdx.x; i < n; i += (uint64_t)gridDim.x * kWG) {
        float v;
        if (src_dt == VX_DT_F32) v = ((const float*)src)[i];
        else if (src_dt == VX_DT_F16) v = vx_f16_bits_to_f32(((const uint16_t*)src)[i]);
        else v = vx_bf16_bits_to_f32(((const uint16_t*)src)[i]);
        if (dst_dt == VX_DT_F32) ((float*)dst)[i] = v;
        else ((uint16_t*)dst)[i] = vx_f32_to_f16_bits(v);
    }
}

__global__ __launch_bounds__(kWG) void vx_rmsnorm_kernel(const float* x, const float* w, uint32_t n, float eps, float* y) {
    __shared__ float red[4];
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += kWG) ss += x[i] * x[i];
    ss = vx_block_sum<4>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)n + eps);
    for (uint32_t i = threadIdx.x; i < n; i += kWG) y[i] = (x[i] * inv) * w[i];
}

__global__ __launch_bounds__(kWG) void vx_argmax_kernel(const float* x, uint32_t n, uint32_t* out) {
    __shared__ float s_v[4];
    __shared__ uint32_t s_i[4];
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t i = threadIdx.x; i < n; i += kWG)
        if (vx_better(x[i], i, bv, bi)) { bv = x[i]; bi = i; }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        if (vx_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
    __syncthreads();
    if (threadIdx.x == 0) {
        for (int w = 1; w < 4; ++w)
            if (vx_better(s_v[w], s_i[w], s_v[0], s_i[0])) { s_v[0] = s_v[w]; s_i[0] = s_i[w]; }
        *out = s_i[0] == 0xFFFFFFFFu ? 0u : s_i[0];
    }
}

// =============================================================================================
// Launch helpers
// =============================================================================================
namespace {

template <int D, int G, bool PS, int W, int R = 1, bool RC = false>
hipError_t vx_attn_launch_w(const VxAttnArgs& a, hipStream_t st) {
    constexpr size_t lds = vx_attn_lds_bytes<D, G, W, R>();
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)vx_attn_kernel<D, G, W, PS, R, RC>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        attr_set = true;
    }
    const uint32_t rows = a.batch ? a.batch : 1u;
    hipLaunchKernelGGL((vx_attn_kernel<D, G, W, PS, R, RC>), dim3(a.splits, a.hkv, (rows + R - 1u) / R), dim3(64 * W), lds,
                       st, a);
    return hipGetLastError();
}

template <int D, int G, bool PS>
hipError_t vx_attn_launch_ps(const VxAttnArgs& a, hipStream_t st) {
    if constexpr (PS) {
        // prefill chunks: 16 / G rows per workgroup (4-wave workgroups)
        constexpr int R = 16 / G;
        if constexpr (R > 1)
            if (a.prefill) return vx_attn_launch_w<D, G, PS, 4, R>(a, st);
        // 4 waves, two workgroups per CU, where 8-wave workgroups (one per CU) would need a second
        // round and 4 waves still take every 32-position chunk a split can attend in one pass (the
        // prefill chunks of short prompts: 64 rows x 8 KV heads = 512 workgroups, <= 128 positions)
        const uint32_t chunk = ((a.s_max + a.splits - 1u) / a.splits + 31u) & ~31u;
        const uint32_t span = a.max_len ? min(a.max_len, chunk) : chunk;
        const uint64_t wgs = (uint64_t)a.splits * a.hkv * (a.batch ? a.batch : 1u);
        if (wgs > 256u && span <= 4u * 32u) return vx_attn_launch_w<D, G, PS, 4>(a, st);
    }
    if constexpr (!PS)
        if (a.rope_cur && a.state && a.batch <= 1u && !a.prefill) return vx_attn_launch_w<D, G, PS, 8, 1, true>(a, st);
    return vx_attn_launch_w<D, G, PS, 8>(a, st);
}

template <int D, int G>
hipError_t vx_attn_launch_t(const VxAttnArgs& a, hipStream_t st) {
    if (a.qkv_nparts > 8 || (a.qkv_nparts && (!a.qkv_part || a.partials_only == 0))) return hipErrorInvalidValue;
    hipError_t e0 = a.qkv_nparts ? vx_attn_launch_ps<D, G, true>(a, st) : vx_attn_launch_ps<D, G, false>(a, st);
    if (e0 != hipSuccess) return e0;
    hipError_t e = hipGetLastError();
    if (e == hipSuccess && a.splits > 1 && !a.partials_only) {
        if (a.batch > 1) return hipErrorInvalidValue;  // batched steps merge with vx_bmerge_kernel
        hipLaunchKernelGGL((vx_attn_merge_kernel<D>), dim3(a.hq), dim3(D), 0, st, a);
        e = hipGetLastError();
    }
    return e;
}

}  // namespace

// Upper bound on GEMV workgroups (waves loop over the remaining tiles).
uint32_t vx_gemv_max_wgs_default() { return 512u; }

hipError_t vx_launch_gemv(const VxMat& m, const VxGemvArgs& a, int epi, uint32_t max_wgs, hipStream_t st) {
    switch (m.fmt) {
        case VX_FMT_Q4: return vx_launch_gemv_tiled<VX_FMT_Q4>(m, a, epi, max_wgs, st);
        case VX_FMT_G64: return vx_launch_gemv_g64(m, a, epi, max_wgs, st);
        case VX_FMT_F32:
        case VX_FMT_F16: return vx_launch_gemv_f(m, a, epi, vx_gemv_wgs(m.n_tiles, max_wgs), st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t vx_launch_argmax_finalize(const float* cand_v, const uint32_t* cand_i, uint32_t n, VeloxDecodeState* state,
                                     uint32_t* ring, const uint32_t* prompt, const uint32_t* prompt_len,
                                     uint32_t* token_out, uint64_t mask, hipStream_t st) {
    hipLaunchKernelGGL(vx_argmax_finalize_kernel, dim3(1), dim3(256), 0, st, cand_v, cand_i, n, state, ring, prompt,
                       prompt_len, token_out, mask);
    return hipGetLastError();
}

uint32_t vx_gemv_grid(uint32_t n_tiles, uint32_t max_wgs) { return vx_gemv_wgs(n_tiles, max_wgs); }

hipError_t vx_launch_attention(const VxAttnArgs& a, uint32_t d, hipStream_t st) {
    if (a.hkv == 0 || a.hq % a.hkv != 0 || a.splits == 0 || a.splits > 64 || a.s_max == 0 || (a.s_cap & 31u) ||
        a.s_cap < a.s_max)
        return hipErrorInvalidValue;
    VxAttnArgs b = a;
    b.chunk = ((a.s_max + a.splits - 1u) / a.splits + 31u) & ~31u;
    const uint32_t G = a.hq / a.hkv;
    if (d == 64) {
        switch (G) {
            case 1: return vx_attn_launch_t<64, 1>(b, st);
            case 2: return vx_attn_launch_t<64, 2>(b, st);
            case 3: return vx_attn_launch_t<64, 3>(b, st);
            case 4: return vx_attn_launch_t<64, 4>(b, st);
            case 8: return vx_attn_launch_t<64, 8>(b, st);
            default: return hipErrorInvalidValue;
        }
    }
    if (d == 128) {
        switch (G) {
            case 1: return vx_attn_launch_t<128, 1>(b, st);
            case 2: return vx_attn_launch_t<128, 2>(b, st);
            case 4: return vx_attn_launch_t<128, 4>(b, st);
            case 7: return vx_attn_launch_t<128, 7>(b, st);
            case 8: return vx_attn_launch_t<128, 8>(b, st);
            default: return hipErrorInvalidValue;
        }
    }
    return hipErrorInvalidValue;
}

hipError_t vx_launch_embed(const VxMat& m, const VeloxDecodeState* state, uint32_t fixed_token, float* h,
                           uint64_t mask, hipStream_t st, const float2* rope, float2* rope_cur, uint32_t half,
                           uint32_t s_max) {
    const uint32_t nb = m.k >> 5;
    if (rope_cur && (!rope || half == 0 || half > kWG || s_max == 0)) return hipErrorInvalidValue;
    hipLaunchKernelGGL(vx_embed_kernel, dim3((nb + kWG - 1) / kWG), dim3(kWG), 0, st, m, state, fixed_token, h, mask,
                       rope, rope_cur, half, s_max);
    return hipGetLastError();
}

hipError_t vx_launch_set_state(VeloxDecodeState* state, uint64_t step, uint32_t token, hipStream_t st) {
    hipLaunchKernelGGL(vx_set_state_kernel, dim3(1), dim3(1), 0, st, state, step, token);
    return hipGetLastError();
}

static inline dim3 vx_grid_for(size_t n) { return dim3((unsigned)((n + kWG - 1) / kWG)); }

hipError_t vx_launch_repack(const void* blocks, uint32_t rows, uint32_t row0, uint32_t pair_part, const VxMat& m,
                            hipStream_t st) {
    const size_t n = (size_t)rows * (m.k >> 5);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(vx_repack_kernel, vx_grid_for(n), dim3(kWG), 0, st, (const uint8_t*)blocks, rows, row0,
                       pair_part, m);
    return hipGetLastError();
}

hipError_t vx_launch_synth_q4(const VxMat& m, uint32_t rows, uint32_t row0, uint32_t pair_part, uint64_t stream,
                              float coef, hipStream_t st) {
    const size_t n = (size_t)rows * (m.k >> 5);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(vx_synth_q4_kernel, vx_grid_for(n), dim3(kWG), 0, st, m, rows, row0, pair_part, stream, coef);
    return hipGetLastError();
}

hipError_t vx_launch_fill_normal(float* out, uint64_t n, uint64_t stream, float coef, float mean, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const size_t g = (n + kWG - 1) / kWG;
    hipLaunchKernelGGL(vx_fill_normal_kernel, dim3((unsigned)(g < 65536 ? g : 65536)), dim3(kWG), 0, st, out, n,
                       stream, coef, mean);
    return hipGetLastError();
}

hipError_t vx_launch_fill_normal_f16(uint16_t* out, uint64_t n, uint64_t stream, float coef, float mean, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const size_t g = (n + kWG - 1) / kWG;
    hipLaunchKernelGGL(vx_fill_normal_f16_kernel, dim3((unsigned)(g < 65536 ? g : 65536)), dim3(kWG), 0, st, out, n,
                       stream, coef, mean);
    return hipGetLastError();
}

hipError_t vx_launch_fill_kv(uint16_t* layer_base, uint32_t hkv, uint32_t s_cap, uint32_t d, uint32_t n_pos,
                             uint64_t stream_k, uint64_t stream_v, float coef, hipStream_t st) {
    const uint64_t n = 2ULL * hkv * n_pos * d;
    if (n == 0) return hipSuccess;
    const size_t g = (n + kWG - 1) / kWG;
    hipLaunchKernelGGL(vx_fill_kv_kernel, dim3((unsigned)(g < 65536 ? g : 65536)), dim3(kWG), 0, st, layer_base, hkv,
                       s_cap, d, n_pos, stream_k, stream_v, coef);
    return hipGetLastError();
}

hipError_t vx_launch_dequant(const VxMat& m, float* out, hipStream_t st) {
    const size_t n = (size_t)(m.paired ? 2u * m.n : m.n) * (m.k >> 5);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(vx_dequant_kernel, vx_grid_for(n), dim3(kWG), 0, st, m, out);
    return hipGetLastError();
}

hipError_t vx_launch_quantize(const float* x, uint32_t rows, uint32_t k, void* blocks, hipStream_t st) {
    const size_t n = (size_t)rows * (k >> 5);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(vx_quantize_kernel, vx_grid_for(n), dim3(kWG), 0, st, x, rows, k, (uint8_t*)blocks);
    return hipGetLastError();
}

hipError_t vx_launch_convert(const void* src, uint32_t src_dt, void* dst, uint32_t dst_dt, uint64_t n, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const size_t g = (n + kWG - 1) / kWG;
    hipLaunchKernelGGL(vx_convert_kernel, dim3((unsigned)(g < 65536 ? g : 65536)), dim3(kWG), 0, st, src, src_dt, dst,
                       dst_dt, n);
    return hipGetLastError();
}

hipError_t vx_launch_rmsnorm(const float* x, const float* w, uint32_t n, float eps, float* y, hipStream_t st) {
    hipLaunchKernelGGL(vx_rmsnorm_kernel, dim3(1), dim3(kWG), 0, st, x, w, n, eps, y);
    return hipGetLastError();
}

hipError_t vx_launch_argmax(const float* x, uint32_t n, uint32_t* out, hipStream_t st) {
    hipLaunchKernelGGL(vx_argmax_kernel, dim3(1), dim3(kWG), 0, st, x, n, out);
    return hipGetLastError();
}
