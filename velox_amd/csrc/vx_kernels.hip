// vx_kernels.hip -- hand-written gfx950 (CDNA4) kernels of the batch-1 decode step.
//
// Replaces the emitted CUDA kernels of src/codegen.rs:1104-2582 (warp-per-row GEMV with
// 32-bit loads, single-block RMSNorm, separate RoPE, sequential-over-t attention, 2-stage argmax)
// with an MI355X design:
//   * Q4_0 GEMV: wave64 tiles of R = 64/S rows x S lanes per row; every lane streams one
//     16-byte code word (one 32-weight block) per iteration with fully coalesced 1 KiB wave loads
//     of a layout repacked at load time; x lives in LDS as fp16; nibbles are unpacked with the
//     0x6400 magic-exponent trick and consumed by v_dot2c_f32_f16 with fp32 accumulation; the
//     Q4_0 offset -8 is folded into one per-block correction. RMSNorm runs in the prologue,
//     residual / SwiGLU / argmax in the epilogue.
//   * Decode attention: split-K over the sequence, RoPE + bf16 KV append in the prologue,
//     online softmax per split, LSE merge by the last workgroup of each KV head.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "vx_common.h"

typedef _Float16 vx_h2 __attribute__((ext_vector_type(2)));
typedef uint32_t vx_u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kWG = 256;  // threads per workgroup (4 wave64)
constexpr int kU = 8;     // GEMV iterations in flight per lane (8 x 16 B)

__device__ __forceinline__ float vx_h2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)h)); }

// 8 weights of one code dword against 8 fp16 activations (4 half2). Nibble p of the low half
// holds element 2p, nibble p of the high half element 2p+1, so (h_p.x, h_p.y) = 1024 + q for the
// consecutive pair (x[2p], x[2p+1]).
__device__ __forceinline__ float vx_dot8(uint32_t q, uint4 xq, float acc) {
    const uint32_t m = 0x000F000Fu, bias = 0x64006400u;
    const uint32_t h0 = (q & m) | bias;
    const uint32_t h1 = ((q >> 4) & m) | bias;
    const uint32_t h2 = ((q >> 8) & m) | bias;
    const uint32_t h3 = ((q >> 12) & m) | bias;
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(vx_h2, h0), __builtin_bit_cast(vx_h2, xq.x), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(vx_h2, h1), __builtin_bit_cast(vx_h2, xq.y), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(vx_h2, h2), __builtin_bit_cast(vx_h2, xq.z), acc, false);
    acc = __builtin_amdgcn_fdot2(__builtin_bit_cast(vx_h2, h3), __builtin_bit_cast(vx_h2, xq.w), acc, false);
    return acc;
}

__device__ __forceinline__ float vx_wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}
__device__ __forceinline__ float vx_wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off));
    return v;
}

// (value, index) ordering of the reference's strict '>' scan: larger value wins, equal values
// resolve to the lower index; NaN never wins.
__device__ __forceinline__ bool vx_better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

// Block-wide sum over 256 threads; red must hold 4 floats. Result broadcast to all threads.
__device__ __forceinline__ float vx_block_sum(float v, float* red) {
    v = vx_wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    return (red[0] + red[1]) + (red[2] + red[3]);
}

// Places one GGML Q4_0 block (scale bits d, 16 bytes qs: element j low nibble of qs[j],
// element j+16 high nibble) into the tiled layout at physical row `phys`, block b.
__device__ __forceinline__ void vx_store_tiled_block(const VxMat& m, uint32_t phys, uint32_t b, uint16_t d,
                                                     const uint8_t* qs) {
    uint32_t dw[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        uint32_t v = 0;
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int e0 = 8 * w + 2 * p, e1 = e0 + 1;
            const uint32_t q0 = e0 < 16 ? (qs[e0] & 15u) : (qs[e0 - 16] >> 4);
            const uint32_t q1 = e1 < 16 ? (qs[e1] & 15u) : (qs[e1 - 16] >> 4);
            v |= (q0 << (4 * p)) | (q1 << (16 + 4 * p));
        }
        dw[w] = v;
    }
    const uint32_t R = 64u / m.s;
    const uint32_t tile = phys / R, rr = phys % R, i = b / m.s, s = b % m.s;
    const size_t off = ((size_t)tile * m.n_iter + i) * 64u + rr * m.s + s;
    ((uint4*)m.codes)[off] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
    ((uint16_t*)m.scales)[off] = d;
}

// Logical row j of a (possibly paired) matrix -> physical tiled row.
__device__ __forceinline__ uint32_t vx_phys_row(const VxMat& m, uint32_t j, uint32_t pair_part) {
    if (!m.paired) return j;
    const uint32_t half = (64u / m.s) / 2u;
    return (j / half) * (2u * half) + pair_part * half + (j % half);
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

__device__ __forceinline__ float vx_normal_value(uint64_t stream, uint64_t idx, float coef, float mean) {
#pragma clang fp contract(off)
    return mean + (float)vx_normal_int(stream, idx) * coef;
}

}  // namespace

// =============================================================================================
// Fused Q4_0 GEMV
// =============================================================================================
template <int S, int EPI>
__global__ __launch_bounds__(kWG) void vx_gemv_q4_kernel(VxGemvArgs a) {
    extern __shared__ __align__(16) unsigned char vx_smem[];
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr int R = 64 / S;
    const uint32_t K = a.k, nb = K >> 5;
    __half* xs = (__half*)vx_smem;
    float* corr = (float*)(vx_smem + (size_t)K * 2u);
    float* red = corr + nb;
    const int tid = threadIdx.x;

    // ---- prologue: optional RMSNorm scale (src/runtime.rs:588-601), x -> fp16 in LDS ----
    float inv_rms = 1.0f;
    if (a.gain) {
        float ss = 0.0f;
        for (uint32_t i = (uint32_t)tid * 4u; i < K; i += kWG * 4u) {
            const float4 v = *(const float4*)(a.x + i);
            ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        }
        ss = vx_block_sum(ss, red + 4);
        inv_rms = 1.0f / sqrtf(ss / (float)K + a.eps);
    }
    for (uint32_t g = tid; g < (K >> 3); g += kWG) {
        float4 v0 = *(const float4*)(a.x + 8u * g);
        float4 v1 = *(const float4*)(a.x + 8u * g + 4u);
        if (a.gain) {
            const float4 g0 = *(const float4*)(a.gain + 8u * g);
            const float4 g1 = *(const float4*)(a.gain + 8u * g + 4u);
            v0 = make_float4((v0.x * inv_rms) * g0.x, (v0.y * inv_rms) * g0.y, (v0.z * inv_rms) * g0.z,
                             (v0.w * inv_rms) * g0.w);
            v1 = make_float4((v1.x * inv_rms) * g1.x, (v1.y * inv_rms) * g1.y, (v1.z * inv_rms) * g1.z,
                             (v1.w * inv_rms) * g1.w);
        }
        const __half h[8] = {__float2half(v0.x), __float2half(v0.y), __float2half(v0.z), __float2half(v0.w),
                             __float2half(v1.x), __float2half(v1.y), __float2half(v1.z), __float2half(v1.w)};
        *(uint4*)(xs + 8u * g) = *(const uint4*)h;
        float s = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += __half2float(h[e]);
        // the four 8-element groups of one 32-block sit in four consecutive lanes
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        if ((g & 3u) == 0u) corr[g >> 2] = -1032.0f * s;
    }
    __syncthreads();

    // ---- main loop: wave-per-tile, lanes stream 16-byte code words ----
    const int lane = tid & 63, wave = tid >> 6;
    const int r = lane / S, s = lane % S;
    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    const uint32_t waves_total = gridDim.x * (kWG / 64);
    for (uint32_t tile = blockIdx.x * (kWG / 64) + wave; tile < a.n_tiles; tile += waves_total) {
        uint32_t row;
        bool row_ok;
        if constexpr (EPI == VX_EPI_SWIGLU) {
            row = tile * (R / 2) + (r % (R / 2));  // logical j of this lane's gate/up row
            row_ok = row < a.n;                    // a.n = F for paired matrices
        } else {
            row = tile * R + r;
            row_ok = row < a.n;
        }
        const size_t base = (size_t)tile * a.n_iter * 64u + lane;
        float acc = 0.0f;
        for (uint32_t i0 = 0; i0 < a.n_iter; i0 += kU) {
            uint4 c[kU];
            uint32_t dsc[kU];
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const uint32_t i = i0 + u, b = i * S + s;
                if (i < a.n_iter && b < nb && row_ok) {
                    const vx_u32x4 cv = __builtin_nontemporal_load((const vx_u32x4*)a.codes + base + (size_t)i * 64u);
                    c[u] = make_uint4(cv.x, cv.y, cv.z, cv.w);
                    dsc[u] = __builtin_nontemporal_load((const unsigned short*)a.scales + base + (size_t)i * 64u);
                } else {
                    c[u] = make_uint4(0, 0, 0, 0);
                    dsc[u] = 0;
                }
            }
#pragma unroll
            for (int u = 0; u < kU; ++u) {
                const uint32_t i = i0 + u, b = i * S + s;
                if (i < a.n_iter && b < nb && row_ok) {
                    const uint4* xq = (const uint4*)(xs + b * 32u);
                    float dot = corr[b];
                    dot = vx_dot8(c[u].x, xq[0], dot);
                    dot = vx_dot8(c[u].y, xq[1], dot);
                    dot = vx_dot8(c[u].z, xq[2], dot);
                    dot = vx_dot8(c[u].w, xq[3], dot);
                    acc = fmaf(vx_h2f(dsc[u]), dot, acc);
                }
            }
        }
#pragma unroll
        for (int off = S / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off);

        if constexpr (EPI == VX_EPI_STORE) {
            if (s == 0 && row_ok) a.y[row] = a.bias ? acc + a.bias[row] : acc;
        } else if constexpr (EPI == VX_EPI_RESID) {
            if (s == 0 && row_ok) a.y[row] = a.res[row] + acc;
        } else if constexpr (EPI == VX_EPI_SWIGLU) {
            const float up = __shfl_down(acc, 32);  // partner up row is 32 lanes above
            if (s == 0 && r < R / 2 && row_ok) {
                const float g = acc;
                a.y[row] = (g / (1.0f + expf(-g))) * up;  // src/runtime.rs:1064-1066
            }
        } else {  // VX_EPI_ARGMAX
            if (s == 0 && row_ok) {
                a.y[row] = acc;
                if (vx_better(acc, row, best_v, best_i)) { best_v = acc; best_i = row; }
            }
        }
    }

    if constexpr (EPI == VX_EPI_ARGMAX) {
        __shared__ float s_v[4];
        __shared__ uint32_t s_i[4];
        __shared__ int s_last;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) {
            const float ov = __shfl_xor(best_v, off);
            const uint32_t oi = __shfl_xor(best_i, off);
            if (vx_better(ov, oi, best_v, best_i)) { best_v = ov; best_i = oi; }
        }
        if (lane == 0) { s_v[wave] = best_v; s_i[wave] = best_i; }
        __syncthreads();
        if (tid == 0) {
            float bv = s_v[0];
            uint32_t bi = s_i[0];
            for (int w = 1; w < 4; ++w)
                if (vx_better(s_v[w], s_i[w], bv, bi)) { bv = s_v[w]; bi = s_i[w]; }
            a.cand_v[blockIdx.x] = bv;
            a.cand_i[blockIdx.x] = bi;
            __threadfence();
            const uint32_t prev = atomicAdd(a.counter, 1u);
            s_last = (prev == gridDim.x - 1u);
        }
        __syncthreads();
        if (s_last) {
            __threadfence();
            float bv = -INFINITY;
            uint32_t bi = 0xFFFFFFFFu;
            for (uint32_t j = tid; j < gridDim.x; j += kWG) {
                const float v = a.cand_v[j];
                const uint32_t ii = a.cand_i[j];
                if (vx_better(v, ii, bv, bi)) { bv = v; bi = ii; }
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) {
                const float ov = __shfl_xor(bv, off);
                const uint32_t oi = __shfl_xor(bi, off);
                if (vx_better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
            }
            __syncthreads();
            if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
            __syncthreads();
            if (tid == 0) {
                for (int w = 1; w < 4; ++w)
                    if (vx_better(s_v[w], s_i[w], s_v[0], s_i[0])) { s_v[0] = s_v[w]; s_i[0] = s_i[w]; }
                // all-NaN or empty logits: token 0, as the reference's scan from -inf
                const uint32_t win = s_i[0] == 0xFFFFFFFFu ? 0u : s_i[0];
                if (a.token_out) *a.token_out = win;
                if (a.state) {
                    // src/codegen.rs:1666-1676: ring write, then device state advance
                    const uint64_t step = a.state->step;
                    if (a.ring) {
                        __atomic_store_n(a.ring + (step & (VELOX_HIP_RING_SIZE - 1u)), win, __ATOMIC_RELAXED);
                        __threadfence_system();
                    }
                    const uint32_t plen = a.prompt_len ? *a.prompt_len : 0u;
                    const uint32_t next = (step + 1u < (uint64_t)plen) ? a.prompt[step + 1u] : win;
                    a.state->token = next;
                    a.state->step = step + 1u;
                }
                *a.counter = 0u;
            }
        }
    }
}

// =============================================================================================
// Split-K decode attention with RoPE + KV append prologue and last-workgroup LSE merge.
// =============================================================================================
template <int D, int G>
__global__ __launch_bounds__(kWG) void vx_attn_kernel(VxAttnArgs a) {
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr int HALF = D / 2, TG = kWG / D;
    __shared__ float q_s[G * D];
    __shared__ float kn[D], vn[D];
    __shared__ float p_s[G][kWG];
    __shared__ float red[G][4];
    __shared__ float o_red[TG > 1 ? TG - 1 : 1][G * D];
    __shared__ int s_last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const uint32_t g = blockIdx.y, sp = blockIdx.x;
    const uint64_t step = a.state ? a.state->step : (uint64_t)a.fixed_pos;
    const uint32_t pos = step < (uint64_t)a.s_max ? (uint32_t)step : a.s_max - 1u;  // safe_step clamp
    const uint32_t len = pos + 1u;
    const uint32_t chunk = (len + a.splits - 1u) / a.splits;
    const uint32_t t0 = sp * chunk;
    const uint32_t t1 = min(len, t0 + chunk);

    const float* q = a.qkv;
    const float* k = a.qkv + (size_t)a.hq * D;
    const float* v = k + (size_t)a.hkv * D;
    const float2* rp = a.rope + (size_t)pos * HALF;
    // rotate-half RoPE (src/runtime.rs:745-768) on this group's q heads and the new k
    for (int p = tid; p < (G + 1) * HALF; p += kWG) {
        const int hh = p / HALF, j = p % HALF;
        const float* src = hh < G ? q + (size_t)(g * G + hh) * D : k + (size_t)g * D;
        const float2 o = vx_rope_pair(src[j], src[j + HALF], rp[j]);
        const float o1 = o.x, o2 = o.y;
        if (hh < G) {
            q_s[hh * D + j] = o1;
            q_s[hh * D + j + HALF] = o2;
        } else {
            kn[j] = vx_bf16_bits_to_f32(vx_f32_to_bf16_bits(o1));
            kn[j + HALF] = vx_bf16_bits_to_f32(vx_f32_to_bf16_bits(o2));
        }
    }
    for (int d = tid; d < D; d += kWG) vn[d] = vx_bf16_bits_to_f32(vx_f32_to_bf16_bits(v[(size_t)g * D + d]));
    __syncthreads();

    uint16_t* Kc = a.kv + (size_t)g * a.s_max * D;
    uint16_t* Vc = a.kv + ((size_t)a.hkv + g) * a.s_max * D;
    if (sp == 0) {
        for (int d = tid; d < D; d += kWG) {
            Kc[(size_t)pos * D + d] = (uint16_t)(__builtin_bit_cast(uint32_t, kn[d]) >> 16);
            Vc[(size_t)pos * D + d] = (uint16_t)(__builtin_bit_cast(uint32_t, vn[d]) >> 16);
        }
    }

    float m_run[G], l_run[G], o_acc[G];
#pragma unroll
    for (int h = 0; h < G; ++h) { m_run[h] = -INFINITY; l_run[h] = 0.0f; o_acc[h] = 0.0f; }
    const int pd = tid % D, ptg = tid / D;

    for (uint32_t tt0 = t0; tt0 < t1; tt0 += kWG) {
        const uint32_t t = tt0 + tid;
        const bool valid = t < t1;
        float sc[G];
#pragma unroll
        for (int h = 0; h < G; ++h) sc[h] = 0.0f;
        if (valid) {
            if (t == pos) {
                for (int d = 0; d < D; ++d) {
                    const float kv = kn[d];
#pragma unroll
                    for (int h = 0; h < G; ++h) sc[h] += q_s[h * D + d] * kv;
                }
            } else {
                const uint4* krow = (const uint4*)(Kc + (size_t)t * D);
                for (int c8 = 0; c8 < D / 8; ++c8) {
                    const uint4 w = krow[c8];
                    const uint32_t wv[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float k0 = __builtin_bit_cast(float, wv[e] << 16);
                        const float k1 = __builtin_bit_cast(float, wv[e] & 0xFFFF0000u);
                        const int d = c8 * 8 + 2 * e;
#pragma unroll
                        for (int h = 0; h < G; ++h) {
                            sc[h] += q_s[h * D + d] * k0;
                            sc[h] += q_s[h * D + d + 1] * k1;
                        }
                    }
                }
            }
        }
        // tile max per head
#pragma unroll
        for (int h = 0; h < G; ++h) {
            sc[h] = valid ? sc[h] * a.scale : -INFINITY;
            const float wm = vx_wave_max(sc[h]);
            if (lane == 0) red[h][wave] = wm;
        }
        __syncthreads();
        float alpha[G], mnew[G];
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float tm = fmaxf(fmaxf(red[h][0], red[h][1]), fmaxf(red[h][2], red[h][3]));
            mnew[h] = fmaxf(m_run[h], tm);
            alpha[h] = (m_run[h] == -INFINITY) ? 0.0f : expf(m_run[h] - mnew[h]);
            const float p = valid ? expf(sc[h] - mnew[h]) : 0.0f;
            p_s[h][tid] = p;
            sc[h] = p;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const float ws = vx_wave_sum(sc[h]);
            if (lane == 0) red[h][wave] = ws;
        }
        __syncthreads();
#pragma unroll
        for (int h = 0; h < G; ++h) {
            l_run[h] = l_run[h] * alpha[h] + ((red[h][0] + red[h][1]) + (red[h][2] + red[h][3]));
            m_run[h] = mnew[h];
            o_acc[h] *= alpha[h];
        }
        // P.V: thread (pd, ptg) accumulates column pd over the tile positions ptg, ptg+TG, ...
        const uint32_t ntile = min((uint32_t)kWG, t1 - tt0);
        for (uint32_t tp = ptg; tp < ntile; tp += TG) {
            const uint32_t tt = tt0 + tp;
            const float vv = (tt == pos) ? vn[pd] : vx_bf16_bits_to_f32(Vc[(size_t)tt * D + pd]);
#pragma unroll
            for (int h = 0; h < G; ++h) o_acc[h] += p_s[h][tp] * vv;
        }
        __syncthreads();
    }
    // combine the TG partial column sums
    if (TG > 1) {
        if (ptg > 0) {
#pragma unroll
            for (int h = 0; h < G; ++h) o_red[ptg - 1][h * D + pd] = o_acc[h];
        }
        __syncthreads();
        if (ptg == 0) {
            for (int gg = 1; gg < TG; ++gg)
#pragma unroll
                for (int h = 0; h < G; ++h) o_acc[h] += o_red[gg - 1][h * D + pd];
        }
    }
    if (ptg == 0) {
#pragma unroll
        for (int h = 0; h < G; ++h) {
            const size_t hq_idx = (size_t)g * G + h;
            a.part_o[(hq_idx * a.splits + sp) * D + pd] = o_acc[h];
            if (pd == 0) {
                a.part_ml[(hq_idx * a.splits + sp) * 2] = m_run[h];
                a.part_ml[(hq_idx * a.splits + sp) * 2 + 1] = l_run[h];
            }
        }
    }
    __threadfence();
    __syncthreads();
    if (tid == 0) {
        const uint32_t prev = atomicAdd(a.counters + g, 1u);
        s_last = (prev == a.splits - 1u);
    }
    __syncthreads();
    if (!s_last) return;
    __threadfence();
    for (int idx = tid; idx < G * D; idx += kWG) {
        const int h = idx / D, d = idx % D;
        const size_t hq_idx = (size_t)g * G + h;
        float M = -INFINITY;
        for (uint32_t j = 0; j < a.splits; ++j) M = fmaxf(M, a.part_ml[(hq_idx * a.splits + j) * 2]);
        float L = 0.0f, O = 0.0f;
        for (uint32_t j = 0; j < a.splits; ++j) {
            const float mj = a.part_ml[(hq_idx * a.splits + j) * 2];
            if (mj == -INFINITY) continue;
            const float w = expf(mj - M);
            L += a.part_ml[(hq_idx * a.splits + j) * 2 + 1] * w;
            O += a.part_o[(hq_idx * a.splits + j) * D + d] * w;
        }
        a.out[hq_idx * D + d] = L > 0.0f ? O / L : 0.0f;
    }
    if (tid == 0) a.counters[g] = 0u;
}

// =============================================================================================
// Small kernels: embedding gather, decode state, loaders, parity helpers
// =============================================================================================
__global__ __launch_bounds__(kWG) void vx_embed_kernel(VxMat m, const VeloxDecodeState* state, uint32_t fixed_token,
                                                       float* h, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    const uint32_t token = state ? state->token : fixed_token;
    const uint32_t b = blockIdx.x * kWG + threadIdx.x, nb = m.k >> 5;
    if (b >= nb || token >= m.n) return;  // src/codegen.rs:2386-2390 guard
    const uint32_t phys = vx_phys_row(m, token, 0);
    const uint32_t R = 64u / m.s;
    const size_t off = ((size_t)(phys / R) * m.n_iter + b / m.s) * 64u + (phys % R) * m.s + b % m.s;
    const uint4 c = m.codes[off];
    const float d = vx_h2f(m.scales[off]);
    const uint32_t dw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            h[b * 32 + 8 * w + 2 * p] = (float)((int)((dw[w] >> (4 * p)) & 15u) - 8) * d;
            h[b * 32 + 8 * w + 2 * p + 1] = (float)((int)((dw[w] >> (16 + 4 * p)) & 15u) - 8) * d;
        }
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

__global__ __launch_bounds__(kWG) void vx_fill_kv_kernel(uint16_t* base, uint32_t hkv, uint32_t s_max, uint32_t d,
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
        base[(((uint64_t)kv * hkv + g) * s_max + t) * d + dd] = vx_f32_to_bf16_bits(v);
    }
}

__global__ __launch_bounds__(kWG) void vx_dequant_kernel(VxMat m, float* out) {
    const uint32_t nb = m.k >> 5;
    const uint32_t logical_rows = m.paired ? 2u * m.n : m.n;
    const size_t idx = (size_t)blockIdx.x * kWG + threadIdx.x;
    if (idx >= (size_t)logical_rows * nb) return;
    const uint32_t lr = (uint32_t)(idx / nb), b = (uint32_t)(idx % nb);
    const uint32_t phys = m.paired ? vx_phys_row(m, lr % m.n, lr / m.n) : lr;
    const uint32_t R = 64u / m.s;
    const size_t off = ((size_t)(phys / R) * m.n_iter + b / m.s) * 64u + (phys % R) * m.s + b % m.s;
    const uint4 c = m.codes[off];
    const float d = vx_h2f(m.scales[off]);
    const uint32_t dw[4] = {c.x, c.y, c.z, c.w};
    float* o = out + (size_t)lr * m.k + (size_t)b * 32u;
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            o[8 * w + 2 * p] = (float)((int)((dw[w] >> (4 * p)) & 15u) - 8) * d;
            o[8 * w + 2 * p + 1] = (float)((int)((dw[w] >> (16 + 4 * p)) & 15u) - 8) * d;
        }
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

__global__ __launch_bounds__(kWG) void vx_rmsnorm_kernel(const float* x, const float* w, uint32_t n, float eps, float* y) {
    __shared__ float red[4];
    float ss = 0.0f;
    for (uint32_t i = threadIdx.x; i < n; i += kWG) ss += x[i] * x[i];
    ss = vx_block_sum(ss, red);
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
template <int S, int EPI>
hipError_t vx_gemv_launch_t(const VxGemvArgs& a, uint32_t max_wgs, hipStream_t st) {
    const uint32_t nb = a.k >> 5;
    const size_t lds = (size_t)a.k * 2u + (size_t)nb * 4u + 64u;
    static size_t attr_lds = 64u * 1024u;
    if (lds > attr_lds) {
        if (hipFuncSetAttribute((const void*)vx_gemv_q4_kernel<S, EPI>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        attr_lds = lds;
    }
    uint32_t wgs = (a.n_tiles + 3u) / 4u;
    if (wgs > max_wgs) wgs = max_wgs;
    if (wgs == 0) wgs = 1;
    hipLaunchKernelGGL((vx_gemv_q4_kernel<S, EPI>), dim3(wgs), dim3(kWG), lds, st, a);
    return hipGetLastError();
}

template <int EPI>
hipError_t vx_gemv_dispatch_s(uint32_t s, const VxGemvArgs& a, uint32_t max_wgs, hipStream_t st) {
    switch (s) {
        case 4: return vx_gemv_launch_t<4, EPI>(a, max_wgs, st);
        case 8: return vx_gemv_launch_t<8, EPI>(a, max_wgs, st);
        case 16: return vx_gemv_launch_t<16, EPI>(a, max_wgs, st);
        case 32: return vx_gemv_launch_t<32, EPI>(a, max_wgs, st);
        case 64:
            if constexpr (EPI != VX_EPI_SWIGLU) return vx_gemv_launch_t<64, EPI>(a, max_wgs, st);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

template <int D, int G>
hipError_t vx_attn_launch_t(const VxAttnArgs& a, hipStream_t st) {
    hipLaunchKernelGGL((vx_attn_kernel<D, G>), dim3(a.splits, a.hkv), dim3(kWG), 0, st, a);
    return hipGetLastError();
}
}  // namespace

uint32_t vx_gemv_max_wgs_default() { return 2048u; }

hipError_t vx_launch_gemv(const VxMat& m, const VxGemvArgs& a0, int epi, uint32_t max_wgs, hipStream_t st) {
    VxGemvArgs a = a0;
    a.codes = m.codes;
    a.scales = m.scales;
    a.n = m.n;
    a.k = m.k;
    a.n_tiles = m.n_tiles;
    a.n_iter = m.n_iter;
    if (m.k == 0 || (m.k & 31u) != 0) return hipErrorInvalidValue;
    if ((epi == VX_EPI_SWIGLU) != (m.paired != 0)) return hipErrorInvalidValue;
    switch (epi) {
        case VX_EPI_STORE: return vx_gemv_dispatch_s<VX_EPI_STORE>(m.s, a, max_wgs, st);
        case VX_EPI_RESID: return vx_gemv_dispatch_s<VX_EPI_RESID>(m.s, a, max_wgs, st);
        case VX_EPI_SWIGLU: return vx_gemv_dispatch_s<VX_EPI_SWIGLU>(m.s, a, max_wgs, st);
        case VX_EPI_ARGMAX: return vx_gemv_dispatch_s<VX_EPI_ARGMAX>(m.s, a, max_wgs, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t vx_launch_attention(const VxAttnArgs& a, uint32_t d, hipStream_t st) {
    if (a.hkv == 0 || a.hq % a.hkv != 0 || a.splits == 0 || a.s_max == 0) return hipErrorInvalidValue;
    const uint32_t G = a.hq / a.hkv;
    if (d == 64) {
        switch (G) {
            case 1: return vx_attn_launch_t<64, 1>(a, st);
            case 2: return vx_attn_launch_t<64, 2>(a, st);
            case 3: return vx_attn_launch_t<64, 3>(a, st);
            case 4: return vx_attn_launch_t<64, 4>(a, st);
            case 8: return vx_attn_launch_t<64, 8>(a, st);
            default: return hipErrorInvalidValue;
        }
    }
    if (d == 128) {
        switch (G) {
            case 1: return vx_attn_launch_t<128, 1>(a, st);
            case 2: return vx_attn_launch_t<128, 2>(a, st);
            case 4: return vx_attn_launch_t<128, 4>(a, st);
            case 7: return vx_attn_launch_t<128, 7>(a, st);
            case 8: return vx_attn_launch_t<128, 8>(a, st);
            default: return hipErrorInvalidValue;
        }
    }
    return hipErrorInvalidValue;
}

hipError_t vx_launch_embed(const VxMat& m, const VeloxDecodeState* state, uint32_t fixed_token, float* h,
                           uint64_t mask, hipStream_t st) {
    const uint32_t nb = m.k >> 5;
    hipLaunchKernelGGL(vx_embed_kernel, dim3((nb + kWG - 1) / kWG), dim3(kWG), 0, st, m, state, fixed_token, h, mask);
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

hipError_t vx_launch_fill_kv(uint16_t* layer_base, uint32_t hkv, uint32_t s_max, uint32_t d, uint32_t n_pos,
                             uint64_t stream_k, uint64_t stream_v, float coef, hipStream_t st) {
    const uint64_t n = 2ULL * hkv * n_pos * d;
    if (n == 0) return hipSuccess;
    const size_t g = (n + kWG - 1) / kWG;
    hipLaunchKernelGGL(vx_fill_kv_kernel, dim3((unsigned)(g < 65536 ? g : 65536)), dim3(kWG), 0, st, layer_base, hkv,
                       s_max, d, n_pos, stream_k, stream_v, coef);
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

hipError_t vx_launch_rmsnorm(const float* x, const float* w, uint32_t n, float eps, float* y, hipStream_t st) {
    hipLaunchKernelGGL(vx_rmsnorm_kernel, dim3(1), dim3(kWG), 0, st, x, w, n, eps, y);
    return hipGetLastError();
}

hipError_t vx_launch_argmax(const float* x, uint32_t n, uint32_t* out, hipStream_t st) {
    hipLaunchKernelGGL(vx_argmax_kernel, dim3(1), dim3(kWG), 0, st, x, n, out);
    return hipGetLastError();
}
