// vx_mla.hip -- the DeepSeek-V3 absorbed multi-head latent attention layer on gfx950: fp8 (e4m3fn,
// 128x128 block scales) projection weights and a bf16 latent KV cache, for 1..32 sequences.
//
// The reference's MLA (src/runtime.rs:845-1044, emitted as velox_cuda_fused_mla_absorbed_attn,
// src/codegen.rs:2001-2109) is a single-latent-head simplification; this is the full form of the
// same absorbed computation (benchmark configuration 4): per head h,
//   q_abs_h = W_uk[h]^T q_nope_h,  s_ht = scale (q_abs_h . c_t + rope(q_rope_h) . kr_t),
//   ctx_h = softmax_t(s_ht) . c_t,  o_h = W_uv[h] ctx_h,  h_out = h + W_o [o_1 .. o_H].
// One layer step is 9 launches: RMSNorm -> GEMM [W_qa; W_kva] (split over K) -> prep (q / latent
// RMSNorms, RoPE of the new k_rope, latent append) -> GEMM W_qb -> grouped GEMM W_uk^T (absorption)
// -> attention (split over positions) -> merge -> grouped GEMM W_uv -> GEMM W_o (split over K) ->
// residual. Every GEMM is the same fp8 kernel: weights converted exactly to fp16 in registers
// (v_cvt_scalef32_pk_f16_fp8), activations fp16, v_mfma_f32_16x16x32_f16, block scales on the
// fp32 partial sums.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include <type_traits>

#include "vx_common.h"
#include "vx_mla.h"

namespace {

typedef _Float16 vm_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 vm_h2 __attribute__((ext_vector_type(2)));
typedef float vm_f4 __attribute__((ext_vector_type(4)));
typedef uint32_t vm_u4 __attribute__((ext_vector_type(4)));

constexpr int kFWaves = 4, kFDepth = 4;  // fp8 GEMM: waves per workgroup, k-tiles in flight per wave

// f32 -> e4m3fn, round to nearest even, saturating at +-448: the integer steps of the oracle's
// vxo_f32_to_e4m3, so device-synthesized codes equal the host's bit for bit.
__device__ uint8_t vm_f32_to_e4m3(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 24) & 0x80u, a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint8_t)(sign | 0x7Fu);
    if (a >= 0x43E00000u) return (uint8_t)(sign | 0x7Eu);
    const int e = (int)(a >> 23) - 127;
    if (e < -6) {
        if (a < 0x00800000u) return (uint8_t)sign;
        const uint32_t mant = (a & 0x7FFFFFu) | 0x800000u;
        const int shift = 14 - e;
        if (shift > 25) return (uint8_t)sign;
        uint32_t q = mant >> shift;
        const uint32_t rem = mant & ((1u << shift) - 1u), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint8_t)(sign | q);
    }
    uint32_t m = (a & 0x7FFFFFu) >> 20, ex = (uint32_t)(e + 7);
    const uint32_t rem = a & 0xFFFFFu, half = 0x80000u;
    if (rem > half || (rem == half && (m & 1u))) ++m;
    if (m == 8u) { m = 0u; ++ex; }
    if (ex > 15u || (ex == 15u && m == 7u)) return (uint8_t)(sign | 0x7Eu);
    return (uint8_t)(sign | (ex << 3) | m);
}

// Eight fp8 codes (bytes of two dwords, in order) -> eight fp16, exactly.
__device__ __forceinline__ vm_h8 vm_fp8x8(uint32_t a, uint32_t b) {
    const vm_h2 p0 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(a, 1.0f, false);
    const vm_h2 p1 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(a, 1.0f, true);
    const vm_h2 p2 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(b, 1.0f, false);
    const vm_h2 p3 = __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(b, 1.0f, true);
    vm_h8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

__device__ __forceinline__ vm_h8 vm_f32x8_to_h8(float4 lo, float4 hi) {
    vm_h8 r;
    r[0] = (_Float16)lo.x; r[1] = (_Float16)lo.y; r[2] = (_Float16)lo.z; r[3] = (_Float16)lo.w;
    r[4] = (_Float16)hi.x; r[5] = (_Float16)hi.y; r[6] = (_Float16)hi.z; r[7] = (_Float16)hi.w;
    return r;
}

__device__ __forceinline__ float vm_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// The seeded N(0, sigma) value of the oracle's vxo_normal: an exact integer times coef.
__device__ __forceinline__ float vm_normal(uint64_t stream, uint64_t idx, float coef) {
#pragma clang fp contract(off)
    return (float)vx_normal_int(stream, idx) * coef;
}

template <int NT>
__device__ __forceinline__ float vm_block_sum(float v, float* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < NT / 64; ++w) t += red[w];
    return t;
}

// Rotate-half RoPE pair (src/runtime.rs:761-764), unfused.
__device__ __forceinline__ float2 vm_rope_pair(float x1, float x2, float2 cs) {
#pragma clang fp contract(off)
    return make_float2(x1 * cs.x - x2 * cs.y, x2 * cs.x + x1 * cs.y);
}

}  // namespace

// =============================================================================================
// fp8 block-scaled GEMM: y[m][n] = sum_k x[m][k] W[n][k]
// =============================================================================================
// Each wave owns MR 16-row tiles over its split's k-tiles and keeps kFDepth k-tiles of weights and
// activations in flight: tile kt's 16 bytes per lane are exactly the B operands of two MFMAs
// (k-elements 16 grp + 0..7 and + 8..15 of row col), the activations of sequence col the matching
// A operands, shared by the MR tiles. Per k-tile: two MFMAs into a fresh accumulator, then
// acc += block scale * it.
template <int MT, int MR, bool XF32>
__global__ __launch_bounds__(64 * kFWaves) void vx_f8gemm_kernel(VxF8GemmArgs a) {
    if ((a.active_mask & 1ULL) == 0ULL) return;
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const uint32_t g = blockIdx.z, ks = blockIdx.y;
    const uint32_t rt0 = (blockIdx.x * kFWaves + (uint32_t)wave) * MR;
    const uint32_t kt0 = ks * a.n_kt / gridDim.y, kt1 = (ks + 1u) * a.n_kt / gridDim.y;
    const uint4* W[MR];
    const float* S[MR];
#pragma unroll
    for (int r = 0; r < MR; ++r) {
        const uint32_t rt = min(rt0 + (uint32_t)r, a.n_rt - 1u);
        W[r] = a.codes + g * a.w_gstride + (size_t)rt * a.n_kt * 64u + lane;
        S[r] = a.scales + g * a.s_gstride + (size_t)rt * a.n_kb;
    }
    const uint32_t m_last = a.batch - 1u;
    size_t xoff[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        xoff[mt] = g * a.x_gstride + (size_t)min((uint32_t)(16 * mt + col), m_last) * a.ldx + 16u * grp;
    constexpr int XW = XF32 ? 4 : 2;  // 16-byte activation loads per lane and k-tile
    uint4 wr[kFDepth][MR];
    uint4 xr[kFDepth][MT][XW];
    auto issue = [&](int u, uint32_t kt) {
#pragma unroll
        for (int r = 0; r < MR; ++r) wr[u][r] = W[r][(size_t)kt * 64u];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            if constexpr (XF32) {
                const uint4* xp = (const uint4*)((const float*)a.x + xoff[mt] + (size_t)kt * 64u);
#pragma unroll
                for (int w = 0; w < XW; ++w) xr[u][mt][w] = xp[w];
            } else {
                const uint4* xp = (const uint4*)((const uint16_t*)a.x + xoff[mt] + (size_t)kt * 64u);
#pragma unroll
                for (int w = 0; w < XW; ++w) xr[u][mt][w] = xp[w];
            }
        }
    };
    vm_f4 acc[MR][MT];
#pragma unroll
    for (int r = 0; r < MR; ++r)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[r][mt] = vm_f4{0.f, 0.f, 0.f, 0.f};
    const uint32_t kt_last = kt1 > kt0 ? kt1 - 1u : kt0;
#pragma unroll
    for (int u = 0; u < kFDepth; ++u) issue(u, min(kt0 + (uint32_t)u, kt_last));
    for (uint32_t base = kt0; base < kt1; base += kFDepth) {
#pragma unroll
        for (int u = 0; u < kFDepth; ++u) {
            const uint32_t kt = base + (uint32_t)u;
            if (kt < kt1) {
                vm_h8 x0[MT], x1[MT];
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    if constexpr (XF32) {
                        x0[mt] = vm_f32x8_to_h8(__builtin_bit_cast(float4, xr[u][mt][0]), __builtin_bit_cast(float4, xr[u][mt][1]));
                        x1[mt] = vm_f32x8_to_h8(__builtin_bit_cast(float4, xr[u][mt][2]), __builtin_bit_cast(float4, xr[u][mt][3]));
                    } else {
                        x0[mt] = __builtin_bit_cast(vm_h8, xr[u][mt][0]);
                        x1[mt] = __builtin_bit_cast(vm_h8, xr[u][mt][1]);
                    }
                }
#pragma unroll
                for (int r = 0; r < MR; ++r) {
                    const float s = S[r][kt >> 1];
                    const vm_h8 w0 = vm_fp8x8(wr[u][r].x, wr[u][r].y), w1 = vm_fp8x8(wr[u][r].z, wr[u][r].w);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt) {
                        vm_f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0[mt], w0, vm_f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                        c = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1[mt], w1, c, 0, 0, 0);
                        acc[r][mt] += s * c;
                    }
                }
            }
            issue(u, min(kt + (uint32_t)kFDepth, kt_last));
        }
    }
#pragma unroll
    for (int r = 0; r < MR; ++r) {
        const uint32_t rt = rt0 + (uint32_t)r;
        if (rt >= a.n_rt) continue;
        if (a.y16) {  // fp16 for a following GEMM: the rounding its fp32 activation loads would apply
            uint16_t* y = a.y16 + g * a.y_gstride + 16u * rt + col;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t m = (uint32_t)(16 * mt + 4 * grp + i);
                    if (m < a.batch) y[(size_t)m * a.ldy] = __builtin_bit_cast(uint16_t, (_Float16)acc[r][mt][i]);
                }
            continue;
        }
        float* y = a.y + g * a.y_gstride + (gridDim.y > 1u ? ks * a.pstride : 0u) + 16u * rt + col;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = (uint32_t)(16 * mt + 4 * grp + i);
                if (m < a.batch) y[(size_t)m * a.ldy] = acc[r][mt][i];
            }
    }
}

// =============================================================================================
// fp8 block-scaled GEMV (one sequence): the same tiled weights without the matrix cores
// =============================================================================================
// With one sequence the MFMA form computes 16 columns of which one is used and loads the activation
// fragment twice per weight word. Here lane (row c = lane & 15, group q = lane >> 4) of a wave takes
// the 16 weights of its row at k-elements 64 kt + 16 q + 0..15 (its bytes of tile kt's word),
// converts them exactly to fp16 and dots them against x staged once per workgroup in LDS (fp16,
// the rounding the MFMA form applies) with v_dot2_f32_f16, one block-scale FMA per k-tile. KW waves
// share a row tile, splitting its k-tiles; their sums meet in LDS and the first of them writes the
// 16 rows. Waves stream D words ahead, unconditionally (a clamped re-read past the end): 8 where
// eight waves share a tile (long k-ranges), else 4 (the re-reads past a short range cost more than
// the deeper queue gains).
constexpr int kFGWaves = 8;

// The activation row of group g as the LSE merge of its split partials (VxF8GemmArgs::m_part_o):
// the group's splits x lr fp16 partials come into LDS with 16-byte loads (all in flight at once),
// then thread c sums column c over the splits in split order with vx_mla_merge_kernel's weights and
// operations, so the fp32 context before its fp16 rounding is the one that kernel writes; after a
// barrier the fp16 row goes to the start of LDS, where the GEMV reads its activations. The
// launcher admits lr <= the workgroup's threads and splits x lr x 2 bytes <= 64 KiB.
__device__ __forceinline__ void vm_merge_stage(const VxF8GemmArgs& a, uint32_t g, unsigned char* smem) {
    __shared__ float s_w[64];
    const uint32_t lr = a.n_kt * 64u, splits = a.m_splits, tid = threadIdx.x, nt = blockDim.x;
    const uint4* po = (const uint4*)(a.m_part_o + (size_t)g * splits * lr);
    uint4* stage = (uint4*)smem;
    const uint32_t n16 = splits * lr / 8u;  // 16-byte units
    constexpr int U = 8;  // units per thread per pass: 64 KiB over 512 threads in one pass
    for (uint32_t i0 = 0; i0 < n16; i0 += U * nt) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) v[u] = po[min(i0 + (uint32_t)u * nt + tid, n16 - 1u)];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (i0 + (uint32_t)u * nt + tid < n16) stage[i0 + (uint32_t)u * nt + tid] = v[u];
    }
    if (tid < 64u) {
        const float* pml = a.m_part_ml + (size_t)g * splits * 2u;
        const uint32_t j = tid;
        const float mj = j < splits ? pml[2 * j] : -INFINITY;
        const float lj = j < splits ? pml[2 * j + 1] : 0.0f;
        float M = mj;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
        const float wj = mj == -INFINITY ? 0.0f : vm_exp2(mj - M);
        float Ls = lj * wj;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) Ls += __shfl_xor(Ls, off);
        s_w[j] = Ls > 0.0f ? wj * lj / Ls : 0.0f;  // the partials are o_j / l_j
    }
    __syncthreads();
    const uint16_t* st16 = (const uint16_t*)smem;
    float acc = 0.0f;
    if (tid < lr)
        for (uint32_t j = 0; j < splits; ++j)
            acc = fmaf(s_w[j], (float)__builtin_bit_cast(_Float16, st16[(size_t)j * lr + tid]), acc);
    __syncthreads();  // every column read before the row overwrites the first split's
    if (tid < lr) ((uint16_t*)smem)[tid] = __builtin_bit_cast(uint16_t, (_Float16)acc);
}

template <int KW, bool XF32>
__device__ __forceinline__ void vm_f8gemv_body(const VxF8GemmArgs& a) {
    extern __shared__ __align__(16) unsigned char vm_smem[];
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr int TPW = kFGWaves / KW;  // row tiles per workgroup
    constexpr int D = KW == 8 ? 8 : 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const uint32_t g = blockIdx.z, ks = blockIdx.y, kw = (uint32_t)wave % KW, tw = (uint32_t)wave / KW;
    const uint32_t rt = blockIdx.x * TPW + tw, rtc = min(rt, a.n_rt - 1u);
    // the workgroup's k-tiles (its split), then this wave's share of them
    const uint32_t kt0 = ks * a.n_kt / gridDim.y, kt1 = (ks + 1u) * a.n_kt / gridDim.y;
    const uint32_t w0 = kt0 + kw * (kt1 - kt0) / KW, w1 = kt0 + (kw + 1u) * (kt1 - kt0) / KW;
    const uint4* W = a.codes + g * a.w_gstride + (size_t)rtc * a.n_kt * 64u + lane;
    const float* S = a.scales + g * a.s_gstride + (size_t)rtc * a.n_kb;
    const uint32_t wl = w1 > w0 ? w1 - 1u : w0;
    uint4 wr[D];
#pragma unroll
    for (int u = 0; u < D; ++u) wr[u] = W[(size_t)min(w0 + (uint32_t)u, wl) * 64u];
    // x over the split's k-range -> LDS as fp16 (8 elements per thread and pass); with a gain, x is
    // first RMSNorm'd over its whole row (every workgroup sums the row's squares itself), in the
    // operation order of the batched RMSNorm kernel: (x * inv_rms) * gain, rounded to fp16
    uint4* xs = (uint4*)vm_smem;
    float inv = 1.0f;
    // the activation row's 4 elements at e (fp32 x): x itself, or the sum of its K-split partials
    const uint32_t nparts = a.x_nparts > 1u ? a.x_nparts : 1u;
    auto x4 = [&](size_t e) {
        const float* xb = (const float*)a.x + e;
        float4 v = *(const float4*)xb;
        for (uint32_t s = 1; s < nparts; ++s) {
            const float4 w = *(const float4*)(xb + s * a.x_pstride);
            v.x += w.x; v.y += w.y; v.z += w.z; v.w += w.w;
        }
        return v;
    };
    const uint32_t n8 = (kt1 - kt0) * 8u;
    // one pass where the workgroup stages the whole row and a thread holds at most two 8-element units:
    // the RMSNorm sum of squares comes from the registers the staging uses (one load round, not two)
    constexpr uint32_t NT1 = 64u * kFGWaves;
    const bool one_pass = XF32 && a.gain && gridDim.y == 1u && n8 <= 2u * NT1;
    float4 xu[4];
    if constexpr (XF32) {
        if (a.gain) {
            __shared__ float red_n[kFGWaves];
            const uint32_t K = a.n_kt * 64u;
            float ss = 0.0f;
            if (one_pass) {
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const uint32_t i = min((uint32_t)tid + (uint32_t)u * NT1, n8 - 1u);
                    const size_t e = g * a.x_gstride + 8u * i;
                    xu[2 * u] = x4(e);
                    xu[2 * u + 1] = x4(e + 4);
                }
#pragma unroll
                for (int u = 0; u < 2; ++u)
                    if ((uint32_t)tid + (uint32_t)u * NT1 < n8) {
                        const float4 v0 = xu[2 * u], v1 = xu[2 * u + 1];
                        ss += v0.x * v0.x + v0.y * v0.y + v0.z * v0.z + v0.w * v0.w;
                        ss += v1.x * v1.x + v1.y * v1.y + v1.z * v1.z + v1.w * v1.w;
                    }
            } else {
                for (uint32_t i = (uint32_t)tid; i < K / 4u; i += NT1) {
                    const float4 v = x4(g * a.x_gstride + 4u * i);
                    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
                }
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
            if (lane == 0) red_n[wave] = ss;
            __syncthreads();
            float t = 0.0f;
#pragma unroll
            for (int w = 0; w < kFGWaves; ++w) t += red_n[w];
            inv = 1.0f / sqrtf(t / (float)K + a.eps);
        }
    }
    if constexpr (XF32) {
        if (a.m_part_o) {
            vm_merge_stage(a, g, vm_smem);
            __syncthreads();
        }
    }
    for (uint32_t i = (uint32_t)tid; i < n8 && !(XF32 && a.m_part_o); i += NT1) {
        const size_t e = g * a.x_gstride + (size_t)kt0 * 64u + 8u * i;
        if constexpr (XF32) {
            float4 lo, hi;
            if (one_pass) {
                const bool second = i >= NT1;  // (a thread's second unit: i = tid + NT1)
                lo = second ? xu[2] : xu[0];
                hi = second ? xu[3] : xu[1];
            } else {
                lo = x4(e);
                hi = x4(e + 4);
            }
            if (a.gain) {
#pragma clang fp contract(off)
                const size_t ge = (size_t)kt0 * 64u + 8u * i;
                const float4 g0 = *(const float4*)(a.gain + ge), g1 = *(const float4*)(a.gain + ge + 4);
                lo = make_float4((lo.x * inv) * g0.x, (lo.y * inv) * g0.y, (lo.z * inv) * g0.z, (lo.w * inv) * g0.w);
                hi = make_float4((hi.x * inv) * g1.x, (hi.y * inv) * g1.y, (hi.z * inv) * g1.z, (hi.w * inv) * g1.w);
            }
            xs[i] = __builtin_bit_cast(uint4, vm_f32x8_to_h8(lo, hi));
        } else {
            xs[i] = *(const uint4*)((const uint16_t*)a.x + e);
        }
    }
    __syncthreads();
    float acc = 0.0f;
    for (uint32_t base = w0; base < w1; base += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const uint32_t kt = base + (uint32_t)u;
            if (kt < w1) {
                const uint32_t xi = (kt - kt0) * 8u + 2u * (uint32_t)grp;
                const vm_h8 x0 = __builtin_bit_cast(vm_h8, xs[xi]), x1 = __builtin_bit_cast(vm_h8, xs[xi + 1u]);
                const vm_h8 f0 = vm_fp8x8(wr[u].x, wr[u].y), f1 = vm_fp8x8(wr[u].z, wr[u].w);
                float d = 0.0f;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    d = __builtin_amdgcn_fdot2(vm_h2{f0[2 * j], f0[2 * j + 1]}, vm_h2{x0[2 * j], x0[2 * j + 1]}, d, false);
                    d = __builtin_amdgcn_fdot2(vm_h2{f1[2 * j], f1[2 * j + 1]}, vm_h2{x1[2 * j], x1[2 * j + 1]}, d, false);
                }
                acc = fmaf(S[kt >> 1], d, acc);
            }
            wr[u] = W[(size_t)min(kt + (uint32_t)D, wl) * 64u];
        }
    }
    // the row's four k-groups, then the KW waves of the tile
    acc += __shfl_xor(acc, 16);
    acc += __shfl_xor(acc, 32);
    float* red = (float*)vm_smem;  // x is no longer read: every wave passed its last LDS read below
    if constexpr (KW > 1) {
        __syncthreads();
        if (lane < 16) red[(tw * KW + kw) * 16u + (uint32_t)lane] = acc;
        __syncthreads();
        if (kw != 0) return;
        acc = 0.0f;
#pragma unroll
        for (int w = 0; w < KW; ++w) acc += red[(tw * KW + (uint32_t)w) * 16u + (uint32_t)lane % 16u];
    }
    if (lane >= 16 || rt >= a.n_rt) return;
    const size_t o = g * a.y_gstride + 16u * rt + (uint32_t)col;
    if (a.y16) {
        a.y16[o] = __builtin_bit_cast(uint16_t, (_Float16)acc);
    } else {
        float* y = a.y + o + (gridDim.y > 1u ? ks * a.pstride : 0u);
        *y = a.add_y ? *y + acc : acc;
    }
}

template <int KW, bool XF32>
__global__ __launch_bounds__(64 * kFGWaves) void vx_f8gemv_kernel(VxF8GemmArgs a) {
    vm_f8gemv_body<KW, XF32>(a);
}

// The same structure for 2..16 sequences on the matrix cores: the workgroup stages its split's
// activations of all 16 rows (zero past the batch) in LDS, fp16 [16][XR]; per k-tile a wave takes
// the A operands of its two MFMAs (row col, k-elements 16 grp + 0..7 and + 8..15) from LDS and the B
// operands from its weight word, then acc += block scale * the tile's product. KW waves per row tile
// meet in LDS; the first writes 16 rows x the batch's sequences.
template <int KW, bool XF32>
__global__ __launch_bounds__(64 * kFGWaves) void vx_f8gemm_x_kernel(VxF8GemmArgs a) {
    extern __shared__ __align__(16) unsigned char vm_smem[];
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr int TPW = kFGWaves / KW, D = KW == 8 ? 8 : 4;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int col = lane & 15, grp = lane >> 4;
    const uint32_t g = blockIdx.z, ks = blockIdx.y, kw = (uint32_t)wave % KW, tw = (uint32_t)wave / KW;
    const uint32_t rt = blockIdx.x * TPW + tw, rtc = min(rt, a.n_rt - 1u);
    const uint32_t kt0 = ks * a.n_kt / gridDim.y, kt1 = (ks + 1u) * a.n_kt / gridDim.y;
    const uint32_t w0 = kt0 + kw * (kt1 - kt0) / KW, w1 = kt0 + (kw + 1u) * (kt1 - kt0) / KW;
    const uint4* W = a.codes + g * a.w_gstride + (size_t)rtc * a.n_kt * 64u + lane;
    const float* S = a.scales + g * a.s_gstride + (size_t)rtc * a.n_kb;
    const uint32_t wl = w1 > w0 ? w1 - 1u : w0;
    uint4 wr[D];
#pragma unroll
    for (int u = 0; u < D; ++u) wr[u] = W[(size_t)min(w0 + (uint32_t)u, wl) * 64u];
    // x rows 0..15 over the split's k-range -> LDS fp16, rows XR elements apart (16 bytes of padding
    // per row: the 16 rows' operand reads fall in different banks)
    uint4* xs = (uint4*)vm_smem;
    const uint32_t n8 = (kt1 - kt0) * 8u, xr8 = n8 + 1u;  // 8-element units per row, row pitch
    for (uint32_t i = (uint32_t)tid; i < 16u * n8; i += 64u * kFGWaves) {
        const uint32_t m = i / n8, u = i % n8;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (m < a.batch) {
            const size_t e = g * a.x_gstride + (size_t)m * a.ldx + (size_t)kt0 * 64u + 8u * u;
            if constexpr (XF32) {
                const float4 lo = *(const float4*)((const float*)a.x + e), hi = *(const float4*)((const float*)a.x + e + 4);
                v = __builtin_bit_cast(uint4, vm_f32x8_to_h8(lo, hi));
            } else {
                v = *(const uint4*)((const uint16_t*)a.x + e);
            }
        }
        xs[m * xr8 + u] = v;
    }
    __syncthreads();
    // The block scales come as vector loads in a ring beside the weight words (in order with them:
    // a scalar load per k-tile waited on with the LDS reads, one memory round trip per tile), and
    // each tile's scale multiply-add waits one tile: the next tile's MFMAs are issued first, so the
    // product has completed when the VALU reads it. Past the wave's range a tile re-reads the last
    // one and adds with scale 0 (no branch in the loop); the sums keep the k order.
    uint32_t vzero;  // 0 in a VGPR the compiler cannot see through: the scale loads stay vector loads
    asm volatile("v_mov_b32 %0, 0" : "=v"(vzero));
    const float* Sv = S + vzero;
    float sr[D];
#pragma unroll
    for (int u = 0; u < D; ++u) sr[u] = Sv[min(w0 + (uint32_t)u, wl) >> 1];
    vm_f4 acc = vm_f4{0.f, 0.f, 0.f, 0.f}, tprev = vm_f4{0.f, 0.f, 0.f, 0.f};
    float sprev = 0.0f;
    // a tile's A operands are read from LDS one tile ahead (read just before its MFMAs, every tile
    // waited out an LDS round trip)
    auto xidx = [&](uint32_t kt) { return (uint32_t)col * xr8 + (min(kt, wl) - kt0) * 8u + 2u * (uint32_t)grp; };
    uint4 xc0 = xs[xidx(w0)], xc1 = xs[xidx(w0) + 1u];
    for (uint32_t base = w0; base < w1; base += D) {
#pragma unroll
        for (int u = 0; u < D; ++u) {
            const uint32_t kt = base + (uint32_t)u;
            const uint32_t xn = xidx(kt + 1u);
            const uint4 xn0 = xs[xn], xn1 = xs[xn + 1u];
            __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of this tile's MFMAs
            const vm_h8 x0 = __builtin_bit_cast(vm_h8, xc0), x1 = __builtin_bit_cast(vm_h8, xc1);
            xc0 = xn0;
            xc1 = xn1;
            const vm_h8 f0 = vm_fp8x8(wr[u].x, wr[u].y), f1 = vm_fp8x8(wr[u].z, wr[u].w);
            vm_f4 t = __builtin_amdgcn_mfma_f32_16x16x32_f16(x0, f0, vm_f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
            t = __builtin_amdgcn_mfma_f32_16x16x32_f16(x1, f1, t, 0, 0, 0);
            acc += sprev * tprev;
            tprev = t;
            sprev = kt < w1 ? sr[u] : 0.0f;
            wr[u] = W[(size_t)min(kt + (uint32_t)D, wl) * 64u];
            sr[u] = Sv[min(kt + (uint32_t)D, wl) >> 1];
        }
    }
    acc += sprev * tprev;
    vm_f4* red = (vm_f4*)vm_smem;  // reuses x: every wave passed its last LDS read at the barrier below
    if constexpr (KW > 1) {
        __syncthreads();
        red[(tw * KW + kw) * 64u + (uint32_t)lane] = acc;
        __syncthreads();
        if (kw != 0) return;
        acc = vm_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int w = 0; w < KW; ++w) acc += red[(tw * KW + (uint32_t)w) * 64u + (uint32_t)lane];
    }
    if (rt >= a.n_rt) return;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t m = 4u * (uint32_t)grp + (uint32_t)i;
        if (m >= a.batch) continue;
        const size_t o = g * a.y_gstride + (size_t)m * a.ldy + 16u * rt + (uint32_t)col;
        if (a.y16) a.y16[o] = __builtin_bit_cast(uint16_t, (_Float16)acc[i]);
        else a.y[o + (gridDim.y > 1u ? ks * a.pstride : 0u)] = acc[i];
    }
}

namespace {

template <int KW>
void vx_f8gemm_x_launch_t(const VxF8GemmArgs& a, uint32_t groups, size_t lds, hipStream_t st) {
    constexpr int TPW = kFGWaves / KW;
    const dim3 grid((a.n_rt + TPW - 1) / TPW, a.ksplit, groups), block(64 * kFGWaves);
    if (a.x_f32) hipLaunchKernelGGL((vx_f8gemm_x_kernel<KW, true>), grid, block, lds, st, a);
    else hipLaunchKernelGGL((vx_f8gemm_x_kernel<KW, false>), grid, block, lds, st, a);
}

template <int KW>
void vx_f8gemv_launch_t(const VxF8GemmArgs& a, uint32_t groups, size_t lds, hipStream_t st) {
    constexpr int TPW = kFGWaves / KW;
    const dim3 grid((a.n_rt + TPW - 1) / TPW, a.ksplit, groups), block(64 * kFGWaves);
    if (a.x_f32) hipLaunchKernelGGL((vx_f8gemv_kernel<KW, true>), grid, block, lds, st, a);
    else hipLaunchKernelGGL((vx_f8gemv_kernel<KW, false>), grid, block, lds, st, a);
}

template <int MT, int MR>
void vx_f8gemm_launch_t(const VxF8GemmArgs& a, uint32_t groups, hipStream_t st) {
    const uint32_t tiles_per_wg = kFWaves * MR;
    const dim3 grid((a.n_rt + tiles_per_wg - 1) / tiles_per_wg, a.ksplit, groups), block(64 * kFWaves);
    if (a.x_f32) hipLaunchKernelGGL((vx_f8gemm_kernel<MT, MR, true>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((vx_f8gemm_kernel<MT, MR, false>), grid, block, 0, st, a);
}

}  // namespace

// Row tiles per wave: 4 once the activation fragments of >= 8 sequences outweigh the weights.
uint32_t vx_f8gemm_rows_per_wave(uint32_t batch) { return batch >= 8 ? 4u : 1u; }

hipError_t vx_launch_f8gemm(const VxF8GemmArgs& a, uint32_t groups, hipStream_t st) {
    if (a.n_rt == 0 || a.n_kt == 0 || a.batch == 0 || a.batch > 32 || a.ksplit == 0 || a.ksplit > a.n_kt ||
        groups == 0 || (a.ldx & 7u) || a.n_kb != (a.n_kt + 1u) / 2u)
        return hipErrorInvalidValue;
    if (a.ksplit > 1u && a.pstride < (uint64_t)a.batch * a.ldy) return hipErrorInvalidValue;
    if ((a.y16 != nullptr) == (a.y != nullptr) || (a.y16 && a.ksplit != 1u)) return hipErrorInvalidValue;
    if (a.add_y && (a.batch != 1u || a.ksplit != 1u || a.y16)) return hipErrorInvalidValue;
    if (a.gain && (a.batch != 1u || !a.x_f32 || a.x_gstride)) return hipErrorInvalidValue;
    if (a.x_nparts > 1u && (!a.gain || a.x_nparts > 16u || (a.x_pstride & 3u) || a.m_part_o)) return hipErrorInvalidValue;
    if (a.m_part_o && (a.batch != 1u || !a.x_f32 || a.ksplit != 1u || a.gain || !a.m_part_ml || a.m_splits == 0 ||
                       a.m_splits > 64u || a.n_kt * 64u > 64u * kFGWaves ||
                       (uint64_t)a.m_splits * a.n_kt * 128u > 64u * 1024u))
        return hipErrorInvalidValue;
    // up to 16 sequences: activations staged in LDS (one sequence: the GEMV, else the MFMA form), if
    // the longest split's fp16 activations fit 64 KB (16 padded rows for the MFMA form; at least the
    // waves' sums that reuse the space). Waves per row tile: the fewest giving >= 256 workgroups, as
    // long as each wave keeps >= 2 k-tiles.
    const size_t kspan = (a.n_kt + a.ksplit - 1u) / a.ksplit;  // k-tiles of the longest split
    size_t lds = a.batch == 1u ? kspan * 128u : 16u * (kspan * 128u + 16u);
    if (a.m_part_o) lds = (size_t)a.m_splits * a.n_kt * 128u;  // the staged partials (the row reuses them)
    const size_t red = a.batch == 1u ? (size_t)kFGWaves * 16u * 4u : (size_t)kFGWaves * 64u * 16u;
    if (lds < red) lds = red;
    if (a.batch == 1u && lds > 64u * 1024u) return hipErrorInvalidValue;
    if (a.batch <= 16u && lds <= 64u * 1024u) {
        const uint32_t kts = a.n_kt / a.ksplit;  // k-tiles of the shortest split
        auto wgs = [&](uint32_t kw) { return (a.n_rt + kFGWaves / kw - 1u) / (kFGWaves / kw) * a.ksplit * groups; };
        uint32_t kw = 1u;
        while (kw < (uint32_t)kFGWaves && wgs(kw) < 256u && kts / (2u * kw) >= 2u) kw *= 2u;
        if (a.batch == 1u) {
            switch (kw) {
                case 1: vx_f8gemv_launch_t<1>(a, groups, lds, st); break;
                case 2: vx_f8gemv_launch_t<2>(a, groups, lds, st); break;
                case 4: vx_f8gemv_launch_t<4>(a, groups, lds, st); break;
                default: vx_f8gemv_launch_t<8>(a, groups, lds, st); break;
            }
        } else {
            switch (kw) {
                case 1: vx_f8gemm_x_launch_t<1>(a, groups, lds, st); break;
                case 2: vx_f8gemm_x_launch_t<2>(a, groups, lds, st); break;
                case 4: vx_f8gemm_x_launch_t<4>(a, groups, lds, st); break;
                default: vx_f8gemm_x_launch_t<8>(a, groups, lds, st); break;
            }
        }
        return hipGetLastError();
    }
    if (a.add_y) return hipErrorInvalidValue;
    // fewer row tiles per wave while the grid would leave CUs idle (< 256 workgroups): a wave's row
    // tiles only share its activation loads, the per-row arithmetic is the same
    uint32_t mr = vx_f8gemm_rows_per_wave(a.batch);
    auto wgs = [&](uint32_t r) { return (a.n_rt + kFWaves * r - 1u) / (kFWaves * r) * a.ksplit * groups; };
    while (mr > 1u && wgs(mr) < 256u) mr >>= 1;
    if (a.batch <= 16) {
        if (mr == 4u) vx_f8gemm_launch_t<1, 4>(a, groups, st);
        else if (mr == 2u) vx_f8gemm_launch_t<1, 2>(a, groups, st);
        else vx_f8gemm_launch_t<1, 1>(a, groups, st);
    } else {
        if (mr == 4u) vx_f8gemm_launch_t<2, 4>(a, groups, st);
        else if (mr == 2u) vx_f8gemm_launch_t<2, 2>(a, groups, st);
        else vx_f8gemm_launch_t<2, 1>(a, groups, st);
    }
    return hipGetLastError();
}

// =============================================================================================
// Weight synthesis / repack into the tiled fp8 layout
// =============================================================================================
// Source element of destination (g, r, k): the maps of VxF8Dest.
__device__ __forceinline__ void vm_dest_src(const VxF8Dest& d, uint32_t g, uint32_t r, uint32_t k, uint32_t& sr,
                                            uint32_t& sc) {
    if (d.map == VX_MAP_UKT) { sr = g * (d.dn + d.dv) + k; sc = r; }
    else if (d.map == VX_MAP_UV) { sr = g * (d.dn + d.dv) + d.dn + r; sc = k; }
    else { sr = d.row_off + r; sc = k; }
}

// Block scales of a synthesized source matrix: amax / 448 per 128x128 block (vxo_fp8_quantize).
__global__ __launch_bounds__(256) void vx_f8_synth_scales_kernel(float* scales, uint32_t rows, uint32_t cols,
                                                                 uint64_t stream, float coef) {
    __shared__ float red[4];
    const uint32_t cbn = (cols + 127u) / 128u, rb = blockIdx.x / cbn, cb = blockIdx.x % cbn;
    float amax = 0.0f;
    for (uint32_t i = threadIdx.x; i < 128u * 128u; i += 256u) {
        const uint32_t r = rb * 128u + i / 128u, c = cb * 128u + i % 128u;
        if (r < rows && c < cols) amax = fmaxf(amax, fabsf(vm_normal(stream, (uint64_t)r * cols + c, coef)));
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    if (threadIdx.x == 0) {
        const float m = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
        scales[blockIdx.x] = m > 0.0f ? m / 448.0f : 1.0f;
    }
}

// One 16-byte lane word of the destination per thread: 16 codes of row r, columns 16 j .. + 15.
__global__ __launch_bounds__(256) void vx_f8_pack_kernel(VxF8Dest d) {
    const uint64_t words_per_g = (uint64_t)(d.rows / 16u) * d.n_kt * 64u;
    const uint64_t idx = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (idx >= words_per_g * d.groups) return;
    const uint32_t g = (uint32_t)(idx / words_per_g);
    const uint64_t w = idx % words_per_g;
    const uint32_t lane = (uint32_t)(w % 64u), tile = (uint32_t)(w / 64u);
    const uint32_t rt = tile / d.n_kt, kt = tile % d.n_kt;
    const uint32_t r = rt * 16u + lane % 16u, k0 = kt * 64u + 16u * (lane / 16u);
    const uint32_t scbn = (d.src_cols + 127u) / 128u;
    uint32_t b[4] = {0u, 0u, 0u, 0u};
    for (int e = 0; e < 16; ++e) {
        const uint32_t k = k0 + (uint32_t)e;
        if (k >= d.cols) continue;
        uint32_t sr, sc;
        vm_dest_src(d, g, r, k, sr, sc);
        uint32_t code;
        if (d.src_codes) {
            code = d.src_codes[(size_t)sr * d.src_cols + sc];
        } else {
            code = vm_f32_to_e4m3(vm_normal(d.stream, (uint64_t)sr * d.src_cols + sc, d.coef) /
                                  d.src_scales[(sr / 128u) * scbn + sc / 128u]);
        }
        b[e >> 2] |= code << (8 * (e & 3));
    }
    d.codes[g * d.w_gstride + ((size_t)(d.row_tile0 + rt) * d.n_kt + kt) * 64u + lane] = make_uint4(b[0], b[1], b[2], b[3]);
    if (lane == 0 && (kt & 1u) == 0u) {
        // the scale of (row tile, 128-column block): the source block of its first element
        uint32_t sr, sc;
        vm_dest_src(d, g, rt * 16u, kt * 64u, sr, sc);
        d.scales[g * d.s_gstride + (size_t)(d.row_tile0 + rt) * d.n_kb + kt / 2u] = d.src_scales[(sr / 128u) * scbn + sc / 128u];
    }
}

hipError_t vx_launch_f8_synth_scales(float* scales, uint32_t rows, uint32_t cols, uint64_t stream, float coef,
                                     hipStream_t st) {
    const uint32_t n = ((rows + 127u) / 128u) * ((cols + 127u) / 128u);
    hipLaunchKernelGGL(vx_f8_synth_scales_kernel, dim3(n), dim3(256), 0, st, scales, rows, cols, stream, coef);
    return hipGetLastError();
}

hipError_t vx_launch_f8_pack(const VxF8Dest& d, hipStream_t st) {
    if ((d.rows & 15u) || d.cols != d.n_kt * 64u) return hipErrorInvalidValue;
    const uint64_t n = (uint64_t)(d.rows / 16u) * d.n_kt * 64u * d.groups;
    hipLaunchKernelGGL(vx_f8_pack_kernel, dim3((unsigned)((n + 255u) / 256u)), dim3(256), 0, st, d);
    return hipGetLastError();
}

// =============================================================================================
// Layer-step kernels
// =============================================================================================

// Per sequence (one workgroup): sum the K-split partials (all of an element's partials loaded at
// once); q latent RMSNorm -> fp16 (or q -> fp32); latent RMSNorm and RoPE of k_rope -> bf16 cache
// row pos (src/runtime.rs:588-601, 745-768).
constexpr uint32_t kMlaMaxParts = 16;

// The new position's latent row of sequence b: the K-split partials of outputs [q_part, na) summed,
// latent RMSNorm (kv_norm), RoPE of the rope part, bf16 -> cache row pos (src/runtime.rs:588-601,
// 745-768), by the NT threads of a workgroup; cs: LDS for lr + dr floats.
template <int NT>
__device__ __forceinline__ void vm_prep_latent(const VxMlaPrepArgs& a, uint32_t b, float* cs) {
    __shared__ float red[NT / 64];
    const uint32_t tid = threadIdx.x;
    const uint64_t step = a.states[b].step;
    const uint32_t pos = step < (uint64_t)a.s_max ? (uint32_t)step : a.s_max - 1u;
    const float* pb = a.parts + (size_t)b * a.na;
    for (uint32_t i = a.q_part + tid; i < a.na; i += NT) {
        float p[kMlaMaxParts];
#pragma unroll
        for (uint32_t s = 0; s < kMlaMaxParts; ++s) p[s] = pb[min(s, a.nparts - 1u) * a.pstride + i];
        float v = 0.0f;
#pragma unroll
        for (uint32_t s = 0; s < kMlaMaxParts; ++s)
            if (s < a.nparts) v += p[s];
        cs[i - a.q_part] = v;
    }
    __syncthreads();
    uint16_t* row = a.cache + (size_t)b * a.cache_bstride + (size_t)pos * (a.lr + a.dr);
    float inv = 1.0f;
    if (a.kv_norm) {
        float ss = 0.0f;
        for (uint32_t i = tid; i < a.lr; i += NT) ss += cs[i] * cs[i];
        ss = vm_block_sum<NT>(ss, red);
        inv = 1.0f / sqrtf(ss / (float)a.lr + a.eps);
    }
    for (uint32_t i = tid; i < a.lr; i += NT) {
#pragma clang fp contract(off)
        const float v = a.kv_norm ? (cs[i] * inv) * a.g_kva[i] : cs[i];
        row[i] = vx_f32_to_bf16_bits(v);
    }
    const uint32_t half = a.dr / 2u;
    for (uint32_t j = tid; j < half; j += NT) {
        const float2 o = vm_rope_pair(cs[a.lr + j], cs[a.lr + j + half], a.rope[(size_t)pos * half + j]);
        row[a.lr + j] = vx_f32_to_bf16_bits(o.x);
        row[a.lr + j + half] = vx_f32_to_bf16_bits(o.y);
    }
}

// One sequence: W_qb's GEMV (its prologue summing the q-latent partials and normalizing them) with
// one more workgroup, the grid's last, that appends the new latent row (the prep kernel's other half,
// off the GEMV's critical path).
template <int KW>
__global__ __launch_bounds__(64 * kFGWaves) void vx_f8gemv_prep_kernel(VxF8GemmArgs g, VxMlaPrepArgs p) {
    if (blockIdx.x == gridDim.x - 1u) {
        if ((p.active_mask & 1ULL) == 0ULL) return;
        extern __shared__ __align__(16) unsigned char vm_smem[];
        vm_prep_latent<64 * kFGWaves>(p, 0u, (float*)vm_smem);
        return;
    }
    vm_f8gemv_body<KW, true>(g);
}

__global__ __launch_bounds__(1024) void vx_mla_prep_kernel(VxMlaPrepArgs a) {
    if ((a.active_mask & 1ULL) == 0ULL) return;
    extern __shared__ __align__(16) unsigned char vm_smem[];
    float* qs = (float*)vm_smem;                  // [q_lora]
    float* cs = qs + (a.q_lora ? a.q_lora : 1u);  // [lr + dr]
    __shared__ float red[16];
    // grid (batch, 2): workgroup y = 0 takes the q outputs, y = 1 the latent and rope outputs
    const uint32_t b = blockIdx.x, tid = threadIdx.x, part = blockIdx.y;
    if (part == 1) {
        vm_prep_latent<1024>(a, b, cs);
        return;
    }
    const float* pb = a.parts + (size_t)b * a.na;
    for (uint32_t i = tid; i < a.q_part; i += 1024u) {
        float p[kMlaMaxParts];
#pragma unroll
        for (uint32_t s = 0; s < kMlaMaxParts; ++s) p[s] = pb[min(s, a.nparts - 1u) * a.pstride + i];
        float v = 0.0f;
#pragma unroll
        for (uint32_t s = 0; s < kMlaMaxParts; ++s)
            if (s < a.nparts) v += p[s];
        if (a.q_lora) qs[i] = v;
        else a.q32[(size_t)b * a.q_part + i] = v;
    }
    __syncthreads();
    if (a.q_lora) {
        float ss = 0.0f;
        for (uint32_t i = tid; i < a.q_lora; i += 1024u) ss += qs[i] * qs[i];
        ss = vm_block_sum<1024>(ss, red);
        const float inv = 1.0f / sqrtf(ss / (float)a.q_lora + a.eps);
        for (uint32_t i = tid; i < a.q_lora; i += 1024u) {
#pragma clang fp contract(off)
            const float v = (qs[i] * inv) * a.g_qa[i];
            a.q16[(size_t)b * a.ldq16 + i] = __half_as_ushort(__float2half(v));
        }
    }
}

template <int LR, int DR, int W, int LS>
constexpr size_t vx_mla_attn_lds() {  // the chunk's rows [c | kr], the waves' partial scores
    return (size_t)32 * (LR + DR + 8) * 2 + (size_t)W * LS * 2 * 64 * 16;
}

typedef short vm_s4 __attribute__((ext_vector_type(4)));
typedef __bf16 vm_b8 __attribute__((ext_vector_type(8)));

constexpr float kMlaLazy = 8.0f;  // log2 headroom of the attention's stale running maximum

// Four 16-bit values per lane from LDS, transposed within each 16-lane group: lane i of a group
// receives element i % 4 of the words that lanes 4 e + i / 4 (e = 0..3) address (ds_read_b64_tr_b16).
__device__ __forceinline__ vm_s4 vm_lds_tr4(const __bf16* p) {
    return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) vm_s4*)p);
}

// Absorbed MLA attention of one (split, sequence, group of 16 W heads). The split's positions go
// through LDS in chunks of 32, as the cache holds them (bf16 rows, copied with no conversion); the
// scores read them as rows and P.V reads the latent part transposed (ds_read_b64_tr_b16: the 8
// positions of one dimension that a lane's MFMA operand takes, from the row layout, with no
// transposed copy). Both products run on v_mfma_f32_16x16x32_bf16 with q and P rounded to bf16 (an
// fp16 copy of each chunk cost about a third of the kernel's VALU instructions).
// LS waves share each 16 heads: each computes the heads' partial scores S^T[pos][head] = [c | kr] .
// [q_abs | rope(q_rope)] over 1 / LS of the dimensions (its q operands, built once, stay in
// registers), the partials meet in LDS, every wave runs the log2-domain online
// softmax on the same sums and accumulates its 1 / LS of the latent dimensions of
// O[head][latent] += P c on MFMA (fewer registers: two waves per SIMD). Writes the split's (m, l, o).
template <int LR, int DR, int W, int LS>
__global__ __launch_bounds__(64 * W * LS, 1) void vx_mla_attn_kernel(VxMlaAttnArgs a) {
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr int R = LR + DR, NCK = R / 32, NB = LR / 16, NBW = NB / LS, KP = R + 8, NT = 64 * W * LS;
    static_assert(NB % LS == 0, "whole 16-dimension blocks per wave");
    extern __shared__ __align__(16) unsigned char vm_smem[];
    __bf16* k_s = (__bf16*)vm_smem;                          // [32][KP]: rows [c | kr], bf16 as cached
    vm_f4* ps_s = (vm_f4*)(vm_smem + (size_t)32 * KP * 2);  // partial scores [W LS][2][64]
    constexpr int NCH = NCK / LS;                            // 32-dimension chunks of a wave's scores
    static_assert(NCK % LS == 0, "whole 32-dimension chunks per wave");
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int hg = wave / LS, ls = wave % LS;  // head group of the workgroup, latent part
    const int col = lane & 15, grp = lane >> 4;
    const uint32_t sp = blockIdx.x, b = blockIdx.y;
    const uint32_t head = (blockIdx.z * W + (uint32_t)hg) * 16u + (uint32_t)col;
    const uint64_t step = a.states[b].step;
    const uint32_t pos = step < (uint64_t)a.s_max ? (uint32_t)step : a.s_max - 1u;
    const uint32_t len = pos + 1u;
    const uint32_t chunk = ((a.s_max + a.splits - 1u) / a.splits + 31u) & ~31u;
    const uint32_t t0 = sp * chunk, t1 = min(len, t0 + chunk);
    const uint32_t n_chunks = t1 > t0 ? (t1 - t0 + 31u) >> 5 : 0u;
    const uint16_t* cb_base = a.cache + (size_t)b * a.cache_bstride;

    // ---- the chunk's rows into registers (rows clamped to pos: past t1 they are masked), one
    // register set: chunk i + 1 is loaded while chunk i is computed. Unit un = 16-byte block un % (R / 8)
    // of row un / (R / 8): consecutive lanes read and write consecutive 16 bytes of a row ----
    constexpr int RB = R / 8, NU = (32 * RB + NT - 1) / NT;
    uint4 kr[NU];
    auto load_chunk = [&](uint32_t cb) {
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int un = min(tid + u * NT, 32 * RB - 1), r = un / RB, db = un % RB;
            kr[u] = *(const uint4*)(cb_base + (size_t)min(cb + (uint32_t)r, pos) * R + 8 * db);
        }
    };
    load_chunk(t0 < len ? t0 : pos & ~31u);

    // ---- q operands of head col: latent dims scaled, the RoPE part rotated, as fp16; each lane's 8
    // consecutive dimensions of a 32-dimension chunk come as vector loads (the RoPE part's 8 stay
    // within one half of the rotation). Wave ls of a head group keeps the q chunks of its share of
    // the score dimensions in registers ----
    vm_b8 qreg[NCH];
    {
        const float* qa = a.qabs + ((size_t)b * a.nh + head) * LR;
        const float* qr = a.q32 + (size_t)b * a.nh * a.dq + (size_t)head * a.dq + a.dn;
        const float2* rp = a.rope + (size_t)pos * (DR / 2);
#pragma unroll
        for (int cc = 0; cc < NCH; ++cc) {  // compile-time register index
            const int c = ls * NCH + cc;
            const int d0 = 32 * c + 8 * grp;
            float v[8];
            if (d0 < LR) {
                const float4 x0 = *(const float4*)(qa + d0), x1 = *(const float4*)(qa + d0 + 4);
                v[0] = x0.x; v[1] = x0.y; v[2] = x0.z; v[3] = x0.w;
                v[4] = x1.x; v[5] = x1.y; v[6] = x1.z; v[7] = x1.w;
            } else {
                constexpr int h2 = DR / 2;
                const int r0 = d0 - LR, i0 = r0 % h2;
                float x1[8], x2[8];
                float2 cs[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    x1[e] = qr[i0 + e];
                    x2[e] = qr[i0 + e + h2];
                    cs[e] = rp[i0 + e];
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float2 o = vm_rope_pair(x1[e], x2[e], cs[e]);
                    v[e] = r0 < h2 ? o.x : o.y;
                }
            }
            vm_b8 q;
#pragma unroll
            for (int e = 0; e < 8; ++e) q[e] = (__bf16)(v[e] * a.qscale);
            qreg[cc] = q;
        }
    }

    float m_run = -INFINITY, l_run = 0.0f;
    vm_f4 o_acc[NBW];  // latent blocks ls NBW .. + NBW - 1
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) o_acc[nb] = vm_f4{0.f, 0.f, 0.f, 0.f};

    auto chunk_step = [&](uint32_t ci) {
        const uint32_t cb = t0 + 32u * ci;
        __syncthreads();  // the previous chunk is consumed
#pragma unroll
        for (int u = 0; u < NU; ++u) {
            const int un = tid + u * NT;
            if (un < 32 * RB) *(vm_b8*)(k_s + (un / RB) * KP + 8 * (un % RB)) = __builtin_bit_cast(vm_b8, kr[u]);
        }
        __syncthreads();
        if (ci + 1u < n_chunks) load_chunk(cb + 32u);
        // scores: sc[bb][i] = S[position cb + 16 bb + 4 grp + i][head col]
        vm_f4 sc[2] = {vm_f4{0.f, 0.f, 0.f, 0.f}, vm_f4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int cc = 0; cc < NCH; ++cc) {
            const int c = ls * NCH + cc;
            const vm_b8 qop = qreg[cc];
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                const vm_b8 kop = *(const vm_b8*)(k_s + (16 * bb + col) * KP + 32 * c + 8 * grp);
                sc[bb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kop, qop, sc[bb], 0, 0, 0);
            }
        }
        {
            // the head group's LS partial scores, added in ls order by every wave (the same sums)
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) ps_s[(wave * 2 + bb) * 64 + lane] = sc[bb];
            __syncthreads();
#pragma unroll
            for (int bb = 0; bb < 2; ++bb) {
                vm_f4 t = vm_f4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int l = 0; l < LS; ++l) t += ps_s[((hg * LS + l) * 2 + bb) * 64 + lane];
                sc[bb] = t;
            }
        }
        float pr[8];
        float mx = -INFINITY;
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t p = cb + 16u * bb + 4u * grp + i;
                pr[4 * bb + i] = p < t1 ? sc[bb][i] : -INFINITY;
                mx = fmaxf(mx, pr[4 * bb + i]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // lazy rescale: the reference maximum m_run moves only when a score exceeds it by more than
        // 2^kMlaLazy (log2 units), so p = 2^(s - m_run) <= 2^kMlaLazy stays small and
        // the accumulators are rescaled only on such a jump; before the first finite maximum they
        // are still zero
        const float m_new = (m_run == -INFINITY || mx > m_run + kMlaLazy) ? mx : m_run;
        const float alpha = m_run == -INFINITY ? 0.0f : vm_exp2(m_run - m_new);
        const bool grew = m_run != -INFINITY && m_new != m_run;
        float lt = 0.0f;
        vm_b8 pop;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float p = pr[e] == -INFINITY ? 0.0f : vm_exp2(pr[e] - m_new);
            lt += p;
            pop[e] = (__bf16)p;
        }
        l_run = l_run * alpha + lt;
        m_run = m_new;
        if (__any(grew)) {  // wave-uniform
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float ai = __shfl(alpha, 4 * grp + i);
#pragma unroll
                for (int nb = 0; nb < NBW; ++nb) o_acc[nb][i] *= ai;
            }
        }
        // B operand of latent block nb: lane (dimension col, group grp) takes positions 4 grp + e and
        // 16 + 4 grp + e (e = 0..3), the positions of pop's elements; lane j of the group addresses
        // row 4 grp + j / 4 (+ 16), dimensions 4 (j % 4) .. + 3 of the block
        const __bf16* vb = k_s + (4 * grp + (col >> 2)) * KP + 16 * ls * NBW + 4 * (col & 3);
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) {
            const vm_s4 lo = vm_lds_tr4(vb + 16 * nb), hi = vm_lds_tr4(vb + 16 * KP + 16 * nb);
            const vm_b8 vop = __builtin_bit_cast(vm_b8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            o_acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop, vop, o_acc[nb], 0, 0, 0);
        }
    };
    for (uint32_t ci = 0; ci < n_chunks; ++ci) chunk_step(ci);

    // ---- the split's partial: o_acc[nb][i] is head 4 grp + i of the wave, latent dim
    // 16 (ls NBW + nb) + col; stored as o / l in fp16 (a convex combination of latent rows, so
    // within their range; an empty split stores 0) ----
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    const uint32_t hbase = (blockIdx.z * W + (uint32_t)hg) * 16u;
    const size_t bh = (size_t)b * a.nh;
    if (lane < 16 && ls == 0) {
        a.part_ml[((bh + hbase + lane) * a.splits + sp) * 2] = m_run;
        a.part_ml[((bh + hbase + lane) * a.splits + sp) * 2 + 1] = l_run;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float lh = __shfl(l_run, 4 * grp + i);  // l of head 4 grp + i (lanes 0..15 hold heads 0..15)
        const float inv = lh > 0.0f ? 1.0f / lh : 0.0f;
        uint16_t* po = a.part_o + ((bh + hbase + 4u * grp + i) * a.splits + sp) * LR + 16 * ls * NBW + col;
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) po[16 * nb] = __builtin_bit_cast(uint16_t, (_Float16)(o_acc[nb][i] * inv));
    }
}

// LSE merge of the split partials of one (head, sequence) -> ctx[b][h][LR] fp32. A workgroup covers
// 128 latent dimensions of its (head, sequence) (grid z), one per thread. The first NL splits'
// loads are issued before the split weights are computed (they do not depend on them), then NL at
// a time ahead of their adds (the adds stay in split order); NL = 8 for at most 8 splits, so no
// load repeats a clamped split.
template <int NL>
__global__ __launch_bounds__(128) void vx_mla_merge_kernel(const uint16_t* part_o, const float* part_ml, uint32_t nh,
                                                           uint32_t splits, uint32_t lr, float* ctx, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    __shared__ float s_w[64];
    const size_t bh = (size_t)blockIdx.y * nh + blockIdx.x;
    const uint16_t* po = part_o + bh * splits * lr;
    const uint32_t d = blockIdx.z * 128u + threadIdx.x, dc = min(d, lr - 1u);
    float v[NL];
    auto load = [&](uint32_t j0) {
#pragma unroll
        for (uint32_t u = 0; u < (uint32_t)NL; ++u)
            v[u] = (float)__builtin_bit_cast(_Float16, po[(size_t)min(j0 + u, splits - 1u) * lr + dc]);
    };
    load(0u);
    const float* pml = part_ml + bh * splits * 2u;
    if (threadIdx.x < 64) {
        const int j = threadIdx.x;
        const float mj = j < (int)splits ? pml[2 * j] : -INFINITY;
        const float lj = j < (int)splits ? pml[2 * j + 1] : 0.0f;
        float M = mj;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
        const float wj = mj == -INFINITY ? 0.0f : vm_exp2(mj - M);
        float Ls = lj * wj;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) Ls += __shfl_xor(Ls, off);
        s_w[j] = Ls > 0.0f ? wj * lj / Ls : 0.0f;  // the partials are o_j / l_j
    }
    __syncthreads();
    float acc = 0.0f;
    for (uint32_t j0 = 0; j0 < splits; j0 += (uint32_t)NL) {
        if (j0) load(j0);
#pragma unroll
        for (uint32_t u = 0; u < (uint32_t)NL; ++u)
            if (j0 + u < splits) acc = fmaf(s_w[j0 + u], v[u], acc);
    }
    if (d < lr) ctx[bh * lr + d] = acc;
}

// h[b] += the K-split partials of W_o, in split order.
__global__ __launch_bounds__(256) void vx_mla_resid_kernel(float* h, const float* parts, uint32_t nparts,
                                                           uint64_t pstride, uint32_t n, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    const uint32_t i = blockIdx.x * 256u + threadIdx.x, b = blockIdx.y;
    if (i >= n) return;
    float v = h[(size_t)b * n + i];
    for (uint32_t s = 0; s < nparts; ++s) v += parts[s * pstride + (size_t)b * n + i];
    h[(size_t)b * n + i] = v;
}

// W_qb's one-sequence GEMV (x the q-latent partials, normalized in its prologue) plus the workgroup
// that appends the new latent row (p: the prep kernel's arguments, sequence 0).
hipError_t vx_launch_f8gemv_prep(const VxF8GemmArgs& a, const VxMlaPrepArgs& p, hipStream_t st) {
    if (a.batch != 1u || !a.x_f32 || !a.gain || a.ksplit != 1u || a.m_part_o || !a.y || a.add_y || a.n_rt == 0 ||
        a.n_kt == 0 || a.n_kb != (a.n_kt + 1u) / 2u || p.nparts == 0 || p.nparts > kMlaMaxParts ||
        p.na != p.q_part + p.lr + p.dr || (p.dr & 1u) || !p.cache || !p.states)
        return hipErrorInvalidValue;
    if (a.x_nparts > 1u && (a.x_nparts > 16u || (a.x_pstride & 3u))) return hipErrorInvalidValue;
    size_t lds = (size_t)a.n_kt * 128u;
    const size_t red = (size_t)kFGWaves * 16u * 4u, lat = (size_t)(p.na - p.q_part) * 4u;
    if (lds < red) lds = red;
    if (lds < lat) lds = lat;
    if (lds > 64u * 1024u) return hipErrorInvalidValue;
    const uint32_t kts = a.n_kt;
    auto wgs = [&](uint32_t kw) { return (a.n_rt + kFGWaves / kw - 1u) / (kFGWaves / kw); };
    uint32_t kw = 1u;
    while (kw < (uint32_t)kFGWaves && wgs(kw) < 256u && kts / (2u * kw) >= 2u) kw *= 2u;
    const dim3 block(64 * kFGWaves);
    switch (kw) {
        case 1: hipLaunchKernelGGL(vx_f8gemv_prep_kernel<1>, dim3(wgs(1) + 1u), block, lds, st, a, p); break;
        case 2: hipLaunchKernelGGL(vx_f8gemv_prep_kernel<2>, dim3(wgs(2) + 1u), block, lds, st, a, p); break;
        case 4: hipLaunchKernelGGL(vx_f8gemv_prep_kernel<4>, dim3(wgs(4) + 1u), block, lds, st, a, p); break;
        default: hipLaunchKernelGGL(vx_f8gemv_prep_kernel<8>, dim3(wgs(8) + 1u), block, lds, st, a, p); break;
    }
    return hipGetLastError();
}

hipError_t vx_launch_mla_prep(const VxMlaPrepArgs& a, uint32_t batch, hipStream_t st) {
    const size_t lds = ((size_t)(a.q_lora ? a.q_lora : 1u) + a.lr + a.dr) * 4;
    if (lds > 60000 || a.na != a.q_part + a.lr + a.dr || (a.dr & 1u) || a.nparts == 0 || a.nparts > kMlaMaxParts)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(vx_mla_prep_kernel, dim3(batch, 2), dim3(1024), lds, st, a);
    return hipGetLastError();
}

template <int LR, int DR, int W, int LS>
hipError_t vx_mla_attn_launch_t(const VxMlaAttnArgs& a, uint32_t batch, hipStream_t st) {
    constexpr size_t lds = vx_mla_attn_lds<LR, DR, W, LS>();
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)vx_mla_attn_kernel<LR, DR, W, LS>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        attr_set = true;
    }
    hipLaunchKernelGGL((vx_mla_attn_kernel<LR, DR, W, LS>), dim3(a.splits, batch, a.nh / (16u * W)),
                       dim3(64 * W * LS), lds, st, a);
    return hipGetLastError();
}

hipError_t vx_launch_mla_attn(const VxMlaAttnArgs& a, uint32_t lr, uint32_t dr, uint32_t batch, hipStream_t st) {
    if (a.splits == 0 || a.splits > 64 || (a.s_cap & 31u) || a.s_cap < a.s_max || a.nh % 16u || dr != 64u)
        return hipErrorInvalidValue;
    // 4-wave workgroups (32 heads) where 8-wave ones (64 heads) would leave CUs idle: B=1 at 64
    // splits, 12.7 against 16.8 us (2-wave ones: 16.5)
    if (lr == 512 && a.nh % 64u == 0 && (uint64_t)a.splits * batch * (a.nh / 64u) < 256u)
        return vx_mla_attn_launch_t<512, 64, 2, 2>(a, batch, st);
    if (lr == 512 && a.nh % 64u == 0) return vx_mla_attn_launch_t<512, 64, 4, 2>(a, batch, st);
    if (lr == 128 && a.nh % 16u == 0) return vx_mla_attn_launch_t<128, 64, 1, 2>(a, batch, st);
    return hipErrorInvalidValue;
}

hipError_t vx_launch_mla_merge(const uint16_t* part_o, const float* part_ml, uint32_t nh, uint32_t splits, uint32_t lr,
                               float* ctx, uint32_t batch, uint64_t mask, hipStream_t st) {
    if (splits == 0 || splits > 64 || lr == 0) return hipErrorInvalidValue;
    const dim3 grid(nh, batch, (lr + 127u) / 128u);
    if (splits <= 8u)
        hipLaunchKernelGGL(vx_mla_merge_kernel<8>, grid, dim3(128), 0, st, part_o, part_ml, nh, splits, lr, ctx, mask);
    else
        hipLaunchKernelGGL(vx_mla_merge_kernel<32>, grid, dim3(128), 0, st, part_o, part_ml, nh, splits, lr, ctx, mask);
    return hipGetLastError();
}

hipError_t vx_launch_mla_resid(float* h, const float* parts, uint32_t nparts, uint64_t pstride, uint32_t n,
                               uint32_t batch, uint64_t mask, hipStream_t st) {
    hipLaunchKernelGGL(vx_mla_resid_kernel, dim3((n + 255u) / 256u, batch), dim3(256), 0, st, h, parts, nparts, pstride,
                       n, mask);
    return hipGetLastError();
}

// Latent rows [0, n_pos) of one sequence := bf16 of seeded N(0, sigma): element (t, d) draws index
// t * row + d of the stream (the tests' numpy fill of the same stream, rounded to bf16).
__global__ __launch_bounds__(256) void vx_mla_fill_cache_kernel(uint16_t* dst, uint64_t n, uint64_t stream, float coef) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < n; i += (uint64_t)gridDim.x * 256u)
        dst[i] = vx_f32_to_bf16_bits(vm_normal(stream, i, coef));
}

hipError_t vx_launch_mla_fill_cache(uint16_t* dst, uint64_t n, uint64_t stream, float coef, hipStream_t st) {
    if (n == 0) return hipSuccess;
    const uint64_t g = (n + 255u) / 256u;
    hipLaunchKernelGGL(vx_mla_fill_cache_kernel, dim3((unsigned)(g < 65536u ? g : 65536u)), dim3(256), 0, st, dst, n,
                       stream, coef);
    return hipGetLastError();
}

// End of an MLA decode step: every active sequence's position moves to the next one (the reference's
// graph step advances its state in its final kernel, src/codegen.rs:1590-1677).
__global__ __launch_bounds__(64) void vx_mla_advance_kernel(VeloxDecodeState* states, uint32_t batch, uint64_t mask) {
    if (!(mask & 1ULL)) return;
    const uint32_t b = threadIdx.x;
    if (b < batch) states[b].step += 1u;
}

hipError_t vx_launch_mla_advance(VeloxDecodeState* states, uint32_t batch, uint64_t mask, hipStream_t st) {
    if (batch == 0 || batch > 64) return hipErrorInvalidValue;
    hipLaunchKernelGGL(vx_mla_advance_kernel, dim3(1), dim3(64), 0, st, states, batch, mask);
    return hipGetLastError();
}
