// vx_gemv_g64.hip -- the reference's asymmetric group-64 4-bit format (quant_mode 2) on gfx950.
//
// The reference converts fp32 weights at load with velox_cuda_quantize_q4_group64_kernel
// (src/codegen.rs:2337-2370): per 64 consecutive weights of a row, s = (max - min) / 15 and m = min
// as fp16, q = clamp(rint((w - m) / s), 0, 15) against the fp16-rounded s and m; a weight is
// fmaf(q, s, m) (:2248-2265, :2381-2410). Here the same codes and scales land in the tiled layout
// of the 4-bit GEMV (vx_gemv_q4.h): the group's 32-weight halves are blocks 2g and 2g + 1, the even
// block's 16-bit slot holding s and the odd block's m. The GEMV instantiations of this format live
// in this translation unit, compiled beside vx_kernels.hip's Q4_0 ones.
#include "vx_gemv_q4.h"

namespace {

// One group: the reference's quantizer restated with contraction-free IEEE operations (correctly
// rounded division is HIP's default; rint is round-half-even like __float2int_rn).
__device__ __forceinline__ void vx_g64_quantize_group(const float (&x)[64], uint16_t* s_bits, uint16_t* m_bits,
                                                      uint8_t (&q)[64]) {
#pragma clang fp contract(off)
    float fmin = x[0], fmax = x[0];
#pragma unroll
    for (int i = 1; i < 64; ++i) {
        if (x[i] < fmin) fmin = x[i];
        if (x[i] > fmax) fmax = x[i];
    }
    const float scale_f = (fmax > fmin) ? ((fmax - fmin) / 15.0f) : 0.0f;
    *s_bits = vx_f32_to_f16_bits(scale_f);
    *m_bits = vx_f32_to_f16_bits(fmin);
    const float s_exact = vx_f16_bits_to_f32(*s_bits), m_exact = vx_f16_bits_to_f32(*m_bits);
    const float inv_s = (s_exact > 1.0e-12f) ? (1.0f / s_exact) : 0.0f;
#pragma unroll
    for (int i = 0; i < 64; ++i) {
        const float v = rintf((x[i] - m_exact) * inv_s);
        // the reference converts to int first (__float2int_rn), then clamps: NaN -> 0 there too
        const int qi = v != v ? 0 : (v < 0.0f ? 0 : (v > 15.0f ? 15 : (int)v));
        q[i] = (uint8_t)qi;
    }
}

// Stores group g of physical row `phys`: codes of blocks 2g and 2g + 1 in the tiled nibble order
// (element e of code dword w at bit 8 (e & 3) + 4 (e >> 2)), s and m in their slots.
__device__ __forceinline__ void vx_g64_store_group(const VxMat& m, uint32_t phys, uint32_t g, const uint8_t (&q)[64],
                                                   uint16_t s_bits, uint16_t m_bits) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        uint32_t dw[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t v = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) v |= (uint32_t)q[32 * half + 8 * w + e] << (8 * (e & 3) + 4 * (e >> 2));
            dw[w] = v;
        }
        const size_t off = vx_tiled_off(m, phys, 2u * g + (uint32_t)half);
        ((uint4*)m.codes)[off] = make_uint4(dw[0], dw[1], dw[2], dw[3]);
        ((uint16_t*)m.scales)[off] = half ? m_bits : s_bits;
    }
}

// fp32 rows [rows][k] (device) -> tiled group-64 rows [row0, row0 + rows) of part pair_part.
__global__ __launch_bounds__(256) void vx_g64_from_rows_kernel(const float* src, uint32_t rows, uint32_t row0,
                                                              uint32_t pair_part, VxMat m) {
    const uint32_t ng = m.k >> 6;
    const size_t idx = (size_t)blockIdx.x * 256u + threadIdx.x;
    if (idx >= (size_t)rows * ng) return;
    const uint32_t r = (uint32_t)(idx / ng), g = (uint32_t)(idx % ng);
    float x[64];
    const float4* p = (const float4*)(src + idx * 64u);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float4 v = p[i];
        x[4 * i] = v.x;
        x[4 * i + 1] = v.y;
        x[4 * i + 2] = v.z;
        x[4 * i + 3] = v.w;
    }
    uint16_t sb, mb;
    uint8_t q[64];
    vx_g64_quantize_group(x, &sb, &mb, q);
    vx_g64_store_group(m, vx_phys_row(m, row0 + r, pair_part), g, q, sb, mb);
}

// The seeded fp32 weights of vx_fill_normal (element (r, c) draws index r k + c), quantized.
__global__ __launch_bounds__(256) void vx_g64_synth_kernel(VxMat m, uint32_t rows, uint32_t row0, uint32_t pair_part,
                                                          uint64_t stream, float coef) {
    const uint32_t ng = m.k >> 6;
    const size_t idx = (size_t)blockIdx.x * 256u + threadIdx.x;
    if (idx >= (size_t)rows * ng) return;
    const uint32_t r = (uint32_t)(idx / ng), g = (uint32_t)(idx % ng);
    float x[64];
    const uint64_t e0 = (uint64_t)r * m.k + (uint64_t)g * 64u;
#pragma unroll 8
    for (int i = 0; i < 64; ++i) x[i] = vx_normal_value(stream, e0 + (uint64_t)i, coef, 0.0f);
    uint16_t sb, mb;
    uint8_t q[64];
    vx_g64_quantize_group(x, &sb, &mb, q);
    vx_g64_store_group(m, vx_phys_row(m, row0 + r, pair_part), g, q, sb, mb);
}

// The reference's own output layout (velox_cuda_quantize_q4_group64_kernel): packed word w of group
// g = q0 | q2 << 4 | q4 << 8 | q6 << 12 | q1 << 16 | q3 << 20 | q5 << 24 | q7 << 28 over elements
// 8w..8w+7, and (s, m) as an fp16 pair per group.
__global__ __launch_bounds__(256) void vx_g64_quantize_ref_kernel(const float* src, uint64_t n_groups,
                                                                 uint32_t* packed, uint16_t* scale_min) {
    const uint64_t g = (uint64_t)blockIdx.x * 256u + threadIdx.x;
    if (g >= n_groups) return;
    float x[64];
#pragma unroll
    for (int i = 0; i < 64; ++i) x[i] = src[g * 64u + (uint64_t)i];
    uint16_t sb, mb;
    uint8_t q[64];
    vx_g64_quantize_group(x, &sb, &mb, q);
    scale_min[2u * g] = sb;
    scale_min[2u * g + 1u] = mb;
#pragma unroll
    for (int w = 0; w < 8; ++w) {
        const uint8_t* e = q + 8 * w;
        packed[g * 8u + (uint64_t)w] = (uint32_t)e[0] | ((uint32_t)e[2] << 4) | ((uint32_t)e[4] << 8) |
                                       ((uint32_t)e[6] << 12) | ((uint32_t)e[1] << 16) | ((uint32_t)e[3] << 20) |
                                       ((uint32_t)e[5] << 24) | ((uint32_t)e[7] << 28);
    }
}

dim3 vx_g64_grid(size_t n) { return dim3((unsigned)((n + 255u) / 256u)); }

}  // namespace

hipError_t vx_launch_gemv_g64(const VxMat& m, const VxGemvArgs& a, int epi, uint32_t max_wgs, hipStream_t st) {
    return vx_launch_gemv_tiled<VX_FMT_G64>(m, a, epi, max_wgs, st);
}

hipError_t vx_launch_g64_from_rows(const float* rows_dev, uint32_t rows, uint32_t row0, uint32_t pair_part,
                                   const VxMat& m, hipStream_t st) {
    if (m.fmt != VX_FMT_G64 || (m.k & 63u) || (m.s & 1u)) return hipErrorInvalidValue;
    const size_t n = (size_t)rows * (m.k >> 6);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(vx_g64_from_rows_kernel, vx_g64_grid(n), dim3(256), 0, st, rows_dev, rows, row0, pair_part, m);
    return hipGetLastError();
}

hipError_t vx_launch_synth_g64(const VxMat& m, uint32_t rows, uint32_t row0, uint32_t pair_part, uint64_t stream,
                               float coef, hipStream_t st) {
    if (m.fmt != VX_FMT_G64 || (m.k & 63u) || (m.s & 1u)) return hipErrorInvalidValue;
    const size_t n = (size_t)rows * (m.k >> 6);
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(vx_g64_synth_kernel, vx_g64_grid(n), dim3(256), 0, st, m, rows, row0, pair_part, stream, coef);
    return hipGetLastError();
}

hipError_t vx_launch_g64_quantize_ref(const float* src, uint64_t n_groups, uint32_t* packed, uint16_t* scale_min,
                                      hipStream_t st) {
    if (n_groups == 0) return hipSuccess;
    hipLaunchKernelGGL(vx_g64_quantize_ref_kernel, vx_g64_grid(n_groups), dim3(256), 0, st, src, n_groups, packed,
                       scale_min);
    return hipGetLastError();
}
