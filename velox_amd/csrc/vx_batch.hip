// vx_batch.hip -- the batched decode and batched prefill steps around the MFMA GEMM (vx_mgemm.hip):
// per-row embedding, RMSNorm into the GEMM's fp16 block-major operands, split merge, argmax
// finalize, and the prefill chunk's row states and K/V rows.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "vx_common.h"

namespace {

typedef _Float16 vx_bh2 __attribute__((ext_vector_type(2)));

// K splits of a RESID GEMM that one batched RMSNorm folds in, loaded kBNormPartGroup at a time
constexpr uint32_t kBNormMaxParts = 32, kBNormPartGroup = 8;

__device__ __forceinline__ float vx_bh2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)h)); }

// (value, index) order of the reference's strict '>' scan: equal values resolve to the lower index
__device__ __forceinline__ bool vx_bbetter(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

}  // namespace

// =============================================================================================
// The rest of a batched decode step: one grid row (or workgroup) per sequence
// =============================================================================================
namespace {

__device__ __forceinline__ uint32_t vx_bnibble(uint32_t dw, int e) { return (dw >> (8 * (e & 3) + 4 * (e >> 2))) & 15u; }

template <int W>
__device__ __forceinline__ float vx_bblock_sum(float v, float* red) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) t += red[w];
    return t;
}

}  // namespace

// h[b] = embedding row of states[b].token, dequantized (src/codegen.rs:2381-2410 per sequence).
__global__ __launch_bounds__(256) void vx_bembed_kernel(VxMat m, const VeloxDecodeState* states, float* h,
                                                        uint32_t ldh, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    const uint32_t b = blockIdx.y, token = states[b].token;
    const uint32_t blk = blockIdx.x * 256u + threadIdx.x, nb = m.k >> 5;
    if (blk >= nb || token >= m.n) return;  // src/codegen.rs:2386-2390 guard
    const uint32_t R = 64u / m.s;
    const size_t off = ((size_t)(token / R) * m.n_iter + blk / m.s) * 64u + (token % R) * m.s + blk % m.s;
    const uint4 c = m.codes[off];
    const float d = vx_bh2f(m.scales[off]);
    const uint32_t dw[4] = {c.x, c.y, c.z, c.w};
    float* o = h + (size_t)b * ldh + (size_t)blk * 32u;
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[8 * w + e] = (float)((int)vx_bnibble(dw[w], e) - 8) * d;
}

// x16[b] = fp16((h[b] / rms(h[b])) * g): the RMSNorm of src/runtime.rs:588-601 per sequence, written
// as the fp16 operand of the batched GEMM (the product is rounded to fp32 first, as in the GEMV).
// With parts, h[b] first takes the K-split partial sums of the RESID GEMM before it, added in split
// order and written back. One workgroup of 1024 threads per sequence holds the row in registers
// (NV float4 per thread), so every load of the row and of its partials is issued at once.
template <int NV>
__global__ __launch_bounds__(1024) void vx_bnorm_kernel(float* h, uint32_t ldh, const float* parts, uint32_t nparts,
                                                        uint64_t pstride, const float* g, uint32_t k, float eps,
                                                        uint16_t* x16, uint32_t ldx, uint32_t xbs, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    __shared__ float red[16];
    const uint32_t b = blockIdx.x, k4 = k >> 2;
    float4* x = (float4*)(h + (size_t)b * ldh);
    float4 v[NV];
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = min(threadIdx.x + 1024u * j, k4 - 1u);
        v[j] = x[i];
    }
    if (parts) {
        // partials added in split order; each group of kBNormPartGroup is loaded before its first
        // add (split index clamped; the adds past nparts are skipped)
        for (uint32_t s0 = 0; s0 < nparts; s0 += kBNormPartGroup) {
            float4 p[kBNormPartGroup][NV];
#pragma unroll
            for (uint32_t s = 0; s < kBNormPartGroup; ++s)
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    const uint32_t i = min(threadIdx.x + 1024u * j, k4 - 1u);
                    p[s][j] = ((const float4*)(parts + min(s0 + s, nparts - 1u) * pstride + (size_t)b * ldh))[i];
                }
#pragma unroll
            for (uint32_t s = 0; s < kBNormPartGroup; ++s)
                if (s0 + s < nparts)
#pragma unroll
                    for (int j = 0; j < NV; ++j) {
                        v[j].x += p[s][j].x;
                        v[j].y += p[s][j].y;
                        v[j].z += p[s][j].z;
                        v[j].w += p[s][j].w;
                    }
        }
#pragma unroll
        for (int j = 0; j < NV; ++j)
            if (threadIdx.x + 1024u * j < k4) x[threadIdx.x + 1024u * j] = v[j];
    }
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NV; ++j)
        if (threadIdx.x + 1024u * j < k4) ss += v[j].x * v[j].x + v[j].y * v[j].y + v[j].z * v[j].z + v[j].w * v[j].w;
    ss = vx_bblock_sum<16>(ss, red);
    const float inv = 1.0f / sqrtf(ss / (float)k + eps);
    const float4* g4 = (const float4*)g;
#pragma unroll
    for (int j = 0; j < NV; ++j) {
        const uint32_t i = threadIdx.x + 1024u * j;
        if (i >= k4) continue;
        const float4 gg = g4[i];
        uint16_t o[4];
        {
#pragma clang fp contract(off)
            o[0] = __half_as_ushort(__float2half((v[j].x * inv) * gg.x));
            o[1] = __half_as_ushort(__float2half((v[j].y * inv) * gg.y));
            o[2] = __half_as_ushort(__float2half((v[j].z * inv) * gg.z));
            o[3] = __half_as_ushort(__float2half((v[j].w * inv) * gg.w));
        }
        *(uint2*)(x16 + (size_t)b * ldx + (size_t)(i >> 3) * xbs + 4u * (i & 7u)) =
            make_uint2(o[0] | ((uint32_t)o[1] << 16), o[2] | ((uint32_t)o[3] << 16));
    }
}

// LSE merge of one sequence's split partials of one q head (m, l in the log2 domain), written as
// the fp16 operand of the o_proj GEMM.
template <int D>
__global__ __launch_bounds__(D) void vx_bmerge_kernel(const float* part_o, const float* part_ml, uint32_t hq,
                                                      uint32_t splits, uint16_t* x16, uint32_t ldx, uint32_t xbs,
                                                      uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    __shared__ float s_w[64];
    const int tid = threadIdx.x;
    const size_t h = blockIdx.x, b = blockIdx.y;
    const float* po = part_o + (b * hq + h) * splits * D;
    const float* pml = part_ml + (b * hq + h) * splits * 2u;
    if (tid < 64) {
        const float mj = tid < (int)splits ? pml[tid * 2] : -INFINITY;
        const float lj = tid < (int)splits ? pml[tid * 2 + 1] : 0.0f;
        float M = mj;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) M = fmaxf(M, __shfl_xor(M, off));
        const float wj = mj == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mj - M);
        float Ls = lj * wj;
#pragma unroll
        for (int off = 32; off > 0; off >>= 1) Ls += __shfl_xor(Ls, off);
        s_w[tid] = Ls > 0.0f ? wj / Ls : 0.0f;
    }
    __syncthreads();
    float acc = 0.0f;
    for (uint32_t j = 0; j < splits; ++j) acc += s_w[j] * po[j * D + tid];
    const size_t e = h * D + tid;
    x16[b * ldx + (e >> 5) * xbs + (e & 31u)] = __half_as_ushort(__float2half(acc));
}

// Per sequence: the argmax over the LM head's workgroup candidates (lowest index on ties), the
// ring entry ring_b[step & 1023], and the state advance with teacher forcing while step + 1 <
// plen_b (src/runtime.rs:1078-1088; src/codegen.rs:1590-1677 per sequence).
__global__ __launch_bounds__(256) void vx_bfinalize_kernel(const float* cand_v, const uint32_t* cand_i, uint32_t n,
                                                           VeloxDecodeState* states, uint32_t* rings,
                                                           const uint32_t* prompts, const uint32_t* plens,
                                                           uint32_t prompt_stride, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    __shared__ float s_v[4];
    __shared__ uint32_t s_i[4];
    const uint32_t b = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t j = tid; j < n; j += 256) {
        const float v = cand_v[(size_t)b * n + j];
        const uint32_t ii = cand_i[(size_t)b * n + j];
        if (vx_bbetter(v, ii, bv, bi)) { bv = v; bi = ii; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        if (vx_bbetter(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w)
            if (vx_bbetter(s_v[w], s_i[w], s_v[0], s_i[0])) { s_v[0] = s_v[w]; s_i[0] = s_i[w]; }
        const uint32_t win = s_i[0] == 0xFFFFFFFFu ? 0u : s_i[0];
        VeloxDecodeState* st = states + b;
        const uint64_t step = st->step;
        if (rings) {
            __atomic_store_n(rings + (size_t)b * VELOX_HIP_RING_SIZE + (step & (VELOX_HIP_RING_SIZE - 1u)), win,
                             __ATOMIC_RELAXED);
            __threadfence_system();
        }
        const uint32_t plen = plens ? plens[b] : 0u;
        const uint32_t next = (step + 1u < (uint64_t)plen) ? prompts[(size_t)b * prompt_stride + step + 1u] : win;
        st->token = next;
        st->step = step + 1u;
    }
}

// ---- batched prefill: the rows of a chunk are consecutive positions of one sequence ----

// Row r of the chunk: position p0 + r, input token prompt[p0 + r].
__global__ __launch_bounds__(64) void vx_prefill_rows_kernel(VeloxDecodeState* rows, uint32_t n_rows, uint64_t p0,
                                                             const uint32_t* prompt, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    for (uint32_t r = threadIdx.x; r < n_rows; r += 64u) {
        rows[r].step = p0 + r;
        rows[r].token = prompt[p0 + r];
    }
}

// K/V of every row into the one sequence's cache before the chunk's attention reads them: RoPE of
// k at the row's position (src/runtime.rs:745-768), bf16 K row and V slot.
__global__ __launch_bounds__(64) void vx_kv_append_rows_kernel(const float* qkv, uint32_t ldq, uint32_t nparts,
                                                               uint64_t pstride, const float* bias, uint32_t hq,
                                                               uint32_t hkv, uint32_t d, const VeloxDecodeState* rows,
                                                               const float2* rope, uint32_t s_max, uint32_t s_cap,
                                                               uint16_t* kv, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    const uint32_t g = blockIdx.x, r = blockIdx.y, half = d / 2u;
    const uint64_t step = rows[r].step;
    const uint32_t pos = step < (uint64_t)s_max ? (uint32_t)step : s_max - 1u;
    const uint32_t kc = (hq + g) * d, vc = (hq + hkv + g) * d;  // columns of this group's k and v
    const float* row = qkv + (size_t)r * ldq;
    // element c of the row: the value, or its K-split partials summed in split order (+ bias), every
    // partial's load issued before the first add
    auto at = [&](uint32_t c) {
        if (nparts == 0) return row[c];
        float t[8];
#pragma unroll
        for (uint32_t p = 0; p < 8; ++p) t[p] = row[min(p, nparts - 1u) * pstride + c];
        float acc = 0.0f;
#pragma unroll
        for (uint32_t p = 0; p < 8; ++p)
            if (p < nparts) acc += t[p];
        return bias ? acc + bias[c] : acc;
    };
    uint16_t* Kc = kv + (size_t)g * s_cap * d;
    uint16_t* Vc = kv + ((size_t)hkv + g) * s_cap * d;
    for (uint32_t j = threadIdx.x; j < half; j += 64u) {
        const float2 cs = rope[(size_t)pos * half + j];
        const float x1 = at(kc + j), x2 = at(kc + j + half);
        float o1, o2;
        {
#pragma clang fp contract(off)
            o1 = x1 * cs.x - x2 * cs.y;
            o2 = x2 * cs.x + x1 * cs.y;
        }
        Kc[(size_t)pos * d + j] = vx_f32_to_bf16_bits(o1);
        Kc[(size_t)pos * d + j + half] = vx_f32_to_bf16_bits(o2);
    }
    uint16_t* vb = Vc + (size_t)(pos >> 5) * d * 32u + vx_vslot(pos & 31u);
    for (uint32_t i = threadIdx.x; i < d; i += 64u) vb[(size_t)i * 32u] = vx_f32_to_bf16_bits(at(vc + i));
}

// Per row: the argmax over the LM head's candidates into the ring at the row's position; the last
// row sets the sequence's state: position p0 + n_rows, the next prompt token while inside the
// prompt, else the argmax (the token-by-token prefill's teacher forcing, src/runtime.rs:1078-1088).
__global__ __launch_bounds__(256) void vx_prefill_finalize_kernel(const float* cand_v, const uint32_t* cand_i,
                                                                  uint32_t n, const VeloxDecodeState* rows,
                                                                  uint32_t n_rows, uint32_t* ring,
                                                                  VeloxDecodeState* state, const uint32_t* prompt,
                                                                  const uint32_t* plen, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    __shared__ float s_v[4];
    __shared__ uint32_t s_i[4];
    const uint32_t r = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    float bv = -INFINITY;
    uint32_t bi = 0xFFFFFFFFu;
    for (uint32_t j = tid; j < n; j += 256) {
        const float v = cand_v[(size_t)r * n + j];
        const uint32_t ii = cand_i[(size_t)r * n + j];
        if (vx_bbetter(v, ii, bv, bi)) { bv = v; bi = ii; }
    }
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        const float ov = __shfl_xor(bv, off);
        const uint32_t oi = __shfl_xor(bi, off);
        if (vx_bbetter(ov, oi, bv, bi)) { bv = ov; bi = oi; }
    }
    if (lane == 0) { s_v[wave] = bv; s_i[wave] = bi; }
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 4; ++w)
            if (vx_bbetter(s_v[w], s_i[w], s_v[0], s_i[0])) { s_v[0] = s_v[w]; s_i[0] = s_i[w]; }
        const uint32_t win = s_i[0] == 0xFFFFFFFFu ? 0u : s_i[0];
        const uint64_t step = rows[r].step;
        if (ring) {
            __atomic_store_n(ring + (step & (VELOX_HIP_RING_SIZE - 1u)), win, __ATOMIC_RELAXED);
            __threadfence_system();
        }
        if (r + 1u == n_rows) {
            const uint32_t p = plen ? plen[0] : 0u;
            state->token = (step + 1u < (uint64_t)p) ? prompt[step + 1u] : win;
            state->step = step + 1u;
        }
    }
}

hipError_t vx_launch_prefill_rows(VeloxDecodeState* rows, uint32_t n_rows, uint64_t p0, const uint32_t* prompt,
                                  uint64_t mask, hipStream_t st) {
    hipLaunchKernelGGL(vx_prefill_rows_kernel, dim3(1), dim3(64), 0, st, rows, n_rows, p0, prompt, mask);
    return hipGetLastError();
}

hipError_t vx_launch_kv_append_rows(const float* qkv, uint32_t ldq, uint32_t nparts, uint64_t pstride,
                                    const float* bias, uint32_t hq, uint32_t hkv, uint32_t d,
                                    const VeloxDecodeState* rows, uint32_t n_rows, const float2* rope, uint32_t s_max,
                                    uint32_t s_cap, uint16_t* kv, uint64_t mask, hipStream_t st) {
    if ((s_cap & 31u) || s_cap < s_max || (d & 1u) || nparts > 8) return hipErrorInvalidValue;
    hipLaunchKernelGGL(vx_kv_append_rows_kernel, dim3(hkv, n_rows), dim3(64), 0, st, qkv, ldq, nparts, pstride, bias,
                       hq, hkv, d, rows, rope, s_max, s_cap, kv, mask);
    return hipGetLastError();
}

hipError_t vx_launch_prefill_finalize(const float* cand_v, const uint32_t* cand_i, uint32_t n,
                                      const VeloxDecodeState* rows, uint32_t n_rows, uint32_t* ring,
                                      VeloxDecodeState* state, const uint32_t* prompt, const uint32_t* plen,
                                      uint64_t mask, hipStream_t st) {
    hipLaunchKernelGGL(vx_prefill_finalize_kernel, dim3(n_rows), dim3(256), 0, st, cand_v, cand_i, n, rows, n_rows,
                       ring, state, prompt, plen, mask);
    return hipGetLastError();
}

hipError_t vx_launch_bembed(const VxMat& m, const VeloxDecodeState* states, uint32_t batch, float* h, uint32_t ldh,
                            uint64_t mask, hipStream_t st) {
    const uint32_t nb = m.k >> 5;
    hipLaunchKernelGGL(vx_bembed_kernel, dim3((nb + 255u) / 256u, batch), dim3(256), 0, st, m, states, h, ldh, mask);
    return hipGetLastError();
}

// Activation operand layout check: row-major (xbs 32, rows ldx >= k apart) or block-major (rows
// ldx >= 32 apart inside blocks of xbs >= batch * ldx elements), with 8-byte aligned 4-element runs.
bool vx_x_layout_ok(uint32_t k, uint32_t ldx, uint32_t xbs, uint32_t batch) {
    if ((ldx & 3u) || (xbs & 3u) || xbs < 32u) return false;
    if (batch <= 1u) return true;  // one row: any row stride
    return xbs == 32u ? ldx >= k : (ldx >= 32u && (uint64_t)xbs >= (uint64_t)batch * ldx);
}

hipError_t vx_launch_bnorm(float* h, uint32_t ldh, const float* parts, uint32_t nparts, uint64_t pstride, const float* g,
                           uint32_t k, float eps, uint16_t* x16, uint32_t ldx, uint32_t xbs, uint32_t batch,
                           uint64_t mask, hipStream_t st) {
    // float4 rows: k, ldh and pstride multiples of 4 (16-byte h and parts rows, 8-byte x16 runs)
    if (k == 0 || (k & 3u) || (ldh & 3u) || ldh < k || !vx_x_layout_ok(k, ldx, xbs, batch)) return hipErrorInvalidValue;
    if (parts && (nparts == 0 || nparts > kBNormMaxParts || (pstride & 3u))) return hipErrorInvalidValue;
    if (!parts) nparts = 0;
    const dim3 grid(batch), block(1024);
    if (k <= 4096u)
        hipLaunchKernelGGL((vx_bnorm_kernel<1>), grid, block, 0, st, h, ldh, parts, nparts, pstride, g, k, eps, x16, ldx,
                           xbs, mask);
    else if (k <= 8192u)
        hipLaunchKernelGGL((vx_bnorm_kernel<2>), grid, block, 0, st, h, ldh, parts, nparts, pstride, g, k, eps, x16, ldx,
                           xbs, mask);
    else  // rows past 8192 would need more than 64 registers of partials per thread
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t vx_launch_bmerge(const float* part_o, const float* part_ml, uint32_t hq, uint32_t d, uint32_t splits,
                            uint16_t* x16, uint32_t ldx, uint32_t xbs, uint32_t batch, uint64_t mask, hipStream_t st) {
    if (splits == 0 || splits > 64 || !vx_x_layout_ok(hq * d, ldx, xbs, batch)) return hipErrorInvalidValue;
    if (d == 64)
        hipLaunchKernelGGL((vx_bmerge_kernel<64>), dim3(hq, batch), dim3(64), 0, st, part_o, part_ml, hq, splits, x16,
                           ldx, xbs, mask);
    else if (d == 128)
        hipLaunchKernelGGL((vx_bmerge_kernel<128>), dim3(hq, batch), dim3(128), 0, st, part_o, part_ml, hq, splits,
                           x16, ldx, xbs, mask);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t vx_launch_bfinalize(const float* cand_v, const uint32_t* cand_i, uint32_t n, VeloxDecodeState* states,
                               uint32_t* rings, const uint32_t* prompts, const uint32_t* plens, uint32_t prompt_stride,
                               uint32_t batch, uint64_t mask, hipStream_t st) {
    hipLaunchKernelGGL(vx_bfinalize_kernel, dim3(batch), dim3(256), 0, st, cand_v, cand_i, n, states, rings, prompts,
                       plens, prompt_stride, mask);
    return hipGetLastError();
}
