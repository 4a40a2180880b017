// vx_gemv_f.hip -- the decode step's GEMV over unquantized weights: the reference's quant_mode 0
// (fp32) and 1 (fp16) rows, stored row-major [rows][k] as the reference's weight arena holds them
// (src/codegen.rs:1024-1028; its emitted velox_cuda_matmul_vec_kernel, src/codegen.rs:1154, and
// velox_cuda_matmul_vec_kernel_f16 / velox_warp_dot_f16, src/codegen.rs:2267-2311, 2412-2420).
// Benchmark configuration 1, the fp32 SmolLM, runs on this kernel.
//
// Same contract as the Q4_0 GEMV (vx_launch_gemv picks this kernel from the matrix format): the
// input (or the LSE merge of split attention partials) is RMSNorm'd into LDS as fp32; each wave
// takes tiles of 4 logical rows (a SwiGLU tile: 4 gate rows and the 4 matching up rows, stored
// as n gate rows followed by n up rows), its lanes stride over the row in 16-byte words (4 fp32
// or 8 fp16 weights), fp32 FMAs, then a 64-lane sum. Epilogues: store (+bias), residual add,
// SwiGLU, or the per-workgroup (max, index) candidate of the LM head.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "vx_common.h"

namespace {

constexpr int kFWaves = 8, kFThreads = 64 * kFWaves, kFRows = 4;

typedef uint32_t vf_u4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float vf_wave_sum(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
    return v;
}

__device__ __forceinline__ bool vf_better(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

// 16 bytes of weights times the matching activations in LDS, accumulated in fp32
template <typename T>
__device__ __forceinline__ float vf_dot16(const vf_u4& w, const float* x, float acc);

template <>
__device__ __forceinline__ float vf_dot16<float>(const vf_u4& w, const float* x, float acc) {
    const float4 xv = *(const float4*)x;
    acc = fmaf(__uint_as_float(w.x), xv.x, acc);
    acc = fmaf(__uint_as_float(w.y), xv.y, acc);
    acc = fmaf(__uint_as_float(w.z), xv.z, acc);
    return fmaf(__uint_as_float(w.w), xv.w, acc);
}

template <>
__device__ __forceinline__ float vf_dot16<__half>(const vf_u4& w, const float* x, float acc) {
    const float4 x0 = *(const float4*)x, x1 = *(const float4*)(x + 4);
    const uint32_t d[4] = {w.x, w.y, w.z, w.w};
    const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        acc = fmaf(__half2float(__ushort_as_half((unsigned short)(d[i] & 0xFFFFu))), xv[2 * i], acc);
        acc = fmaf(__half2float(__ushort_as_half((unsigned short)(d[i] >> 16))), xv[2 * i + 1], acc);
    }
    return acc;
}

template <typename T, int EPI, bool NORM, int SPL>
__global__ __launch_bounds__(kFThreads) void vx_gemv_f_kernel(VxMat m, VxGemvArgs a) {
    extern __shared__ __align__(16) float vf_smem[];
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr uint32_t E = 16u / sizeof(T);     // weights per 16-byte word
    constexpr int PR = EPI == VX_EPI_SWIGLU ? 2 : 1;
    const uint32_t K = m.k;
    float* xs = vf_smem;
    float* red = vf_smem + K;  // [kFWaves] partial sums, then the argmax candidates
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // ---- x (or the merged attention partials) into LDS, with its sum of squares ----
    float ss = 0.0f;
    for (uint32_t i = (uint32_t)tid; i < K / 4u; i += (uint32_t)kFThreads) {
        float4 v;
        if constexpr (SPL == 0) {
            v = ((const float4*)a.x)[i];
        } else {
            // LSE merge of the splits (m, l in the log2 domain; an empty split has m = -inf, l = 0),
            // the merge of tests/empirical_challenge_phase2/test2_split_k_flashdecoding_parity.cu:23-125
            const uint32_t k = 4u * i, h = k / a.att_d, e0 = k - h * a.att_d;
            float M = -INFINITY;
#pragma unroll
            for (int sp = 0; sp < SPL; ++sp) M = fmaxf(M, a.part_ml[((size_t)h * SPL + sp) * 2u]);
            float L = 0.0f, wt[SPL];
#pragma unroll
            for (int sp = 0; sp < SPL; ++sp) {
                const float2 ml = *(const float2*)(a.part_ml + ((size_t)h * SPL + sp) * 2u);
                wt[sp] = ml.x == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(ml.x - M);
                L += wt[sp] * ml.y;
            }
            const float invl = L > 0.0f ? 1.0f / L : 0.0f;
            v = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
            for (int sp = 0; sp < SPL; ++sp) {
                const float ws = wt[sp] * invl;
                const float4 o = *(const float4*)(a.part_o + ((size_t)h * SPL + sp) * a.att_d + e0);
                v.x += ws * o.x; v.y += ws * o.y; v.z += ws * o.z; v.w += ws * o.w;
            }
        }
        ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
        ((float4*)xs)[i] = v;
    }
    if constexpr (NORM) {
        ss = vf_wave_sum(ss);
        if (lane == 0) red[wave] = ss;
        __syncthreads();
        float tot = 0.0f;
#pragma unroll
        for (int v = 0; v < kFWaves; ++v) tot += red[v];
        const float inv = 1.0f / sqrtf(tot / (float)K + a.eps);  // src/runtime.rs:588-601
        for (uint32_t i = (uint32_t)tid; i < K / 4u; i += (uint32_t)kFThreads) {
            const float4 v = ((float4*)xs)[i], g = ((const float4*)a.gain)[i];
            ((float4*)xs)[i] = make_float4((v.x * inv) * g.x, (v.y * inv) * g.y, (v.z * inv) * g.z, (v.w * inv) * g.w);
        }
    }
    __syncthreads();

    // ---- tiles of kFRows logical rows: workgroup b owns a contiguous block, dealt to its waves ----
    const uint32_t b0 = (uint32_t)(((uint64_t)blockIdx.x * m.n_tiles) / gridDim.x);
    const uint32_t b1 = (uint32_t)(((uint64_t)(blockIdx.x + 1u) * m.n_tiles) / gridDim.x);
    const uint32_t nw = K / E;  // 16-byte words per row
    const uint8_t* wbase = (const uint8_t*)m.codes;
    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    for (uint32_t t = b0 + (uint32_t)wave; t < b1; t += (uint32_t)kFWaves) {
        float acc[kFRows][PR];
        const vf_u4* rp[kFRows][PR];
#pragma unroll
        for (int r = 0; r < kFRows; ++r) {
            const uint32_t j = min(t * kFRows + (uint32_t)r, m.n - 1u);  // past the matrix: never stored
#pragma unroll
            for (int p = 0; p < PR; ++p) {
                acc[r][p] = 0.0f;
                rp[r][p] = (const vf_u4*)(wbase + ((size_t)(p ? m.n + j : j) * K) * sizeof(T));
            }
        }
        for (uint32_t c = (uint32_t)lane; c < nw; c += 64u) {
            vf_u4 w[kFRows][PR];
#pragma unroll
            for (int r = 0; r < kFRows; ++r)
#pragma unroll
                for (int p = 0; p < PR; ++p) w[r][p] = __builtin_nontemporal_load(rp[r][p] + c);
#pragma unroll
            for (int r = 0; r < kFRows; ++r)
#pragma unroll
                for (int p = 0; p < PR; ++p) acc[r][p] = vf_dot16<T>(w[r][p], xs + c * E, acc[r][p]);
        }
#pragma unroll
        for (int r = 0; r < kFRows; ++r) {
#pragma unroll
            for (int p = 0; p < PR; ++p) acc[r][p] = vf_wave_sum(acc[r][p]);
            const uint32_t j = t * kFRows + (uint32_t)r;
            if (lane != 0 || j >= m.n) continue;
            if constexpr (EPI == VX_EPI_STORE) {
                a.y[j] = a.bias ? acc[r][0] + a.bias[j] : acc[r][0];
            } else if constexpr (EPI == VX_EPI_RESID) {
                a.y[j] = a.res[j] + acc[r][0];
            } else if constexpr (EPI == VX_EPI_SWIGLU) {
                const float gt = acc[r][0];
                a.y[j] = (gt / (1.0f + expf(-gt))) * acc[r][PR - 1];  // src/runtime.rs:1064-1066
            } else {  // VX_EPI_ARGMAX
                a.y[j] = acc[r][0];
                if (vf_better(acc[r][0], j, best_v, best_i)) { best_v = acc[r][0]; best_i = j; }
            }
        }
    }
    if constexpr (EPI == VX_EPI_ARGMAX) {
        __syncthreads();  // red[] is reused
        if (lane == 0) {
            red[wave] = best_v;
            ((uint32_t*)red)[kFWaves + wave] = best_i;
        }
        __syncthreads();
        if (tid == 0) {
            float bv = red[0];
            uint32_t bi = ((const uint32_t*)red)[kFWaves];
            for (int v = 1; v < kFWaves; ++v)
                if (vf_better(red[v], ((const uint32_t*)red)[kFWaves + v], bv, bi)) {
                    bv = red[v];
                    bi = ((const uint32_t*)red)[kFWaves + v];
                }
            a.cand_v[blockIdx.x] = bv;
            a.cand_i[blockIdx.x] = bi;
        }
    }
}

template <typename T, int EPI, bool NORM, int SPL>
hipError_t vx_gemv_f_launch_t(const VxMat& m, const VxGemvArgs& a, uint32_t wgs, hipStream_t st) {
    const size_t lds = (size_t)m.k * 4u + 2u * kFWaves * 4u;
    // rows wider than 16376 need more than the default 64 KiB of dynamic LDS (up to 128 KiB + 64 B
    // at kVxFloatMaxK, of the 160 KiB a CU has): raised once per instantiation to the widest row
    static bool attr_set = false;
    if (lds > 65536u && !attr_set) {
        if (hipFuncSetAttribute((const void*)vx_gemv_f_kernel<T, EPI, NORM, SPL>,
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)((size_t)kVxFloatMaxK * 4u + 2u * kFWaves * 4u)) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        attr_set = true;
    }
    hipLaunchKernelGGL((vx_gemv_f_kernel<T, EPI, NORM, SPL>), dim3(wgs), dim3(kFThreads), lds, st, m, a);
    return hipGetLastError();
}

template <typename T, int EPI>
hipError_t vx_gemv_f_dispatch(const VxMat& m, const VxGemvArgs& a, uint32_t wgs, hipStream_t st) {
    if constexpr (EPI == VX_EPI_RESID) {
        if (a.gain) return hipErrorInvalidValue;  // the residual epilogue takes raw activations
        if (!a.part_o) return vx_gemv_f_launch_t<T, EPI, false, 0>(m, a, wgs, st);
        if (!a.part_ml || a.att_d == 0 || (a.att_d & 3u) || m.k % a.att_d) return hipErrorInvalidValue;
        switch (a.att_splits) {
            case 1: return vx_gemv_f_launch_t<T, EPI, false, 1>(m, a, wgs, st);
            case 2: return vx_gemv_f_launch_t<T, EPI, false, 2>(m, a, wgs, st);
            case 4: return vx_gemv_f_launch_t<T, EPI, false, 4>(m, a, wgs, st);
            case 8: return vx_gemv_f_launch_t<T, EPI, false, 8>(m, a, wgs, st);
            default: return hipErrorInvalidValue;
        }
    } else {
        if (a.part_o) return hipErrorInvalidValue;
        return a.gain ? vx_gemv_f_launch_t<T, EPI, true, 0>(m, a, wgs, st)
                      : vx_gemv_f_launch_t<T, EPI, false, 0>(m, a, wgs, st);
    }
}

template <typename T>
hipError_t vx_gemv_f_epi(const VxMat& m, const VxGemvArgs& a, int epi, uint32_t wgs, hipStream_t st) {
    switch (epi) {
        case VX_EPI_STORE: return vx_gemv_f_dispatch<T, VX_EPI_STORE>(m, a, wgs, st);
        case VX_EPI_RESID: return vx_gemv_f_dispatch<T, VX_EPI_RESID>(m, a, wgs, st);
        case VX_EPI_SWIGLU: return vx_gemv_f_dispatch<T, VX_EPI_SWIGLU>(m, a, wgs, st);
        case VX_EPI_ARGMAX: return vx_gemv_f_dispatch<T, VX_EPI_ARGMAX>(m, a, wgs, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

hipError_t vx_launch_gemv_f(const VxMat& m, const VxGemvArgs& a, int epi, uint32_t wgs, hipStream_t st) {
    if (m.k == 0 || (m.k & 7u) || m.k > kVxFloatMaxK || m.n == 0) return hipErrorInvalidValue;
    if ((epi == VX_EPI_SWIGLU) != (m.paired != 0)) return hipErrorInvalidValue;
    if (epi == VX_EPI_ARGMAX && (!a.cand_v || !a.cand_i)) return hipErrorInvalidValue;
    if (m.fmt == VX_FMT_F32) return vx_gemv_f_epi<float>(m, a, epi, wgs, st);
    if (m.fmt == VX_FMT_F16) return vx_gemv_f_epi<__half>(m, a, epi, wgs, st);
    return hipErrorInvalidValue;
}
