// vx_batch.hip -- batched decode of up to 32 independent sequences on gfx950: the Q4_0 GEMM of
// all sequences' activations against one pass over the weights, on MFMA.
//
// The reference's batched kernels (src/runners/velox_cuda_runner_k2.cu:553-997) keep B <= 8
// register accumulators per lane and dot the dequantized words on the VALU; at B = 32 a decode
// step of Qwen2.5-7B is 452 GFLOP against 7.7 GB of traffic, beyond the VALU rate, so here every
// 16 weight rows x one 32-weight block is one v_mfma_f32_16x16x32_f16:
//   B operand: lane l holds elements 8*(l/16) .. +7 of weight row (l % 16) as exact fp16 (q - 8),
//              one dword of the Q4_0 code word unpacked with v_perm (1024 + q) and v_pk_add -1032;
//   A operand: lane l holds the same elements of sequence (l % 16) from the fp16 activations;
//   result:    lane l holds rows m = 4 (l / 16) + i, i < 4, of weight row (l % 16), scaled by the
//              block's fp16 scale in fp32 (4 FMAs), so products are exact and sums fp32, as in the
//              single-sequence GEMV.
// Weights stay in the tiled decode layout (no second copy); a workgroup of 4 waves owns 64 weight
// rows (the S layout tiles of R = 64 / S rows each) and stages, per item of S blocks, the tiles'
// code words, their scales and the activation chunk of every sequence in LDS.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "vx_common.h"

namespace {

typedef _Float16 vx_h8 __attribute__((ext_vector_type(8)));
typedef _Float16 vx_bh2 __attribute__((ext_vector_type(2)));
typedef float vx_f4 __attribute__((ext_vector_type(4)));

constexpr int kBWaves = 4, kBThreads = 64 * kBWaves;

__device__ __forceinline__ float vx_bh2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)h)); }

__device__ __forceinline__ bool vx_bbetter(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

// One code dword (8 weights, byte j: element j low nibble, element j + 4 high nibble) -> the 8
// values q - 8 as fp16, in element order.
__device__ __forceinline__ vx_h8 vx_unpack8(uint32_t q) {
    const uint32_t lo = q & 0x0F0F0F0Fu, hi = (q >> 4) & 0x0F0F0F0Fu, c64 = 0x64646464u;
    const vx_bh2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const vx_bh2 p0 = __builtin_bit_cast(vx_bh2, __builtin_amdgcn_perm(c64, lo, 0x04010400u)) + off;
    const vx_bh2 p1 = __builtin_bit_cast(vx_bh2, __builtin_amdgcn_perm(c64, lo, 0x04030402u)) + off;
    const vx_bh2 p2 = __builtin_bit_cast(vx_bh2, __builtin_amdgcn_perm(c64, hi, 0x04010400u)) + off;
    const vx_bh2 p3 = __builtin_bit_cast(vx_bh2, __builtin_amdgcn_perm(c64, hi, 0x04030402u)) + off;
    vx_h8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

}  // namespace

template <int S, int MT>
constexpr size_t vx_bgemm_lds() {
    return (size_t)S * 64 * 16 + (size_t)S * 64 * 2 + (size_t)MT * 16 * S * 32 * 2;
}

template <int S, int EPI, int MT>
__global__ __launch_bounds__(kBThreads) void vx_bgemm_q4_kernel(VxBGemmArgs a) {
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr int R = 64 / S, TPW = S, XC = S * 4;  // rows per tile, tiles per workgroup, x chunks per row
    extern __shared__ __align__(16) unsigned char vx_smem[];
    uint4* c_s = (uint4*)vx_smem;                     // [TPW][64] code words of this item
    uint16_t* s_s = (uint16_t*)(c_s + TPW * 64);      // [TPW][64] their scales
    uint4* x_s = (uint4*)(s_s + TPW * 64);            // [MT * 16][XC] fp16 activations (8 per chunk)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t t0 = blockIdx.x * (uint32_t)TPW, n_iter = a.n_iter;
    const int nl = 16 * wave + (lane & 15), g = lane >> 4;  // this lane's weight row in the workgroup
    const int tl = nl / R, r = nl % R;
    vx_f4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = vx_f4{0.f, 0.f, 0.f, 0.f};

    for (uint32_t it = 0; it < n_iter; ++it) {
        __syncthreads();  // the previous item's operands are consumed
        for (int i = tid; i < TPW * 64; i += kBThreads) {
            const uint32_t t = t0 + (uint32_t)(i >> 6);
            const size_t slot = ((size_t)t * n_iter + it) * 64u + (uint32_t)(i & 63);
            c_s[i] = t < a.n_tiles ? a.codes[slot] : make_uint4(0u, 0u, 0u, 0u);
            s_s[i] = t < a.n_tiles ? a.scales[slot] : (uint16_t)0;
        }
        for (int i = tid; i < MT * 16 * XC; i += kBThreads) {
            const int m = i / XC, ch = i % XC;
            const uint32_t e = it * (uint32_t)(S * 32) + (uint32_t)ch * 8u;
            x_s[i] = ((uint32_t)m < a.batch && e < a.k) ? *(const uint4*)(a.x16 + (size_t)m * a.ldx + e)
                                                        : make_uint4(0u, 0u, 0u, 0u);
        }
        __syncthreads();
#pragma unroll 4
        for (int j = 0; j < S; ++j) {
            const int wi = tl * 64 + r * S + j;  // layout lane (r, block j) of tile tl
            const uint32_t q = ((const uint32_t*)(c_s + wi))[g];
            const float d = vx_bh2f(s_s[wi]);
            const vx_h8 bw = vx_unpack8(q);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const vx_h8 ax = __builtin_bit_cast(vx_h8, x_s[(mt * 16 + (lane & 15)) * XC + j * 4 + g]);
                const vx_f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bw, vx_f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                acc[mt] += d * c;
            }
        }
    }

    // ---- epilogues: lane holds acc[mt][i] for sequence m = 16 mt + 4 g + i of weight row nl ----
    const uint32_t t = t0 + (uint32_t)tl;
    if constexpr (EPI == VX_EPI_SWIGLU) {
        // paired tiles: the first R/2 rows are gate rows, the last R/2 the matching up rows, so the
        // partner of lane l is lane l ^ (R/2), inside its 16-lane group
        const uint32_t j = t * (uint32_t)(R / 2) + (uint32_t)(r % (R / 2));
        const bool ok = t < a.n_tiles && j < a.n;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float up = __shfl_xor(acc[mt][i], R / 2);
                const uint32_t m = (uint32_t)(16 * mt + 4 * g + i);
                if (r < R / 2 && ok && m < a.batch) {
                    const float gt = acc[mt][i];
                    a.out16[(size_t)m * a.ldo + j] = __half_as_ushort(__float2half((gt / (1.0f + expf(-gt))) * up));
                }
            }
    } else {
        const uint32_t n = t * (uint32_t)R + (uint32_t)r;
        const bool ok = t < a.n_tiles && n < a.n;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = (uint32_t)(16 * mt + 4 * g + i);
                if (!ok || m >= a.batch) continue;
                float* yp = a.y + (size_t)m * a.ldy + n;
                if constexpr (EPI == VX_EPI_STORE) *yp = a.bias ? acc[mt][i] + a.bias[n] : acc[mt][i];
                else if constexpr (EPI == VX_EPI_RESID) *yp += acc[mt][i];
                else *yp = acc[mt][i];
            }
        if constexpr (EPI == VX_EPI_ARGMAX) {
            // per sequence: the best (value, lowest index) of this workgroup's 64 rows
            __shared__ float s_v[kBWaves][MT * 16];
            __shared__ uint32_t s_i[kBWaves][MT * 16];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float bv = ok ? acc[mt][i] : -INFINITY;
                    uint32_t bi = ok ? n : 0xFFFFFFFFu;
#pragma unroll
                    for (int off = 1; off < 16; off <<= 1) {
                        const float ov = __shfl_xor(bv, off);
                        const uint32_t oi = __shfl_xor(bi, off);
                        if (vx_bbetter(ov, oi, bv, bi)) { bv = ov; bi = oi; }
                    }
                    if ((lane & 15) == 0) {
                        s_v[wave][16 * mt + 4 * g + i] = bv;
                        s_i[wave][16 * mt + 4 * g + i] = bi;
                    }
                }
            __syncthreads();
            if (tid < MT * 16 && (uint32_t)tid < a.batch) {
                float bv = s_v[0][tid];
                uint32_t bi = s_i[0][tid];
                for (int w = 1; w < kBWaves; ++w)
                    if (vx_bbetter(s_v[w][tid], s_i[w][tid], bv, bi)) { bv = s_v[w][tid]; bi = s_i[w][tid]; }
                a.cand_v[(size_t)tid * gridDim.x + blockIdx.x] = bv;
                a.cand_i[(size_t)tid * gridDim.x + blockIdx.x] = bi;
            }
        }
    }
}

namespace {

template <int S, int EPI, int MT>
hipError_t vx_bgemm_launch_t(const VxBGemmArgs& a, hipStream_t st) {
    constexpr size_t lds = vx_bgemm_lds<S, MT>();
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)vx_bgemm_q4_kernel<S, EPI, MT>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        attr_set = true;
    }
    hipLaunchKernelGGL((vx_bgemm_q4_kernel<S, EPI, MT>), dim3(vx_bgemm_grid(a.n_tiles, S)), dim3(kBThreads), lds, st, a);
    return hipGetLastError();
}

template <int EPI, int MT>
hipError_t vx_bgemm_dispatch_s(uint32_t s, const VxBGemmArgs& a, hipStream_t st) {
    switch (s) {
        case 4: return vx_bgemm_launch_t<4, EPI, MT>(a, st);
        case 8: return vx_bgemm_launch_t<8, EPI, MT>(a, st);
        case 16: return vx_bgemm_launch_t<16, EPI, MT>(a, st);
        case 32: return vx_bgemm_launch_t<32, EPI, MT>(a, st);
        default: return hipErrorInvalidValue;  // S = 64 (one row per tile) has no MFMA grouping here
    }
}

template <int EPI>
hipError_t vx_bgemm_dispatch_mt(uint32_t s, const VxBGemmArgs& a, hipStream_t st) {
    if (a.batch == 0 || a.batch > 32) return hipErrorInvalidValue;
    return a.batch <= 16 ? vx_bgemm_dispatch_s<EPI, 1>(s, a, st) : vx_bgemm_dispatch_s<EPI, 2>(s, a, st);
}

}  // namespace

// Workgroups of a batched GEMM: each covers S layout tiles (64 weight rows).
uint32_t vx_bgemm_grid(uint32_t n_tiles, uint32_t s) { return s ? (n_tiles + s - 1u) / s : 1u; }

hipError_t vx_launch_bgemm(const VxMat& m, const VxBGemmArgs& a0, int epi, hipStream_t st) {
    VxBGemmArgs a = a0;
    a.codes = m.codes;
    a.scales = m.scales;
    a.n = m.n;
    a.k = m.k;
    a.n_tiles = m.n_tiles;
    a.n_iter = m.n_iter;
    if (m.k == 0 || (m.k & 31u) || (a.ldx & 7u) || !a.x16) return hipErrorInvalidValue;
    if ((epi == VX_EPI_SWIGLU) != (m.paired != 0)) return hipErrorInvalidValue;
    switch (epi) {
        case VX_EPI_STORE: return vx_bgemm_dispatch_mt<VX_EPI_STORE>(m.s, a, st);
        case VX_EPI_RESID: return vx_bgemm_dispatch_mt<VX_EPI_RESID>(m.s, a, st);
        case VX_EPI_SWIGLU: return vx_bgemm_dispatch_mt<VX_EPI_SWIGLU>(m.s, a, st);
        case VX_EPI_ARGMAX: return vx_bgemm_dispatch_mt<VX_EPI_ARGMAX>(m.s, a, st);
        default: return hipErrorInvalidValue;
    }
}
