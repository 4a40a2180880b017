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
typedef uint32_t vx_bu4 __attribute__((ext_vector_type(4)));  // a plain vector (HIP's uint4 is a union
                                                               // struct that arrays keep on the stack)

constexpr int kBWaves = 4, kBThreads = 64 * kBWaves;
constexpr uint32_t kBNormMaxParts = 8;  // K splits of a RESID GEMM that one batched RMSNorm folds in

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
    return (size_t)S * 64 * 16 + (size_t)S * 64 * 2 + (size_t)MT * 16 * (S * 4 + 1) * 16;
}

template <int S, int EPI, int MT>
__global__ __launch_bounds__(kBThreads) void vx_bgemm_q4_kernel(VxBGemmArgs a) {
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr int R = 64 / S, TPW = S, XC = S * 4;  // rows per tile, tiles per workgroup, x chunks per row
    constexpr int XP = XC + 1;                      // padded activation row: rows 4 banks apart
    extern __shared__ __align__(16) unsigned char vx_smem[];
    // code words and scales of this item, transposed to [wave][block j][row 0..15]: the 16 lanes
    // that read one dword column of a block read 16 consecutive words (no bank conflicts)
    vx_bu4* c_s = (vx_bu4*)vx_smem;
    uint16_t* s_s = (uint16_t*)(c_s + TPW * 64);
    vx_bu4* x_s = (vx_bu4*)(s_s + TPW * 64);          // [MT * 16][XP] fp16 activations (8 per chunk)
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t t0 = blockIdx.x * (uint32_t)TPW, n_iter = a.n_iter;
    // this workgroup's items: all of them, or the blockIdx.y-th of gridDim.y equal K ranges
    const uint32_t it_begin = blockIdx.y * n_iter / gridDim.y, it_end = (blockIdx.y + 1u) * n_iter / gridDim.y;
    const int nl = 16 * wave + (lane & 15), g = lane >> 4;  // this lane's weight row in the workgroup
    const int tl = nl / R, r = nl % R;
    vx_f4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = vx_f4{0.f, 0.f, 0.f, 0.f};

    // Operands of one item in registers: the next item's loads are issued before the current one
    // is computed from LDS, so HBM latency overlaps the MFMA work. Loads are unconditional (tiles
    // past the matrix re-read its last tile, sequences past the batch the last sequence, elements
    // past K the last chunk); those rows and columns never reach an output, and padded blocks have
    // zero scales.
    constexpr int NC = S / 4, NX = MT * S / 4;  // 16-byte code words and activation chunks per thread
    vx_bu4 cr[NC], xr[NX];
    uint16_t sr[NC];
    const uint32_t t_last = a.n_tiles - 1u, m_last = a.batch - 1u, e_last = a.k - 8u;
    // loads of item `it` into the prefetch registers (a macro keeps the arrays in registers: the
    // same loop behind a lambda called from two places was left on the stack)
#define VX_BGEMM_LOAD(it_)                                                                          \
    do {                                                                                            \
        _Pragma("unroll") for (int u = 0; u < NC; ++u) {                                            \
            const int i = tid + u * kBThreads;                                                      \
            const uint32_t t = min(t0 + (uint32_t)(i >> 6), t_last);                                \
            const size_t slot = ((size_t)t * n_iter + (it_)) * 64u + (uint32_t)(i & 63);            \
            cr[u] = ((const vx_bu4*)a.codes)[slot];                                                 \
            sr[u] = a.scales[slot];                                                                 \
        }                                                                                           \
        _Pragma("unroll") for (int u = 0; u < NX; ++u) {                                            \
            const int i = tid + u * kBThreads;                                                      \
            const uint32_t m = min((uint32_t)(i / XC), m_last);                                     \
            const uint32_t e = min((it_) * (uint32_t)(S * 32) + (uint32_t)(i % XC) * 8u, e_last);   \
            xr[u] = *(const vx_bu4*)(a.x16 + (size_t)m * a.ldx + (size_t)(e >> 5) * a.xbs + (e & 31u)); \
        }                                                                                           \
    } while (0)
    VX_BGEMM_LOAD(it_begin);
    for (uint32_t it = it_begin; it < it_end; ++it) {
        __syncthreads();  // the previous item's operands are consumed
#pragma unroll
        for (int u = 0; u < NC; ++u) {
            // word i = (tile i / 64, layout lane i % 64 = (row r, block s)) -> (wave, s, row in wave)
            const int i = tid + u * kBThreads;
            const int row = (i >> 6) * R + (i & 63) / S, blk = (i & 63) % S;
            const int o = ((row >> 4) * S + blk) * 16 + (row & 15);
            c_s[o] = cr[u];
            s_s[o] = sr[u];
        }
#pragma unroll
        for (int u = 0; u < NX; ++u) {
            const int i = tid + u * kBThreads;
            x_s[(i / XC) * XP + i % XC] = xr[u];
        }
        __syncthreads();
        if (it + 1u < it_end) VX_BGEMM_LOAD(it + 1u);
#pragma unroll 4
        for (int j = 0; j < S; ++j) {
            const int wi = (wave * S + j) * 16 + (lane & 15);  // this lane's row, block j
            const uint32_t q = ((const uint32_t*)(c_s + wi))[g];
            const float d = vx_bh2f(s_s[wi]);
            const vx_h8 bw = vx_unpack8(q);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const vx_h8 ax = __builtin_bit_cast(vx_h8, x_s[(mt * 16 + (lane & 15)) * XP + j * 4 + g]);
                const vx_f4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(ax, bw, vx_f4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                acc[mt] += d * c;
            }
        }
    }
#undef VX_BGEMM_LOAD

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
                    a.out16[(size_t)m * a.ldo + (size_t)(j >> 5) * a.obs + (j & 31u)] =
                        __half_as_ushort(__float2half((gt / (1.0f + expf(-gt))) * up));
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
                else if constexpr (EPI == VX_EPI_RESID) {
                    if (gridDim.y > 1u) a.part[blockIdx.y * a.pstride + (size_t)m * a.ldy + n] = acc[mt][i];
                    else *yp += acc[mt][i];
                } else *yp = acc[mt][i];
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
    hipLaunchKernelGGL((vx_bgemm_q4_kernel<S, EPI, MT>), dim3(vx_bgemm_grid(a.n_tiles, S), a.ksplit > 1u ? a.ksplit : 1u),
                       dim3(kBThreads), lds, st, a);
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
    if (m.k == 0 || (m.k & 31u) || (a.ldx & 7u) || (a.xbs & 7u) || !a.x16 || !vx_x_layout_ok(m.k, a.ldx, a.xbs, a.batch))
        return hipErrorInvalidValue;
    if (epi == VX_EPI_SWIGLU && !vx_x_layout_ok(m.n, a.ldo, a.obs, a.batch)) return hipErrorInvalidValue;
    if ((epi == VX_EPI_SWIGLU) != (m.paired != 0)) return hipErrorInvalidValue;
    if (a.ksplit > 1u && (epi != VX_EPI_RESID || !a.part || a.ksplit > m.n_iter || a.ksplit > kBNormMaxParts ||
                          a.pstride < (uint64_t)a.batch * a.ldy))
        return hipErrorInvalidValue;
    switch (epi) {
        case VX_EPI_STORE: return vx_bgemm_dispatch_mt<VX_EPI_STORE>(m.s, a, st);
        case VX_EPI_RESID: return vx_bgemm_dispatch_mt<VX_EPI_RESID>(m.s, a, st);
        case VX_EPI_SWIGLU: return vx_bgemm_dispatch_mt<VX_EPI_SWIGLU>(m.s, a, st);
        case VX_EPI_ARGMAX: return vx_bgemm_dispatch_mt<VX_EPI_ARGMAX>(m.s, a, st);
        default: return hipErrorInvalidValue;
    }
}

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
        // every partial of every element loaded before the first add (split index clamped; the
        // adds past nparts are skipped)
        float4 p[kBNormMaxParts][NV];
#pragma unroll
        for (uint32_t s = 0; s < kBNormMaxParts; ++s)
#pragma unroll
            for (int j = 0; j < NV; ++j) {
                const uint32_t i = min(threadIdx.x + 1024u * j, k4 - 1u);
                p[s][j] = ((const float4*)(parts + min(s, nparts - 1u) * pstride + (size_t)b * ldh))[i];
            }
#pragma unroll
        for (uint32_t s = 0; s < kBNormMaxParts; ++s)
            if (s < nparts)
#pragma unroll
                for (int j = 0; j < NV; ++j) {
                    v[j].x += p[s][j].x;
                    v[j].y += p[s][j].y;
                    v[j].z += p[s][j].z;
                    v[j].w += p[s][j].w;
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
