// vx_mgemm.hip -- the Q4_0 GEMM of the batched decode and prefill steps on gfx950 (MFMA), over a
// second copy of every matrix in the MFMA operand layout ("M-layout").
//
// M-layout of an [n][k] Q4_0 matrix: 16-row tiles (paired gate/up matrices: gate tile u at 2u,
// the matching up tile at 2u + 1) and groups of four 32-element blocks (k padded to 128 with
// zero-scale blocks). Per (tile, group) 64 words of 16 bytes: lane l holds, for row 16 t + l % 16,
// dword g = l / 16 -- elements 8g .. 8g+7, element e at bit 16 (e & 1) + 4 (e >> 1) -- of each of
// the blocks 4j .. 4j+3, i.e. the B operand of one v_mfma_f32_16x16x32_f16 per block. Scales: fp16
// [tile][group][row][4 blocks]. One 16-byte load per lane per group feeds four MFMAs, straight from
// HBM into registers: no LDS staging and no barriers (the tiled decode layout, made for the
// GEMV's per-row lane streams, needed an LDS transposition per item and held one workgroup per CU).
//
// Per wave: NT tiles x MT groups of 16 activation rows over a range of groups (split-K across grid
// rows). Block b of group j: c = mfma(x[m][32b + 8g .. +7], unpack(dword), 0); acc += d_b * c. The
// products are exact (fp16 activations times integers -8..7), the block scale is applied in fp32
// and the sums are fp32, as in the single-sequence GEMV and the tiled batched GEMM.
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <stdint.h>

#include "vx_common.h"

namespace {

typedef _Float16 vx_mh8 __attribute__((ext_vector_type(8)));
typedef _Float16 vx_mh2 __attribute__((ext_vector_type(2)));
typedef float vx_mf4 __attribute__((ext_vector_type(4)));
typedef uint32_t vx_mu4 __attribute__((ext_vector_type(4)));
typedef uint32_t vx_mu2 __attribute__((ext_vector_type(2)));

constexpr int kMWaves = 4, kMThreads = 64 * kMWaves;

__device__ __forceinline__ float vx_mh2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)h)); }

__device__ __forceinline__ bool vx_mbetter(float v, uint32_t i, float bv, uint32_t bi) {
    return v > bv || (v == bv && i < bi);
}

// One M-layout code dword -> the 8 values q - 8 as fp16 in element order. Element e sits at bit
// 16 (e & 1) + 4 (e >> 1), so each half of the dword holds one element of each pair: under the
// 0x6400 exponent (1024 + q in the mantissa), masks 0x000F000F / 0x00F000F0 of q and of q >> 8 give
// the pairs (e0, e1), (e2, e3) scaled by 16, (e4, e5), (e6, e7) scaled by 16; -1032, or x / 16 - 72
// for the scaled ones, leaves q - 8 exactly (9 instructions per dword).
// (a & m) | e in one VOP3 instruction: GFX9 reads at most one scalar or constant operand per VALU
// instruction, so the compiler splits the two-constant form into v_and + v_or; here the mask comes
// from an SGPR and the exponent pattern from a VGPR.
__device__ __forceinline__ uint32_t vx_and_or(uint32_t a, uint32_t m, uint32_t e) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "s"(m), "v"(e));
    return r;
}

__device__ __forceinline__ vx_mh8 vx_munpack8(uint32_t q, uint32_t e) {
    const uint32_t q8 = q >> 8;
    const vx_mh2 off = {(_Float16)-1032.0f, (_Float16)-1032.0f};
    const vx_mh2 sc = {(_Float16)0.0625f, (_Float16)0.0625f}, off16 = {(_Float16)-72.0f, (_Float16)-72.0f};
    const vx_mh2 p0 = __builtin_bit_cast(vx_mh2, vx_and_or(q, 0x000F000Fu, e)) + off;
    const vx_mh2 p1 = __builtin_bit_cast(vx_mh2, vx_and_or(q, 0x00F000F0u, e)) * sc + off16;
    const vx_mh2 p2 = __builtin_bit_cast(vx_mh2, vx_and_or(q8, 0x000F000Fu, e)) + off;
    const vx_mh2 p3 = __builtin_bit_cast(vx_mh2, vx_and_or(q8, 0x00F000F0u, e)) * sc + off16;
    vx_mh8 r;
    r[0] = p0[0]; r[1] = p0[1]; r[2] = p1[0]; r[3] = p1[1];
    r[4] = p2[0]; r[5] = p2[1]; r[6] = p3[0]; r[7] = p3[1];
    return r;
}

// Tiled-layout dword (element e at bit 8 (e & 3) + 4 (e >> 2)) -> M-layout dword order.
__device__ __forceinline__ uint32_t vx_mreorder(uint32_t t) {
    uint32_t o = 0;
#pragma unroll
    for (int e = 0; e < 8; ++e) o |= ((t >> (8 * (e & 3) + 4 * (e >> 2))) & 15u) << (16 * (e & 1) + 4 * (e >> 1));
    return o;
}

// ---- M-layout copy of a tiled matrix: one thread per (tile, group, lane) ----
__global__ __launch_bounds__(256) void vx_mlayout_kernel(VxMat src, VxMMat dst) {
    const size_t idx = (size_t)blockIdx.x * 256u + threadIdx.x;
    const size_t total = (size_t)dst.n_tiles * dst.n_grp * 64u;
    if (idx >= total) return;
    const uint32_t lane = (uint32_t)(idx & 63u), j = (uint32_t)((idx >> 6) % dst.n_grp);
    const uint32_t t = (uint32_t)((idx >> 6) / dst.n_grp);
    const uint32_t rho = lane & 15u, g = lane >> 4;
    uint32_t row, part = 0;
    if (dst.paired) {
        row = 16u * (t >> 1) + rho;
        part = t & 1u;
    } else {
        row = 16u * t + rho;
    }
    const uint32_t nb = src.k >> 5, R = 64u / src.s;
    uint32_t out[4];
    uint16_t sc[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const uint32_t blk = 4u * j + (uint32_t)b;
        out[b] = 0u;
        sc[b] = 0u;
        if (row < dst.n && blk < nb) {
            uint32_t phys = row;
            if (src.paired) {
                const uint32_t half = R / 2u;
                phys = (row / half) * (2u * half) + part * half + (row % half);
            }
            const size_t off = ((size_t)(phys / R) * src.n_iter + blk / src.s) * 64u + (phys % R) * src.s + blk % src.s;
            const uint4 c = src.codes[off];
            out[b] = vx_mreorder(g == 0 ? c.x : g == 1 ? c.y : g == 2 ? c.z : c.w);
            sc[b] = src.scales[off];
        }
    }
    ((uint4*)dst.codes)[idx] = make_uint4(out[0], out[1], out[2], out[3]);
    if (g == 0) {
        uint2 s;
        s.x = (uint32_t)sc[0] | ((uint32_t)sc[1] << 16);
        s.y = (uint32_t)sc[2] | ((uint32_t)sc[3] << 16);
        ((uint2*)dst.scales)[((size_t)t * dst.n_grp + j) * 16u + rho] = s;
    }
}

// ---- split-K partial sums (+ bias) of a STORE GEMM: y[m][n] = sum_s part[s][m][n] + bias[n] ----
// (accumulate: y[m][n] += the sum instead, the RESID form)
__global__ __launch_bounds__(256) void vx_msum_kernel(const float* part, uint32_t nparts, uint64_t pstride,
                                                      const float* bias, float* y, uint32_t n, uint32_t ldy,
                                                      uint32_t accumulate, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    const uint32_t m = blockIdx.y, c = blockIdx.x * 256u + threadIdx.x;
    if (c >= n) return;
    // every part's load in flight at once (clamped to a loaded part), then the sum in split order
    float v[8];
#pragma unroll
    for (uint32_t p = 0; p < 8; ++p) v[p] = part[min(p, nparts - 1u) * pstride + (size_t)m * ldy + c];
    float s = 0.0f;
#pragma unroll
    for (uint32_t p = 0; p < 8; ++p)
        if (p < nparts) s += v[p];
    if (bias) s += bias[c];
    float* yp = y + (size_t)m * ldy + c;
    *yp = accumulate ? *yp + s : s;
}

}  // namespace

// ---- the GEMM ----
// A workgroup's 4 waves share its NT tiles and split its K range: wave w takes groups j0 + w,
// j0 + w + 4, ... (adjacent 1 KiB words of a tile in flight together), then the partial sums meet
// in LDS in wave order and wave 0 runs the epilogue.
template <int EPI, int MT, int NT>
__global__ __launch_bounds__(kMThreads) void vx_mgemm_kernel(VxMMat w, VxBGemmArgs a) {
    if ((a.active_mask & 1ULL) == 0ULL) return;
    static_assert(EPI != VX_EPI_SWIGLU || NT % 2 == 0, "paired tiles come in (gate, up) pairs");
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int row = lane & 15, g = lane >> 4;
    const uint32_t T0 = blockIdx.x * (uint32_t)NT;
    const uint32_t ng = w.n_grp;
    const uint32_t j0 = blockIdx.y * ng / gridDim.y, j1 = (blockIdx.y + 1u) * ng / gridDim.y;

    // tiles past the matrix re-read its last tile, activation rows past the batch the last row,
    // padded blocks (zero scales) the last real block: every load is in bounds and unconditional
    const vx_mu4* cp[NT];
    const vx_mu2* sp[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t t = min(T0 + (uint32_t)nt, w.n_tiles - 1u);
        cp[nt] = (const vx_mu4*)w.codes + (size_t)t * ng * 64u + lane;
        sp[nt] = (const vx_mu2*)w.scales + (size_t)t * ng * 16u + row;
    }
    const uint16_t* xp[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
        xp[mt] = a.x16 + (size_t)min((uint32_t)(16 * mt + row), a.batch - 1u) * a.ldx + 8 * g;
    const uint32_t xbs = a.xbs;
    const uint32_t b_last = (w.k >> 5) - 1u;

    vx_mf4 acc[NT][MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = vx_mf4{0.f, 0.f, 0.f, 0.f};

    const uint32_t jw = j0 + (uint32_t)wave;  // this wave's first group; then every kMWaves-th
    const uint32_t ngw = jw < j1 ? (j1 - jw + (uint32_t)kMWaves - 1u) / (uint32_t)kMWaves : 0u;
    if (ngw) {
        // Two operand sets ping-pong over pairs of groups: each set's loads are issued before the
        // other set's MFMAs, and the loop body has no branch, so the compiler's waits keep the
        // other set in flight (a branch around the MFMAs made it drain every load per iteration).
        const uint32_t jlast = jw + (ngw - 1u) * (uint32_t)kMWaves;
        const uint32_t e6400 = __builtin_amdgcn_readfirstlane(0x64006400u) + (uint32_t)lane * 0u;  // held in a VGPR
        vx_mu4 cwA[NT], cwB[NT];
        vx_mu2 swA[NT], swB[NT];
        vx_mh8 xaA[MT][4], xaB[MT][4];
#define VX_MG_LOAD(cw_, sw_, xa_, jj_)                                                            \
    do {                                                                                          \
        const uint32_t jc_ = min((jj_), jlast);                                                   \
        _Pragma("unroll") for (int nt = 0; nt < NT; ++nt) {                                       \
            cw_[nt] = cp[nt][(size_t)jc_ * 64u];                                                  \
            sw_[nt] = sp[nt][(size_t)jc_ * 16u];                                                  \
        }                                                                                         \
        _Pragma("unroll") for (int b = 0; b < 4; ++b) {                                           \
            const uint32_t blk_ = min(4u * jc_ + (uint32_t)b, b_last);                            \
            _Pragma("unroll") for (int mt = 0; mt < MT; ++mt)                                     \
                xa_[mt][b] = *(const vx_mh8*)(xp[mt] + (size_t)blk_ * xbs);                       \
        }                                                                                         \
    } while (0)
#define VX_MG_COMPUTE(cw_, sw_, xa_)                                                              \
    do {                                                                                          \
        _Pragma("unroll") for (int b = 0; b < 4; ++b)                                             \
        _Pragma("unroll") for (int nt = 0; nt < NT; ++nt) {                                       \
            const vx_mh8 wb = vx_munpack8(cw_[nt][b], e6400);                                     \
            const vx_mh2 sh = __builtin_bit_cast(vx_mh2, b < 2 ? sw_[nt].x : sw_[nt].y);          \
            const float d = (float)sh[b & 1];                                                     \
            _Pragma("unroll") for (int mt = 0; mt < MT; ++mt) {                                   \
                const vx_mf4 c = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa_[mt][b], wb,           \
                                                                        vx_mf4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0); \
                acc[nt][mt] += d * c;                                                             \
            }                                                                                     \
        }                                                                                         \
    } while (0)
        VX_MG_LOAD(cwA, swA, xaA, jw);
        uint32_t i = 0;
        for (; i + 2u <= ngw; i += 2u) {
            const uint32_t jj = jw + i * (uint32_t)kMWaves;
            VX_MG_LOAD(cwB, swB, xaB, jj + (uint32_t)kMWaves);
            VX_MG_COMPUTE(cwA, swA, xaA);
            VX_MG_LOAD(cwA, swA, xaA, jj + 2u * (uint32_t)kMWaves);  // past the last group: clamped
            VX_MG_COMPUTE(cwB, swB, xaB);
        }
        if (i < ngw) VX_MG_COMPUTE(cwA, swA, xaA);  // odd count: set A holds the last group
#undef VX_MG_LOAD
#undef VX_MG_COMPUTE
    }

    // ---- the 4 waves' partial sums, added in wave order (deterministic) ----
    __shared__ vx_mf4 red_s[kMWaves - 1][NT * MT][64];
    if (wave > 0) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) red_s[wave - 1][nt * MT + mt][lane] = acc[nt][mt];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int wv = 0; wv < kMWaves - 1; ++wv)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[nt][mt] += red_s[wv][nt * MT + mt][lane];

    // ---- epilogues (wave 0): lane holds acc[nt][mt][i] for activation row m = 16 mt + 4 g + i of
    // tile T0 + nt's row 16 t + row ----
    if constexpr (EPI == VX_EPI_SWIGLU) {
#pragma unroll
        for (int u = 0; u < NT / 2; ++u) {
            const uint32_t t = T0 + 2u * (uint32_t)u;  // gate tile; t + 1 its up tile
            const uint32_t jrow = 16u * (t >> 1) + (uint32_t)row;
            if (t >= w.n_tiles || jrow >= w.n) continue;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t m = (uint32_t)(16 * mt + 4 * g + i);
                    if (m >= a.batch) continue;
                    const float gt = acc[2 * u][mt][i], up = acc[2 * u + 1][mt][i];
                    a.out16[(size_t)m * a.ldo + (size_t)(jrow >> 5) * a.obs + (jrow & 31u)] =
                        __half_as_ushort(__float2half((gt / (1.0f + expf(-gt))) * up));
                }
        }
    } else if constexpr (EPI == VX_EPI_ARGMAX) {
        // per activation row: logits, then the best (value, lowest index) of this workgroup's rows
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = (uint32_t)(16 * mt + 4 * g + i);
                float bv = -INFINITY;
                uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const uint32_t t = T0 + (uint32_t)nt, n = 16u * t + (uint32_t)row;
                    if (t < w.n_tiles && n < w.n) {
                        if (m < a.batch) a.y[(size_t)m * a.ldy + n] = acc[nt][mt][i];
                        if (vx_mbetter(acc[nt][mt][i], n, bv, bi)) { bv = acc[nt][mt][i]; bi = n; }
                    }
                }
#pragma unroll
                for (int off = 1; off < 16; off <<= 1) {
                    const float ov = __shfl_xor(bv, off);
                    const uint32_t oi = __shfl_xor(bi, off);
                    if (vx_mbetter(ov, oi, bv, bi)) { bv = ov; bi = oi; }
                }
                if (row == 0 && m < a.batch) {
                    a.cand_v[(size_t)m * gridDim.x + blockIdx.x] = bv;
                    a.cand_i[(size_t)m * gridDim.x + blockIdx.x] = bi;
                }
            }
    } else {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const uint32_t t = T0 + (uint32_t)nt, n = 16u * t + (uint32_t)row;
            if (t >= w.n_tiles || n >= w.n) continue;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t m = (uint32_t)(16 * mt + 4 * g + i);
                    if (m >= a.batch) continue;
                    const float v = acc[nt][mt][i];
                    if (gridDim.y > 1u) {
                        a.part[blockIdx.y * a.pstride + (size_t)m * a.ldy + n] = v;
                    } else {
                        float* yp = a.y + (size_t)m * a.ldy + n;
                        if constexpr (EPI == VX_EPI_STORE) *yp = a.bias ? v + a.bias[n] : v;
                        else *yp += v;
                    }
                }
        }
    }
}

// ---- the GEMM for 17-64 activation rows (prefill chunks, 17-32 sequences) ----
// A workgroup owns 8 tiles over all MT row tiles and its grid row's K range, which its two halves
// of 4 waves split (the first half takes the first ceil(n / 2) groups); in each half wave w owns
// tiles 2w, 2w + 1 (a gate/up pair for SWIGLU). Per group of 4 blocks a half stages the group's
// 4 x MT activation tiles (1 KiB each) once in LDS, in the lane order of the MFMA A operand, and
// its 4 waves read them from there for both their tiles: a quarter of the activation loads of the
// kernel above, whose waves split K and each load their own. Stages are double-buffered, one
// barrier per group; the weights are loaded 4 groups ahead and the activations 2 ahead. The two
// halves put two waves on every SIMD, so one wave's VALU work partly overlaps the other's MFMAs
// (with one 4-wave half, Llama's gate/up at 64 rows kept the matrix cores busy a third of its
// 42 us); their sums meet in LDS at the end. The arithmetic is the kernel above's: exact block
// products, the block scale applied in fp32 (4 VALU per MFMA). Splitting each weight d (q - 8)
// exactly into two fp16 MFMA operands instead (hi = fp16(d (q - 8)), lo = the fused residual) needs
// no scale multiply-adds but twice the MFMAs, and measured slower: on gfx950 a wave's MFMAs and
// another wave's VALU instructions on the same SIMD take about the MFMA time plus half the VALU
// time (timed with MFMA-only and VALU-only waves sharing the SIMDs).
constexpr int kPNT = 2, kPTiles = kPNT * kMWaves;  // tiles per wave, per workgroup
constexpr int kPRing = 4;                           // weight register sets: groups loaded ahead

template <int P>
struct vx_ic {
    static constexpr int value = P;
};

template <int EPI, int MT, int KH>
__global__ __launch_bounds__(kMThreads * KH) void vx_pgemm_kernel(VxMMat w, VxBGemmArgs a) {
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr int NT = kPNT, SU = 4 * MT, UPW = SU / kMWaves;  // 1 KiB units per group, per wave
    static_assert(SU % kMWaves == 0, "whole units per wave");
    static_assert(KH == 1 || KH == 2, "one or two K halves");
    static_assert(sizeof(vx_mh8) * 2 * 2 * SU * 64 >= sizeof(vx_mf4) * kMWaves * NT * MT * 64, "reduction fits");
    extern __shared__ __align__(16) unsigned char vx_psmem[];
    vx_mh8(*xs)[2][SU][64] = (vx_mh8(*)[2][SU][64])vx_psmem;  // [half][stage][block * MT + row tile][lane]
    const int tid = threadIdx.x, lane = tid & 63, wv = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int kh = KH == 1 ? 0 : wv / kMWaves, wave = wv % kMWaves;  // K half, wave within the half
    const int row = lane & 15, g = lane >> 4;
    const uint32_t T0 = blockIdx.x * (uint32_t)kPTiles + 2u * (uint32_t)wave;  // this wave's first tile
    const uint32_t r0 = blockIdx.z * (uint32_t)(16 * MT);  // the workgroup's first activation row
    const uint32_t ng = w.n_grp;
    const uint32_t jg0 = blockIdx.y * ng / gridDim.y, j1 = (blockIdx.y + 1u) * ng / gridDim.y;
    const uint32_t jl = j1 - 1u;  // j1 > jg0: the launcher keeps ksplit <= n_grp
    // both halves run ns steps (the barriers are the workgroup's); the second half's last step has
    // no group when the count is odd
    const uint32_t ns = (j1 - jg0 + (uint32_t)KH - 1u) / (uint32_t)KH;
    const uint32_t j0 = jg0 + (uint32_t)kh * ns, nj = kh ? (j1 - jg0) - ns : ns;

    // tiles past the matrix re-read its last tile, rows past the batch the last row, blocks past k
    // (zero codes and scales) the last real block: every load is in bounds and unconditional
    const vx_mu4* cp[NT];
    const vx_mu2* sp[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        const uint32_t t = min(T0 + (uint32_t)nt, w.n_tiles - 1u);
        cp[nt] = (const vx_mu4*)w.codes + (size_t)t * ng * 64u + lane;
        sp[nt] = (const vx_mu2*)w.scales + (size_t)t * ng * 16u + row;
    }
    // the wave stages units wave, wave + 4, ...: unit u is block u / MT, row tile u % MT; lane
    // (row, g) moves elements 8 g .. 8 g + 7 of the tile's row, the A operand it later reads
    const uint16_t* xsrc[UPW];
    uint32_t xblk[UPW];
#pragma unroll
    for (int i = 0; i < UPW; ++i) {
        const int u = wave + kMWaves * i;
        xblk[i] = (uint32_t)(u / MT);
        xsrc[i] = a.x16 + (size_t)min(r0 + (uint32_t)(16 * (u % MT) + row), a.batch - 1u) * a.ldx + 8 * g;
    }
    const uint32_t xbs = a.xbs, b_last = (w.k >> 5) - 1u;

    vx_mf4 acc[NT][MT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) acc[nt][mt] = vx_mf4{0.f, 0.f, 0.f, 0.f};

    const uint32_t e6400 = __builtin_amdgcn_readfirstlane(0x64006400u) + (uint32_t)lane * 0u;  // held in a VGPR
    // Weights: a ring of kPRing register sets, set i % kPRing holding group j0 + i, refilled with
    // group i + kPRing right after its MFMAs. Activations: XS register sets; group i + 1 goes from
    // set i % XS into LDS stage (i + 1) & 1 after group i's MFMAs, and that set then loads group
    // i + 1 + XS. Every set index is a compile-time constant (the loop is unrolled by the ring size).
    vx_mu4 cw[kPRing][NT];
    vx_mu2 sw[kPRing][NT];
    constexpr int XS = MT <= 4 ? 2 : 1;  // activation register sets (one at 8 row tiles: registers)
    vx_mh8 xr[XS][UPW];
    auto load_w = [&](auto pc, uint32_t j) {
        constexpr int p = decltype(pc)::value;
        const uint32_t jc = min(j, jl);
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            cw[p][nt] = cp[nt][(size_t)jc * 64u];
            sw[p][nt] = sp[nt][(size_t)jc * 16u];
        }
    };
    auto load_x = [&](auto pc, uint32_t j) {
        constexpr int p = decltype(pc)::value;
        const uint32_t jc = min(j, jl);
#pragma unroll
        for (int i = 0; i < UPW; ++i)
            xr[p][i] = *(const vx_mh8*)(xsrc[i] + (size_t)min(4u * jc + xblk[i], b_last) * xbs);
    };
    auto store_x = [&](auto pc, int s) {
        constexpr int p = decltype(pc)::value;
#pragma unroll
        for (int i = 0; i < UPW; ++i) xs[kh][s][wave + kMWaves * i][lane] = xr[p][i];
    };
    // block b of the group: c = mfma(x, q - 8, 0), acc += d_b c -- the arithmetic of the kernel above.
    // Software-pipelined over (block, row tile): the MFMAs of one (b, mt) are issued before the
    // scale multiply-adds of the previous one, so each product has two MFMAs' time to complete
    // before a VALU instruction reads it (written plainly, the compiler gave every MFMA the same
    // result registers and waited out each one with s_nop before its multiply-adds).
    auto compute = [&](auto pc, int s) {
        constexpr int p = decltype(pc)::value;
        vx_mh8 q[NT];
        float d[NT], dprev[NT];
        vx_mf4 cprev[NT];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                q[nt] = vx_munpack8(cw[p][nt][b], e6400);
                d[nt] = (float)__builtin_bit_cast(vx_mh2, b < 2 ? sw[p][nt].x : sw[p][nt].y)[b & 1];
            }
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const vx_mh8 xa = xs[kh][s][b * MT + mt][lane];
                vx_mf4 cnew[NT];
#pragma unroll
                for (int nt = 0; nt < NT; ++nt)
                    cnew[nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xa, q[nt], vx_mf4{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
                if (b | mt) {  // compile-time: the previous (block, row tile)'s products
                    const int pm = mt ? mt - 1 : MT - 1;
#pragma unroll
                    for (int nt = 0; nt < NT; ++nt) acc[nt][pm] += dprev[nt] * cprev[nt];
                }
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    cprev[nt] = cnew[nt];
                    dprev[nt] = d[nt];
                }
            }
        }
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[nt][MT - 1] += dprev[nt] * cprev[nt];
    };
    // group j0 + i (set i % kPRing, stage i & 1), then the loads it frees; a stage is rewritten
    // only after the barrier that follows every wave's reads of it. Past the range the loads are
    // clamped to its last group (in bounds, unused). Vector loads retire in issue order, so the
    // wait before an activation store also waits for every load issued before that activation
    // group: each step issues its activation group before its weight group, and the wait for
    // group i + 1's activations then reaches only the weights of group i + 1 (XS = 2) or i + 2
    // (XS = 1), loaded 3 or 2 steps earlier (issued the other way round, it reached the weights of
    // group i + 2 or i + 3, loaded 2 steps or 1 step earlier). The scheduling barriers keep each
    // step's loads in this order, and the prologue leaves the same loads outstanding as a step
    // does, so the waits the compiler places count the same loads on every path.
    auto step = [&](auto pc, uint32_t i) {
        constexpr int p = decltype(pc)::value;
        if (i < nj) compute(pc, p & 1);  // wave-uniform
        __builtin_amdgcn_sched_barrier(0);
        store_x(vx_ic<p % XS>{}, (p + 1) & 1);
        load_x(vx_ic<p % XS>{}, j0 + i + 1u + (uint32_t)XS);
        load_w(pc, j0 + i + (uint32_t)kPRing);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
    };
    static_assert(kPRing == 4, "the loop below is unrolled by 4");
    // outstanding after the prologue, oldest first: XS = 2: w1 x1 w2 x2 w3; XS = 1: w2 x1 w3 (as
    // after a step of the loop)
    load_w(vx_ic<0>{}, j0);
    if constexpr (XS == 1) load_w(vx_ic<1>{}, j0 + 1u);
    load_x(vx_ic<0>{}, j0);
    if constexpr (XS == 2) load_w(vx_ic<1>{}, j0 + 1u);
    __builtin_amdgcn_sched_barrier(0);
    store_x(vx_ic<0>{}, 0);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (XS == 2) {
        load_x(vx_ic<0>{}, j0 + 1u);
        load_w(vx_ic<2>{}, j0 + 2u);
        load_x(vx_ic<1>{}, j0 + 2u);
    } else {
        load_w(vx_ic<2>{}, j0 + 2u);
        load_x(vx_ic<0>{}, j0 + 1u);
    }
    load_w(vx_ic<3>{}, j0 + 3u);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    uint32_t i = 0;
    for (; i + 4u <= ns; i += 4u) {
        step(vx_ic<0>{}, i);
        step(vx_ic<1>{}, i + 1u);
        step(vx_ic<2>{}, i + 2u);
        step(vx_ic<3>{}, i + 3u);
    }
    if (i < ns) step(vx_ic<0>{}, i);  // the last 1..3 steps (workgroup-uniform branches)
    if (i + 1u < ns) step(vx_ic<1>{}, i + 1u);
    if (i + 2u < ns) step(vx_ic<2>{}, i + 2u);

    // the second half's sums into LDS (the stages are free after the last step's barrier), added
    // to the first half's in that order
    if constexpr (KH == 2) {
        vx_mf4(*red)[NT * MT][64] = (vx_mf4(*)[NT * MT][64])&xs[0][0][0][0];
        if (kh) {
#pragma unroll
            for (int nt = 0; nt < NT; ++nt)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) red[wave][nt * MT + mt][lane] = acc[nt][mt];
        }
        __syncthreads();
        if (kh) return;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[nt][mt] += red[wave][nt * MT + mt][lane];
    }

    // ---- epilogues (every wave, its two tiles): lane holds acc[nt][mt][i] for activation row
    // m = 16 mt + 4 g + i of tile T0 + nt's row 16 t + row ----
    if constexpr (EPI == VX_EPI_SWIGLU) {
        const uint32_t jrow = 16u * (T0 >> 1) + (uint32_t)row;  // T0 the gate tile, T0 + 1 its up tile
        if (T0 < w.n_tiles && jrow < w.n) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t m = r0 + (uint32_t)(16 * mt + 4 * g + i);
                    if (m >= a.batch) continue;
                    const float gt = acc[0][mt][i], up = acc[1][mt][i];
                    a.out16[(size_t)m * a.ldo + (size_t)(jrow >> 5) * a.obs + (jrow & 31u)] =
                        __half_as_ushort(__float2half((gt / (1.0f + expf(-gt))) * up));
                }
        }
    } else if constexpr (EPI == VX_EPI_ARGMAX) {
        // one candidate slot per tile pair, as the kernel above (its workgroups hold one pair)
        const uint32_t slot = T0 >> 1, nslots = (w.n_tiles + 1u) >> 1;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t m = r0 + (uint32_t)(16 * mt + 4 * g + i);
                float bv = -INFINITY;
                uint32_t bi = 0xFFFFFFFFu;
#pragma unroll
                for (int nt = 0; nt < NT; ++nt) {
                    const uint32_t t = T0 + (uint32_t)nt, n = 16u * t + (uint32_t)row;
                    if (t < w.n_tiles && n < w.n) {
                        if (m < a.batch) a.y[(size_t)m * a.ldy + n] = acc[nt][mt][i];
                        if (vx_mbetter(acc[nt][mt][i], n, bv, bi)) { bv = acc[nt][mt][i]; bi = n; }
                    }
                }
#pragma unroll
                for (int off = 1; off < 16; off <<= 1) {
                    const float ov = __shfl_xor(bv, off);
                    const uint32_t oi = __shfl_xor(bi, off);
                    if (vx_mbetter(ov, oi, bv, bi)) { bv = ov; bi = oi; }
                }
                if (row == 0 && m < a.batch && slot < nslots) {
                    a.cand_v[(size_t)m * nslots + slot] = bv;
                    a.cand_i[(size_t)m * nslots + slot] = bi;
                }
            }
    } else {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const uint32_t t = T0 + (uint32_t)nt, n = 16u * t + (uint32_t)row;
            if (t >= w.n_tiles || n >= w.n) continue;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const uint32_t m = r0 + (uint32_t)(16 * mt + 4 * g + i);
                    if (m >= a.batch) continue;
                    const float v = acc[nt][mt][i];
                    if (gridDim.y > 1u) {
                        a.part[blockIdx.y * a.pstride + (size_t)m * a.ldy + n] = v;
                    } else {
                        float* yp = a.y + (size_t)m * a.ldy + n;
                        if constexpr (EPI == VX_EPI_STORE) *yp = a.bias ? v + a.bias[n] : v;
                        else *yp += v;
                    }
                }
        }
    }
}

namespace {

constexpr int kMNT = 2;  // tiles per wave (a gate/up pair for SWIGLU)

// Used for 17-128 rows (Qwen2.5-7B decode at 32 sequences: 9797-9850 -> 9972-10164 tok/s).
// Two K halves per workgroup where the grid is at most one round of workgroups and each has 8 or
// more groups (Llama-3-8B at 64 rows: gate/up 47.5 -> 36.2 us, down); one where the grid already
// fills the CUs or the groups are few (QKV and o_proj split 5-8 ways over K, the LM head).
template <int EPI, int MT, int KH>
hipError_t vx_pgemm_launch_kh(const VxMMat& w, const VxBGemmArgs& a, dim3 grid, hipStream_t st) {
    constexpr size_t lds = (size_t)KH * 2 * 4 * MT * 1024;  // [half][stage][4 MT activation tiles of 1 KiB]
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)vx_pgemm_kernel<EPI, MT, KH>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        attr_set = true;
    }
    grid.z = (a.batch + 16u * MT - 1u) / (16u * MT);  // blocks of 16 MT activation rows
    hipLaunchKernelGGL((vx_pgemm_kernel<EPI, MT, KH>), grid, dim3(KH * kMThreads), lds, st, w, a);
    return hipGetLastError();
}

template <int EPI, int MT>
hipError_t vx_pgemm_launch_t(const VxMMat& w, const VxBGemmArgs& a, hipStream_t st) {
    const uint32_t ks = a.ksplit > 1u ? a.ksplit : 1u;
    const dim3 grid((w.n_tiles + kPTiles - 1u) / kPTiles, ks);
    const uint64_t wgs = (uint64_t)grid.x * ks * ((a.batch + 16u * MT - 1u) / (16u * MT));
    if (wgs <= 256u && w.n_grp / ks >= 8u) return vx_pgemm_launch_kh<EPI, MT, 2>(w, a, grid, st);
    return vx_pgemm_launch_kh<EPI, MT, 1>(w, a, grid, st);
}

template <int EPI, int MT>
hipError_t vx_mgemm_launch_t(const VxMMat& w, const VxBGemmArgs& a, hipStream_t st) {
    const dim3 grid(vx_mgemm_grid(w.n_tiles), a.ksplit > 1u ? a.ksplit : 1u);
    hipLaunchKernelGGL((vx_mgemm_kernel<EPI, MT, kMNT>), grid, dim3(kMThreads), 0, st, w, a);
    return hipGetLastError();
}

template <int EPI>
hipError_t vx_mgemm_dispatch_mt(const VxMMat& w, const VxBGemmArgs& a, hipStream_t st) {
    if (a.batch == 0 || a.batch > 128) return hipErrorInvalidValue;
    if (a.batch <= 16) return vx_mgemm_launch_t<EPI, 1>(w, a, st);  // (the LDS-shared kernel: B=8 3857 -> 3640 tok/s)
    if (a.batch <= 32) return vx_pgemm_launch_t<EPI, 2>(w, a, st);
    if (a.batch <= 48) return vx_pgemm_launch_t<EPI, 3>(w, a, st);
    // 49-128 rows: blocks of 4 row tiles from the grid's z dimension. At 65-128 rows each weight
    // tile is then read by two workgroups, but twice the workgroups (single K halves, two per CU)
    // run out of phase with each other, so one's loads and barrier overlap the other's MFMAs: TTFT
    // at 128 tokens 5.84-5.93 -> 5.70-5.78 ms (Llama-3-8B), 5.73-5.77 -> 5.49-5.55 ms (Qwen2.5-7B)
    // against one block of 8 row tiles (two K halves per workgroup where one round of workgroups
    // holds the grid), same box, three alternating runs each
    return vx_pgemm_launch_t<EPI, 4>(w, a, st);
}

}  // namespace

uint32_t vx_mgemm_grid(uint32_t n_tiles) { return (n_tiles + kMNT - 1u) / kMNT; }
uint32_t vx_pgemm_grid(uint32_t n_tiles) { return (n_tiles + kPTiles - 1u) / kPTiles; }

void vx_mmat_shape(uint32_t n, uint32_t k, uint32_t paired, VxMMat& m) {
    m.n = n;
    m.k = k;
    m.paired = paired;
    const uint32_t t = (n + 15u) / 16u;
    m.n_tiles = paired ? 2u * t : t;
    m.n_grp = (k / 32u + 3u) / 4u;
}

uint64_t vx_mmat_code_bytes(const VxMMat& m) { return (uint64_t)m.n_tiles * m.n_grp * 64u * 16u; }
uint64_t vx_mmat_scale_bytes(const VxMMat& m) { return (uint64_t)m.n_tiles * m.n_grp * 16u * 8u; }

hipError_t vx_launch_mlayout(const VxMat& src, const VxMMat& dst, hipStream_t st) {
    if (src.n != dst.n || src.k != dst.k || src.paired != dst.paired || (src.k & 31u)) return hipErrorInvalidValue;
    const size_t total = (size_t)dst.n_tiles * dst.n_grp * 64u;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(vx_mlayout_kernel, dim3((unsigned)((total + 255u) / 256u)), dim3(256), 0, st, src, dst);
    return hipGetLastError();
}

hipError_t vx_launch_mgemm(const VxMMat& w, const VxBGemmArgs& a, int epi, hipStream_t st) {
    if (w.k == 0 || (w.k & 31u) || (a.ldx & 7u) || (a.xbs & 7u) || !a.x16 || !vx_x_layout_ok(w.k, a.ldx, a.xbs, a.batch))
        return hipErrorInvalidValue;
    if (epi == VX_EPI_SWIGLU && !vx_x_layout_ok(w.n, a.ldo, a.obs, a.batch)) return hipErrorInvalidValue;
    if ((epi == VX_EPI_SWIGLU) != (w.paired != 0)) return hipErrorInvalidValue;
    if (a.ksplit > 1u && ((epi != VX_EPI_RESID && epi != VX_EPI_STORE) || !a.part || a.ksplit > w.n_grp ||
                          a.ksplit > 8u || a.pstride < (uint64_t)a.batch * a.ldy))
        return hipErrorInvalidValue;
    switch (epi) {
        case VX_EPI_STORE: return vx_mgemm_dispatch_mt<VX_EPI_STORE>(w, a, st);
        case VX_EPI_RESID: return vx_mgemm_dispatch_mt<VX_EPI_RESID>(w, a, st);
        case VX_EPI_SWIGLU: return vx_mgemm_dispatch_mt<VX_EPI_SWIGLU>(w, a, st);
        case VX_EPI_ARGMAX: return vx_mgemm_dispatch_mt<VX_EPI_ARGMAX>(w, a, st);
        default: return hipErrorInvalidValue;
    }
}

hipError_t vx_launch_msum(const float* part, uint32_t nparts, uint64_t pstride, const float* bias, float* y,
                          uint32_t n, uint32_t ldy, uint32_t batch, uint32_t accumulate, uint64_t mask,
                          hipStream_t st) {
    if (nparts == 0 || nparts > 8 || batch == 0 || ldy < n || pstride < (uint64_t)batch * ldy)
        return hipErrorInvalidValue;
    const uint32_t gx = (n + 255u) / 256u;
    hipLaunchKernelGGL(vx_msum_kernel, dim3(gx ? gx : 1u, batch), dim3(256), 0, st, part, nparts, pstride, bias, y, n,
                       ldy, accumulate, mask);
    return hipGetLastError();
}
