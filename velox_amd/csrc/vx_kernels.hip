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
//     RMSNorm runs in the prologue, residual / SwiGLU / argmax in the epilogue.
//   * Decode attention: split-K over the sequence, RoPE + bf16 KV append in the prologue,
//     online softmax per split, LSE merge by the last workgroup of each KV head.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "vx_common.h"

typedef _Float16 vx_h2 __attribute__((ext_vector_type(2)));
typedef uint32_t vx_u32x4 __attribute__((ext_vector_type(4)));

namespace {

constexpr int kWG = 256;  // threads per workgroup (4 wave64)


// 2^x on the transcendental unit (the softmax works in the log2 domain)
__device__ __forceinline__ float vx_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float vx_h2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)h)); }

// Code dword layout (8 weights): byte j holds element j in its low nibble and element j + 4 in
// its high nibble. v_perm_b32 places two nibble bytes under the fp16 exponent byte 0x64, giving
// half2 (1024 + q_a, 1024 + q_b) for consecutive elements, consumed by v_dot2c_f32_f16 against the
// matching fp16 activation pair; the -1032 offset is folded into the block correction.
__device__ __forceinline__ uint32_t vx_code_nibble(uint32_t dw, int e) { return (dw >> (8 * (e & 3) + 4 * (e >> 2))) & 15u; }

// Activations of the GEMV: block b of 32 values u is scaled by 2^e (e from its largest magnitude
// m: m 2^e in [2^(B - 1), 2^B), B = kXBits) and rounded to integers X (|X| <= 2^B), written as
// kXDigits balanced base-16 digits c_d in [-8, 7] (X = sum c_d 16^d; c_d + 8 is digit d of
// X + kXOffset, the number with 8 in each digit). Digit d of the 8 values of code dword w sits at
// the same nibble positions as their codes (value j at bit 8 (j & 3) + 4 (j >> 2)), so
// v_dot8_i32_i4 of the code dword xor 0x88888888 (q - 8 as a signed nibble) and the digit dword
// is sum (q - 8) c_d over 8 values, exactly. Zero, NaN and inf blocks keep e = 0.
constexpr int kXDigits = 6;
constexpr int kXBits = 4 * kXDigits - 2;  // balanced digits reach 8 (16^D - 1) / 15 > 2^B
constexpr uint32_t kXOffset = 0x888888u >> (4 * (6 - kXDigits));
static_assert(kXDigits == 5 || kXDigits == 6, "five or six digits: 18 or 22 bits");

__device__ __forceinline__ int vx_xblock_exp(float m) {
    if (!(m > 0.0f) || m > 3.0e38f) return 0;
    const int e = (kXBits - 1) - ((int)((__float_as_uint(m) >> 23) & 255u) - 127);  // B - 1 - floor(log2 m)
    return e < -100 ? -100 : (e > 120 ? 120 : e);
}

__device__ __forceinline__ float vx_pow2f(int e) { return __uint_as_float((uint32_t)(e + 127) << 23); }

template <int CTRL>
__device__ __forceinline__ float vx_dpp(float x) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, true));
}

// Sum over aligned groups of S lanes (S in 2..64): DPP within 16-lane rows, a swizzle across rows.
template <int S>
__device__ __forceinline__ float vx_group_sum(float v) {
    if constexpr (S >= 2) v += vx_dpp<0xB1>(v);   // quad_perm [1,0,3,2]
    if constexpr (S >= 4) v += vx_dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    if constexpr (S >= 8) v += vx_dpp<0x141>(v);  // row_half_mirror
    if constexpr (S >= 16) v += vx_dpp<0x140>(v); // row_mirror
    if constexpr (S >= 32) v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401F));
    if constexpr (S >= 64) v += __shfl_xor(v, 32);
    return v;
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

// Block-wide sum over W waves; red must hold W floats. Result broadcast to all threads.
template <int W>
__device__ __forceinline__ float vx_block_sum(float v, float* red) {
    v = vx_wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.0f;
#pragma unroll
    for (int w = 0; w < W; ++w) t += red[w];
    return t;
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
        for (int e = 0; e < 8; ++e) {
            const int el = 8 * w + e;
            const uint32_t q = el < 16 ? (qs[el] & 15u) : (qs[el - 16] >> 4);
            v |= q << (8 * (e & 3) + 4 * (e >> 2));
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
// Each wave streams the code words of its tiles as one flat sequence of items (tile, iteration):
// kU 16-byte loads stay in flight per lane across tile boundaries. The activations are loaded
// first, then the first kU weight items, so staging x in LDS overlaps the weight fetch. Every
// load outside the last 2*kU items is issued unconditionally: vector memory completes in issue
// order, and with no load under a branch the compiler's s_waitcnt for item u waits for that item
// only, keeping kU items in flight instead of draining the queue once per iteration. Each workgroup
// owns a contiguous block of tiles, dealt to its waves round-robin.
// No workgroup waits on another: the LM head's argmax leaves one candidate per workgroup for
// vx_argmax_finalize_kernel (a release fence per workgroup costs a full L2 write-back on gfx950).
constexpr int kGemvWaves = 8, kGemvU = 4;

template <int S, int EPI, bool NORM, int GX, int SPL>
__global__ __launch_bounds__(64 * kGemvWaves) void vx_gemv_q4_kernel(VxGemvArgs a) {
    extern __shared__ __align__(16) unsigned char vx_smem[];
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr int W = kGemvWaves, kU = kGemvU, R = 64 / S, NT = 64 * W;
    const uint32_t K = a.k, nb = K >> 5, n_iter = a.n_iter;
    // activations: kXDigits planes of nb 16-byte chunks (the 4 digit dwords of one block), then the
    // blocks' unscale factors 2^-e
    uint4* xs4 = (uint4*)vx_smem;
    float* unscale = (float*)(xs4 + (size_t)kXDigits * nb);
    float* red = unscale + nb;
    // the wave index is uniform: readfirstlane lets every per-wave quantity live in SGPRs
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane / S, s = lane % S;
    // workgroup blocks: workgroup b owns tiles [b n / grid, (b + 1) n / grid), dealt to its W waves
    // round-robin, so every workgroup (every CU) streams the same number of tiles
    const uint32_t b0 = (uint32_t)(((uint64_t)blockIdx.x * a.n_tiles) / gridDim.x);
    const uint32_t b1 = (uint32_t)(((uint64_t)(blockIdx.x + 1u) * a.n_tiles) / gridDim.x);
    const uint32_t first = b0 + (uint32_t)wave, step = (uint32_t)W;
    const uint32_t my_tiles = first < b1 ? (b1 - 1u - first) / (uint32_t)W + 1u : 0u;
    const uint32_t total = my_tiles * n_iter;

    auto row_of = [&](uint32_t t) -> uint32_t {
        if constexpr (EPI == VX_EPI_SWIGLU) return t * (R / 2) + (r % (R / 2));  // logical j of gate/up
        else return t * R + r;
    };

    // ---- activations (and the RMSNorm gain) into registers, before any weight load ----
    const uint32_t ng = K >> 3;  // 8-element groups; a multiple of 4
    float4 xv[2 * GX], gv[2 * GX];
    // SPL > 0: the activations are SPL split-K attention partials per head, merged below
    float2 pml[SPL > 0 ? GX : 1][SPL > 0 ? SPL : 1];
    float4 po[SPL > 0 ? GX : 1][SPL > 0 ? SPL : 1][2];
#pragma unroll
    for (int i = 0; i < GX; ++i) {
        const uint32_t g = min((uint32_t)tid + (uint32_t)i * NT, ng - 1u);  // clamped: never a branch
        if constexpr (SPL == 0) {
            xv[2 * i] = *(const float4*)(a.x + 8u * g);
            xv[2 * i + 1] = *(const float4*)(a.x + 8u * g + 4u);
        } else {
            const uint32_t h = (8u * g) / a.att_d, e0 = 8u * g - h * a.att_d;
#pragma unroll
            for (int sp = 0; sp < SPL; ++sp) {
                const size_t hs = (size_t)h * SPL + (uint32_t)sp;
                pml[i][sp] = *(const float2*)(a.part_ml + hs * 2u);
                po[i][sp][0] = *(const float4*)(a.part_o + hs * a.att_d + e0);
                po[i][sp][1] = *(const float4*)(a.part_o + hs * a.att_d + e0 + 4u);
            }
        }
        if constexpr (NORM) {
            gv[2 * i] = *(const float4*)(a.gain + 8u * g);
            gv[2 * i + 1] = *(const float4*)(a.gain + 8u * g + 4u);
        }
    }

    // Code words and scales through buffer descriptors: per-lane offsets are constant, the item
    // offset is wave-uniform (scalar). Padded slots of a tile hold zero codes and zero scales, so
    // they are loaded and contribute exactly 0 without any per-lane branch.
    const __amdgpu_buffer_rsrc_t rc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.codes, (short)0, (int)(a.n_tiles * n_iter * 1024u), 0x00020000);
    const __amdgpu_buffer_rsrc_t rsc =
        __builtin_amdgcn_make_buffer_rsrc((void*)a.scales, (short)0, (int)(a.n_tiles * n_iter * 128u), 0x00020000);
    const uint32_t lane16 = (uint32_t)lane * 16u, lane2 = (uint32_t)lane * 2u;
    vx_u32x4 buf[kU];
    uint32_t sbuf[kU];
    uint32_t nt = 0, ni = 0, nslot = first * n_iter;  // next item: tile index, iteration, 64-lane slot
    auto advance = [&]() {
        if (++ni == n_iter) {
            ni = 0;
            ++nt;
            nslot = (first + nt * step) * n_iter;
        } else {
            ++nslot;
        }
    };
    // unconditional load of the next item; past this wave's last item it re-reads slot 0 (in
    // bounds, cache-resident after the first wave touches it) and the value is never consumed
    auto issue = [&](int u) {
        const uint32_t slot = __builtin_amdgcn_readfirstlane(nt < my_tiles ? nslot : 0u);
        buf[u] = __builtin_amdgcn_raw_buffer_load_b128(rc, lane16, slot * 1024u, 2);
        sbuf[u] = __builtin_amdgcn_raw_buffer_load_b16(rsc, lane2, slot * 128u, 2);
        advance();
    };
#pragma unroll
    for (int u = 0; u < kU; ++u) issue(u);

    if constexpr (SPL > 0) {
        // LSE merge of the splits (m, l in the log2 domain; an empty split has m = -inf, l = 0):
        // x = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s, the merge of
        // tests/empirical_challenge_phase2/test2_split_k_flashdecoding_parity.cu:23-125
#pragma unroll
        for (int i = 0; i < GX; ++i) {
            float M = -INFINITY;
#pragma unroll
            for (int sp = 0; sp < SPL; ++sp) M = fmaxf(M, pml[i][sp].x);
            float L = 0.0f, w[SPL];
#pragma unroll
            for (int sp = 0; sp < SPL; ++sp) {
                w[sp] = pml[i][sp].x == -INFINITY ? 0.0f : vx_exp2(pml[i][sp].x - M);
                L += w[sp] * pml[i][sp].y;
            }
            const float invl = L > 0.0f ? 1.0f / L : 0.0f;
            float4 x0 = make_float4(0.f, 0.f, 0.f, 0.f), x1 = x0;
#pragma unroll
            for (int sp = 0; sp < SPL; ++sp) {
                const float ws = w[sp] * invl;
                x0.x += ws * po[i][sp][0].x; x0.y += ws * po[i][sp][0].y;
                x0.z += ws * po[i][sp][0].z; x0.w += ws * po[i][sp][0].w;
                x1.x += ws * po[i][sp][1].x; x1.y += ws * po[i][sp][1].y;
                x1.z += ws * po[i][sp][1].z; x1.w += ws * po[i][sp][1].w;
            }
            xv[2 * i] = x0;
            xv[2 * i + 1] = x1;
        }
    }

    // ---- RMSNorm scale (src/runtime.rs:588-601) from the registers, plus groups beyond them ----
    float inv_rms = 1.0f;
    if constexpr (NORM) {
        float ss = 0.0f;
#pragma unroll
        for (int i = 0; i < GX; ++i) {
            if ((uint32_t)tid + (uint32_t)i * NT < ng) {
                const float4 v0 = xv[2 * i], v1 = xv[2 * i + 1];
                ss += v0.x * v0.x + v0.y * v0.y + v0.z * v0.z + v0.w * v0.w;
                ss += v1.x * v1.x + v1.y * v1.y + v1.z * v1.z + v1.w * v1.w;
            }
        }
        for (uint32_t g = (uint32_t)tid + GX * NT; g < ng; g += NT) {
            const float4 v0 = *(const float4*)(a.x + 8u * g);
            const float4 v1 = *(const float4*)(a.x + 8u * g + 4u);
            ss += v0.x * v0.x + v0.y * v0.y + v0.z * v0.z + v0.w * v0.w;
            ss += v1.x * v1.x + v1.y * v1.y + v1.z * v1.z + v1.w * v1.w;
        }
        ss = vx_block_sum<W>(ss, red);
        inv_rms = 1.0f / sqrtf(ss / (float)K + a.eps);
    }
    // x -> LDS digit planes [d][b] (16 bytes: the digit dwords of the block's 4 code dwords): the S
    // lanes of a row read blocks b..b+S-1 of one plane at consecutive 16-byte addresses (no LDS
    // bank conflicts). Group g = values 8g..8g+7 = code dword g & 3 of block g >> 2.
    auto stage = [&](uint32_t g, float4 v0, float4 v1, float4 g0, float4 g1) {
        float u[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        if constexpr (NORM) {
            const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) u[e] = (u[e] * inv_rms) * gg[e];
        }
        // the four 8-element groups of one 32-block sit in four consecutive lanes, which are all
        // in range or all out of range (ng is a multiple of 4); nan is NaN when any value is NaN
        // or infinite (the block's result is then NaN, as the fp32 dot product's would be)
        float m = 0.0f, nan = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            m = fmaxf(m, fabsf(u[e]));
            nan += u[e] * 0.0f;
        }
        m = fmaxf(m, __shfl_xor(m, 1));
        m = fmaxf(m, __shfl_xor(m, 2));
        nan += __shfl_xor(nan, 1);
        nan += __shfl_xor(nan, 2);
        const int ex = vx_xblock_exp(m);
        const float sc = vx_pow2f(ex);
        // Y = X + kXOffset (so that its plain base-16 digits are c_d + 8): adding 1.5 * 2^23 to the
        // exactly scaled value rounds it to an integer (to nearest even, |X| <= 2^B <= 2^22) held in
        // the low mantissa bits
        uint32_t Y[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) Y[e] = __float_as_uint(u[e] * sc + 12582912.0f) - (0x4B400000u - kXOffset);
        // byte k of Y holds digits 2k (low nibble) and 2k + 1 (high nibble): gather byte k of
        // values 0-3 and of values 4-7, then split the nibbles into the two digit dwords (values
        // 0-3 in the low nibbles, 4-7 in the high ones); xor 8 turns c_d + 8 into c_d's signed nibble
        uint32_t* dst = (uint32_t*)xs4 + (size_t)(g >> 2) * 4u + (g & 3u);
#pragma unroll
        for (int k = 0; k < (kXDigits + 1) / 2; ++k) {
            const uint32_t sel = 0x0C0C0000u | ((4u + (uint32_t)k) << 8) | (uint32_t)k;
            const uint32_t lw = __builtin_amdgcn_perm(__builtin_amdgcn_perm(Y[3], Y[2], sel),
                                                      __builtin_amdgcn_perm(Y[1], Y[0], sel), 0x05040100u);
            const uint32_t hw = __builtin_amdgcn_perm(__builtin_amdgcn_perm(Y[7], Y[6], sel),
                                                      __builtin_amdgcn_perm(Y[5], Y[4], sel), 0x05040100u);
            const uint32_t d0 = (lw & 0x0F0F0F0Fu) | ((hw << 4) & 0xF0F0F0F0u);
            dst[(size_t)(2 * k) * nb * 4u] = d0 ^ 0x88888888u;
            if (2 * k + 1 < kXDigits) {
                const uint32_t d1 = ((lw >> 4) & 0x0F0F0F0Fu) | (hw & 0xF0F0F0F0u);
                dst[(size_t)(2 * k + 1) * nb * 4u] = d1 ^ 0x88888888u;
            }
        }
        if ((g & 3u) == 0u) unscale[g >> 2] = vx_pow2f(-ex) + nan;
    };
#pragma unroll
    for (int i = 0; i < GX; ++i) {
        const uint32_t g = (uint32_t)tid + (uint32_t)i * NT;
        if (g < ng) stage(g, xv[2 * i], xv[2 * i + 1], gv[2 * i], gv[2 * i + 1]);
    }
    for (uint32_t g = (uint32_t)tid + GX * NT; g < ng; g += NT) {
        const float4 v0 = *(const float4*)(a.x + 8u * g), v1 = *(const float4*)(a.x + 8u * g + 4u);
        float4 g0 = v0, g1 = v1;
        if constexpr (NORM) {
            g0 = *(const float4*)(a.gain + 8u * g);
            g1 = *(const float4*)(a.gain + 8u * g + 4u);
        }
        stage(g, v0, v1, g0, g1);
    }
    __syncthreads();

    // ---- stream: consume slot u, refill it with the item kU ahead, finish tiles on the fly ----
    float best_v = -INFINITY;
    uint32_t best_i = 0xFFFFFFFFu;
    float acc = 0.0f;
    uint32_t ct = 0, ci = 0;  // current item
    auto consume = [&](int u) {
        // padded blocks (b >= nb, zero scale) read a valid activation chunk instead
        const uint32_t b = min(ci * S + s, nb - 1u);
        const vx_u32x4 c = buf[u] ^ 0x88888888u;  // q - 8 as signed nibbles
        int dg[kXDigits];
#pragma unroll
        for (int d = 0; d < kXDigits; ++d) {
            const uint4 xd = xs4[(uint32_t)d * nb + b];
            int t = __builtin_amdgcn_sdot8((int)c.x, (int)xd.x, 0, false);
            t = __builtin_amdgcn_sdot8((int)c.y, (int)xd.y, t, false);
            t = __builtin_amdgcn_sdot8((int)c.z, (int)xd.z, t, false);
            dg[d] = __builtin_amdgcn_sdot8((int)c.w, (int)xd.w, t, false);  // |.| <= 2048
        }
        // sum (q - 8) X = lo + 4096 hi, both below 2^20 in magnitude: exact in fp32, one rounding
        const int lo = dg[0] + dg[1] * 16 + dg[2] * 256;
        const int hi = kXDigits == 6 ? dg[3] + dg[4] * 16 + dg[kXDigits - 1] * 256 : dg[3] + dg[4] * 16;
        const float dot = fmaf((float)hi, 4096.0f, (float)lo);
        acc = fmaf(vx_h2f(sbuf[u]) * unscale[b], dot, acc);
        if (++ci == n_iter) {
            acc = vx_group_sum<S>(acc);
            const uint32_t row = row_of(first + ct * step);
            const bool row_ok = row < a.n;
            if constexpr (EPI == VX_EPI_STORE) {
                if (s == 0 && row_ok) a.y[row] = a.bias ? acc + a.bias[row] : acc;
            } else if constexpr (EPI == VX_EPI_RESID) {
                if (s == 0 && row_ok) a.y[row] = a.res[row] + acc;
            } else if constexpr (EPI == VX_EPI_SWIGLU) {
                const float up = __shfl_down(acc, 32);  // partner up row is 32 lanes above
                if (s == 0 && r < R / 2 && row_ok) {
                    const float gt = acc;
                    a.y[row] = (gt / (1.0f + expf(-gt))) * up;  // src/runtime.rs:1064-1066
                }
            } else {  // VX_EPI_ARGMAX
                if (s == 0 && row_ok) {
                    a.y[row] = acc;
                    if (vx_better(acc, row, best_v, best_i)) { best_v = acc; best_i = row; }
                }
            }
            acc = 0.0f;
            ci = 0;
            ++ct;
        }
    };
    uint32_t f0 = 0;
    // steady state: every refill is a real item of this wave
    for (; f0 + 2u * kU <= total; f0 += kU) {
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            consume(u);
            issue(u);
        }
    }
    // the last (< 2 kU) items: refills only while items remain
    for (; f0 < total; f0 += kU) {
#pragma unroll
        for (int u = 0; u < kU; ++u) {
            if (f0 + u < total) {
                consume(u);
                if (f0 + u + kU < total) issue(u);
            }
        }
    }

    if constexpr (EPI == VX_EPI_ARGMAX) {
        __shared__ float s_v[W];
        __shared__ uint32_t s_i[W];
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
            for (int w = 1; w < W; ++w)
                if (vx_better(s_v[w], s_i[w], bv, bi)) { bv = s_v[w]; bi = s_i[w]; }
            a.cand_v[blockIdx.x] = bv;
            a.cand_i[blockIdx.x] = bi;
        }
    }
}

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
template <int D, int G>
constexpr int vx_attn_hrows() { return G <= 4 ? 4 : 8; }  // head rows of the per-wave O in LDS

template <int D, int G, int W>
constexpr size_t vx_attn_lds_bytes() {
    return (size_t)3 * 16 * (D + 8) * 2 + (size_t)2 * D * 2 + (size_t)W * 16 * 2 * 4 + 16 * 4 +
           (size_t)W * vx_attn_hrows<D, G>() * D * 4;
}

template <int D, int G, int W, bool PS>
__global__ __launch_bounds__(64 * W) void vx_attn_kernel(VxAttnArgs a) {
    if ((a.active_mask & 1ULL) == 0ULL) return;
    constexpr int HALF = D / 2, NT = 64 * W, NC = D / 32, NB = D / 16, HR = vx_attn_hrows<D, G>();
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
    const uint32_t g = blockIdx.y, sp = blockIdx.x, bq = blockIdx.z;  // bq: sequence of a batch
    const uint32_t chunk = ((a.s_max + a.splits - 1u) / a.splits + 31u) & ~31u;
    const uint32_t t0 = sp * chunk;
    uint16_t* kvb = a.kv + (size_t)bq * a.kv_bstride;
    uint16_t* Kc = kvb + (size_t)g * a.s_cap * D;
    uint16_t* Vc = kvb + ((size_t)a.hkv + g) * a.s_cap * D;

    constexpr int NP = (G + 1) * HALF, RP = (NP + NT - 1) / NT;  // RoPE pairs, pairs per thread
    // ---- the decode position first, as a vector load, then the RoPE row it selects; vector loads
    // return in order, so both arrive ahead of the q/k/v and K/V chunk loads issued after them (a
    // scalar state load issued after those waited behind every workgroup's whole burst: ~4 us at 256
    // workgroups) ----
    uint64_t step = (uint64_t)a.fixed_pos;
    if (a.state) step = __hip_atomic_load((uint64_t*)&a.state[bq].step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    step = ((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(step >> 32)) << 32) |
           (uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)step);
    const uint32_t pos = step < (uint64_t)a.s_max ? (uint32_t)step : a.s_max - 1u;  // safe_step clamp
    // cached positions [t0, t1): below pos, or up to pos when a prefill chunk appended its rows
    const uint32_t t1 = min(a.prefill ? pos + 1u : pos, t0 + chunk);
    const uint32_t n_chunks = t1 > t0 ? (t1 - t0 + 31u) >> 5 : 0u;
    const bool has_new = !a.prefill && t0 <= pos && pos < t0 + chunk;  // this split folds in the new position
    const float2* rp = a.rope + (size_t)pos * HALF;
    float2 rcs[RP];
#pragma unroll
    for (int i = 0; i < RP; ++i) rcs[i] = rp[min(tid + i * NT, NP - 1) % HALF];
    __builtin_amdgcn_sched_barrier(0);

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
        const float* base = a.qkv_part + (size_t)bq * a.qkv_bstride;
        const uint32_t np = a.qkv_nparts;
        auto qkv_at = [&](uint32_t c) {
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
            const int hh = p / HALF, j = p % HALF;
            const uint32_t c0 = (hh < G ? (g * G + hh) : (a.hq + g)) * (uint32_t)D + (uint32_t)j;
            r1[i] = qkv_at(c0);
            r2[i] = qkv_at(c0 + HALF);
        }
        vnew = qkv_at(vcol);
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

    // ---- RoPE on this group's q heads and the new k; bf16 K/V row ----
    const float qscale = a.scale * kLog2e;  // scores in the log2 domain
    for (int i = tid; i < 3 * (16 - G) * QP / 2; i += NT) {  // q rows G..15 of every term: zero
        const int t = i / ((16 - G) * QP / 2), r = i % ((16 - G) * QP / 2);
        ((uint32_t*)(qt_s + (t * 16 + G) * QP))[r] = 0u;
    }
#pragma unroll
    for (int i = 0; i < RP; ++i) {
        const int p = tid + i * NT;
        const float2 o = vx_rope_pair(r1[i], r2[i], rcs[i]);
        if (p < NP) {
            const int hh = p / HALF, j = p % HALF;
            if (hh < G) {
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
                pr[4 * b + i] = p < t1 ? sc[b][i] : -INFINITY;
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
    for (int idx = tid; idx < G * D; idx += NT) {
        const int h = idx / D, d = idx % D;
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
        const size_t hq_idx = (size_t)bq * a.hq + (size_t)g * G + h;  // (sequence, q head)
        if (a.splits == 1 && !a.partials_only) {
            a.out[hq_idx * D + d] = l > 0.0f ? o / l : 0.0f;
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
__global__ __launch_bounds__(kWG) void vx_embed_kernel(VxMat m, const VeloxDecodeState* state, uint32_t fixed_token,
                                                       float* h, uint64_t mask) {
    if ((mask & 1ULL) == 0ULL) return;
    const uint32_t token = state ? state->token : fixed_token;
    const uint32_t b = blockIdx.x * kWG + threadIdx.x, nb = m.k >> 5;
    if (b >= nb || token >= m.n) return;  // src/codegen.rs:2386-2390 guard
    if (m.fmt != VX_FMT_Q4) {  // unquantized rows (src/codegen.rs:1108-1117 and its fp16 twin)
#pragma unroll
        for (int e = 0; e < 32; ++e) {
            const size_t i = (size_t)token * m.k + b * 32u + (uint32_t)e;
            h[b * 32 + e] = m.fmt == VX_FMT_F32 ? ((const float*)m.codes)[i]
                                                : __half2float(__ushort_as_half(((const uint16_t*)m.codes)[i]));
        }
        return;
    }
    const uint32_t phys = vx_phys_row(m, token, 0);
    const uint32_t R = 64u / m.s;
    const size_t off = ((size_t)(phys / R) * m.n_iter + b / m.s) * 64u + (phys % R) * m.s + b % m.s;
    const uint4 c = m.codes[off];
    const float d = vx_h2f(m.scales[off]);
    const uint32_t dw[4] = {c.x, c.y, c.z, c.w};
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int e = 0; e < 8; ++e) h[b * 32 + 8 * w + e] = (float)((int)vx_code_nibble(dw[w], e) - 8) * d;
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
    const uint32_t R = 64u / m.s;
    const size_t off = ((size_t)(phys / R) * m.n_iter + b / m.s) * 64u + (phys % R) * m.s + b % m.s;
    const uint4 c = m.codes[off];
    const float d = vx_h2f(m.scales[off]);
    const uint32_t dw[4] = {c.x, c.y, c.z, c.w};
    float* o = out + (size_t)lr * m.k + (size_t)b * 32u;
#pragma unroll
    for (int w = 0; w < 4; ++w)
#pragma unroll
        for (int e = 0; e < 8; ++e) o[8 * w + e] = (float)((int)vx_code_nibble(dw[w], e) - 8) * d;
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
// GEMV grid for n_tiles wave tiles: min(ceil(n_tiles / W), 512, max_wgs) workgroups, each owning an
// equal contiguous block of tiles dealt to its waves round-robin, so every CU streams the same share
// however the workgroups are placed. (Llama-3-8B decode, measured against the alternatives: 714
// tok/s; the same blocks over <= 256 workgroups 708, tiles round-robin over all waves 708, over the
// fewest waves with the largest per-wave tile count 700.)
uint32_t vx_gemv_wgs(uint32_t n_tiles, uint32_t max_wgs) {
    if (n_tiles == 0 || max_wgs == 0) return 1u;
    const uint32_t cap = min(512u, max_wgs);
    const uint32_t w = (n_tiles + kGemvWaves - 1u) / kGemvWaves;
    return w > cap ? cap : (w ? w : 1u);
}

template <int S, int EPI, bool NORM, int GX, int SPL>
hipError_t vx_gemv_launch_t(const VxGemvArgs& a, uint32_t max_wgs, hipStream_t st) {
    constexpr int W = kGemvWaves;
    const uint32_t nb = a.k >> 5;
    const size_t lds = (size_t)nb * (16u * kXDigits + 4u) + 64u;  // K <= 32768: at most 102,464 bytes
    static size_t attr_lds = 64u * 1024u;
    if (lds > attr_lds) {
        if (hipFuncSetAttribute((const void*)vx_gemv_q4_kernel<S, EPI, NORM, GX, SPL>,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        attr_lds = lds;
    }
    const uint32_t wgs = vx_gemv_wgs(a.n_tiles, max_wgs);
    hipLaunchKernelGGL((vx_gemv_q4_kernel<S, EPI, NORM, GX, SPL>), dim3(wgs), dim3(64 * W), lds, st, a);
    return hipGetLastError();
}

// x register groups per thread: ceil(K / 8 / threads) rounded up to 1, 2 or 4 (larger K loops;
// merged attention partials must fit the registers)
template <int S, int EPI, bool NORM, int SPL>
hipError_t vx_gemv_dispatch_gx(const VxGemvArgs& a, uint32_t max_wgs, hipStream_t st) {
    const uint32_t per = ((a.k >> 3) + 64u * kGemvWaves - 1u) / (64u * kGemvWaves);
    if (per <= 1u) return vx_gemv_launch_t<S, EPI, NORM, 1, SPL>(a, max_wgs, st);
    if (per <= 2u) return vx_gemv_launch_t<S, EPI, NORM, 2, SPL>(a, max_wgs, st);
    if (SPL > 0 && per > 4u) return hipErrorInvalidValue;
    return vx_gemv_launch_t<S, EPI, NORM, 4, SPL>(a, max_wgs, st);
}

template <int EPI, bool NORM, int SPL>
hipError_t vx_gemv_dispatch_s(uint32_t s, const VxGemvArgs& a, uint32_t max_wgs, hipStream_t st) {
    switch (s) {
        case 4: return vx_gemv_dispatch_gx<4, EPI, NORM, SPL>(a, max_wgs, st);
        case 8: return vx_gemv_dispatch_gx<8, EPI, NORM, SPL>(a, max_wgs, st);
        case 16: return vx_gemv_dispatch_gx<16, EPI, NORM, SPL>(a, max_wgs, st);
        case 32: return vx_gemv_dispatch_gx<32, EPI, NORM, SPL>(a, max_wgs, st);
        case 64:
            if constexpr (EPI != VX_EPI_SWIGLU) return vx_gemv_dispatch_gx<64, EPI, NORM, SPL>(a, max_wgs, st);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

template <int EPI>
hipError_t vx_gemv_dispatch_norm(uint32_t s, const VxGemvArgs& a, uint32_t max_wgs, hipStream_t st) {
    if constexpr (EPI == VX_EPI_RESID) {
        if (a.gain) return hipErrorInvalidValue;  // the residual epilogue takes raw activations
        if (!a.part_o) return vx_gemv_dispatch_s<EPI, false, 0>(s, a, max_wgs, st);
        // o_proj over split-K attention partials: 8-element groups must not straddle heads
        if (!a.part_ml || a.att_d == 0 || (a.att_d & 7u) || a.k % a.att_d) return hipErrorInvalidValue;
        switch (a.att_splits) {
            case 1: return vx_gemv_dispatch_s<EPI, false, 1>(s, a, max_wgs, st);
            case 2: return vx_gemv_dispatch_s<EPI, false, 2>(s, a, max_wgs, st);
            case 4: return vx_gemv_dispatch_s<EPI, false, 4>(s, a, max_wgs, st);
            case 8: return vx_gemv_dispatch_s<EPI, false, 8>(s, a, max_wgs, st);
            default: return hipErrorInvalidValue;
        }
    } else {
        if (a.part_o) return hipErrorInvalidValue;
        return a.gain ? vx_gemv_dispatch_s<EPI, true, 0>(s, a, max_wgs, st)
                      : vx_gemv_dispatch_s<EPI, false, 0>(s, a, max_wgs, st);
    }
}

template <int D, int G, bool PS, int W>
hipError_t vx_attn_launch_w(const VxAttnArgs& a, hipStream_t st) {
    constexpr size_t lds = vx_attn_lds_bytes<D, G, W>();
    static bool attr_set = false;
    if (!attr_set) {
        if (hipFuncSetAttribute((const void*)vx_attn_kernel<D, G, W, PS>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        attr_set = true;
    }
    hipLaunchKernelGGL((vx_attn_kernel<D, G, W, PS>), dim3(a.splits, a.hkv, a.batch ? a.batch : 1u), dim3(64 * W), lds,
                       st, a);
    return hipGetLastError();
}

template <int D, int G, bool PS>
hipError_t vx_attn_launch_ps(const VxAttnArgs& a, hipStream_t st) {
    if constexpr (PS) {
        // 4 waves, two workgroups per CU, where 8-wave workgroups (one per CU) would need a second
        // round and 4 waves still take every 32-position chunk a split can attend in one pass (the
        // prefill chunks of short prompts: 64 rows x 8 KV heads = 512 workgroups, <= 128 positions)
        const uint32_t chunk = ((a.s_max + a.splits - 1u) / a.splits + 31u) & ~31u;
        const uint32_t span = a.max_len ? min(a.max_len, chunk) : chunk;
        const uint64_t wgs = (uint64_t)a.splits * a.hkv * (a.batch ? a.batch : 1u);
        if (wgs > 256u && span <= 4u * 32u) return vx_attn_launch_w<D, G, PS, 4>(a, st);
    }
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

hipError_t vx_launch_gemv(const VxMat& m, const VxGemvArgs& a0, int epi, uint32_t max_wgs, hipStream_t st) {
    if (m.fmt != VX_FMT_Q4) return vx_launch_gemv_f(m, a0, epi, vx_gemv_wgs(m.n_tiles, max_wgs), st);
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
        case VX_EPI_STORE: return vx_gemv_dispatch_norm<VX_EPI_STORE>(m.s, a, max_wgs, st);
        case VX_EPI_RESID: return vx_gemv_dispatch_norm<VX_EPI_RESID>(m.s, a, max_wgs, st);
        case VX_EPI_SWIGLU: return vx_gemv_dispatch_norm<VX_EPI_SWIGLU>(m.s, a, max_wgs, st);
        case VX_EPI_ARGMAX: return vx_gemv_dispatch_norm<VX_EPI_ARGMAX>(m.s, a, max_wgs, st);
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

hipError_t vx_launch_rmsnorm(const float* x, const float* w, uint32_t n, float eps, float* y, hipStream_t st) {
    hipLaunchKernelGGL(vx_rmsnorm_kernel, dim3(1), dim3(kWG), 0, st, x, w, n, eps, y);
    return hipGetLastError();
}

hipError_t vx_launch_argmax(const float* x, uint32_t n, uint32_t* out, hipStream_t st) {
    hipLaunchKernelGGL(vx_argmax_kernel, dim3(1), dim3(kWG), 0, st, x, n, out);
    return hipGetLastError();
}
