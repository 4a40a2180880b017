// vx_gemv_q4.h -- the tiled 4-bit GEMV of the batch-1 decode step, shared by the translation
// units that instantiate it per weight format (vx_kernels.hip: GGML Q4_0; vx_gemv_g64.hip: the
// reference's asymmetric group-64 format).
#pragma once
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include "vx_common.h"

typedef _Float16 vx_h2 __attribute__((ext_vector_type(2)));
typedef uint32_t vx_u32x4 __attribute__((ext_vector_type(4)));

namespace {


constexpr int kWG = 256;  // threads per workgroup (4 wave64)


// 2^x on the transcendental unit (the softmax works in the log2 domain)
__device__ __forceinline__ float vx_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float vx_h2f(uint32_t h) { return __half2float(__ushort_as_half((unsigned short)h)); }

// Code dword layout (8 weights): byte j holds element j in its low nibble and element j + 4 in
// its high nibble.
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

// Logical row j of a (possibly paired) matrix -> physical tiled row.
__device__ __forceinline__ uint32_t vx_phys_row(const VxMat& m, uint32_t j, uint32_t pair_part) {
    if (!m.paired) return j;
    const uint32_t half = (64u / m.s) / 2u;
    return (j / half) * (2u * half) + pair_part * half + (j % half);
}

// Index of block b of physical row `phys` in the tiled layout: its 16-byte code word and its
// 16-bit slot.
__device__ __forceinline__ size_t vx_tiled_off(const VxMat& m, uint32_t phys, uint32_t b) {
    const uint32_t R = 64u / m.s;
    return ((size_t)(phys / R) * m.n_iter + b / m.s) * 64u + (phys % R) * m.s + b % m.s;
}

// Weight e (0..31) of a tiled block: Q4_0 d (q - 8); group-64 fmaf(q, s, m) (src/codegen.rs:2403-2410).
template <int FMT>
__device__ __forceinline__ float vx_tiled_weight(const uint32_t (&dw)[4], int e, float d_or_s, float m) {
    const uint32_t q = vx_code_nibble(dw[e >> 3], e & 7);
    if constexpr (FMT == VX_FMT_G64) return fmaf((float)q, d_or_s, m);
    else return (float)((int)q - 8) * d_or_s;
}

}  // namespace

// =============================================================================================
// Fused 4-bit GEMV (GGML Q4_0, or the reference's asymmetric group-64 format)
// =============================================================================================
// Both formats share the tiled layout: a 16-byte code word (32 unsigned nibbles q) and a 16-bit
// slot per 32-weight block. Q4_0: the slot is the block's fp16 scale d, w = d (q - 8). Group-64
// (src/codegen.rs:2337-2370, dequant :2248-2265): a 64-weight group is blocks 2g and 2g + 1, the
// even block's slot holds the fp16 scale s and the odd block's the fp16 minimum m, w = q s + m. The
// two blocks of a group sit in lanes s and s ^ 1 of one row (S is even), which exchange their
// slots with one DPP move. With X the block's integer activations (2^-e each) and T their sum:
//   sum w x = s 2^-e sum (q - 8) X + (8 s + m) T,
// the same v_dot8 loop as Q4_0 plus one term from a per-block sum staged beside the digits.
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

// Wave tile t of a workgroup's block -> tile of the matrix (the plain GEMV: the same index).
struct VxTileIdentity {
    __device__ __forceinline__ uint32_t operator()(uint32_t t) const { return t; }
};

// bid: the workgroup's index in the GEMV's own grid (its block of tiles); tmap: the block's tile
// numbering -> the matrix's row tiles (vx_qkv_attn.hip deals one KV head's q/k/v tiles to the
// workgroups of one XCD)
template <int FMT, int S, int EPI, bool NORM, int GX, int SPL, class TM = VxTileIdentity>
__device__ __forceinline__ void vx_gemv_tiled(const VxGemvArgs& a, uint32_t bid = blockIdx.x, TM tmap = TM()) {
    static_assert(FMT == VX_FMT_Q4 || FMT == VX_FMT_G64, "tiled 4-bit formats");
    static_assert(FMT != VX_FMT_G64 || S % 2 == 0, "a group-64 pair of blocks shares one row's lanes");
    constexpr bool G64 = FMT == VX_FMT_G64;
    extern __shared__ __align__(16) unsigned char vx_smem[];
    // (the active-mask test comes after the first loads are issued: a branch here would wait for the
    // kernel arguments once for the mask and again for everything else)
    const bool active = (a.active_mask & 1ULL) != 0ULL;
    constexpr int W = kGemvWaves, kU = kGemvU, R = 64 / S, NT = 64 * W;
    const uint32_t K = a.k, nb = K >> 5, n_iter = a.n_iter;
    // activations: kXDigits planes of nb 16-byte chunks (the 4 digit dwords of one block), then the
    // blocks' unscale factors 2^-e, then (group-64) the blocks' activation sums T
    uint4* xs4 = (uint4*)vx_smem;
    float* unscale = (float*)(xs4 + (size_t)kXDigits * nb);
    float* tsum = unscale + nb;
    float* red = unscale + (G64 ? 2u : 1u) * nb;
    // the wave index is uniform: readfirstlane lets every per-wave quantity live in SGPRs
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane / S, s = lane % S;
    // workgroup blocks: workgroup b owns q or q + 1 consecutive tiles (the launcher's split of n_tiles
    // over the grid, no device division), dealt to its W waves round-robin, so every workgroup (every
    // CU) streams the same number of tiles to within one
    const uint32_t b0 = bid * a.wg_q + min(bid, a.wg_r);
    const uint32_t b1 = b0 + a.wg_q + (bid < a.wg_r ? 1u : 0u);
    const uint32_t first = b0 + (uint32_t)wave, step = (uint32_t)W;
    const uint32_t my_tiles = first < b1 ? (b1 - 1u - first) / (uint32_t)W + 1u : 0u;
    const uint32_t total = my_tiles * n_iter;

    auto row_of = [&](uint32_t t) -> uint32_t {
        if constexpr (EPI == VX_EPI_SWIGLU) return tmap(t) * (R / 2) + (r % (R / 2));  // logical j of gate/up
        else return tmap(t) * R + r;
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
    uint32_t nt = 0, ni = 0, nslot = tmap(first) * n_iter;  // next item: tile index, iteration, 64-lane slot
    auto advance = [&]() {
        if (++ni == n_iter) {
            ni = 0;
            ++nt;
            nslot = tmap(first + nt * step) * n_iter;
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
    if (!active) return;  // uniform: the whole workgroup leaves before the staging barrier

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

    // x -> LDS digit planes [d][b] (16 bytes: the digit dwords of the block's 4 code dwords): the S
    // lanes of a row read blocks b..b+S-1 of one plane at consecutive 16-byte addresses (no LDS
    // bank conflicts). Group g = values 8g..8g+7 = code dword g & 3 of block g >> 2.
    // RMSNorm (src/runtime.rs:588-601): the block-scaled integers hold x * gain at any magnitude, so
    // the stage does not wait for the sum of squares; each thread sums its values' squares while
    // staging, the staging barrier also publishes the waves' sums, and the row results take
    // 1 / rms in the epilogue (sum_k w_k x_k g_k / rms = sum_k w_k (x_k / rms) g_k).
    float ss = 0.0f;
    auto stage = [&](uint32_t g, float4 v0, float4 v1, float4 g0, float4 g1) {
        float u[8] = {v0.x, v0.y, v0.z, v0.w, v1.x, v1.y, v1.z, v1.w};
        if constexpr (NORM) {
            ss += v0.x * v0.x + v0.y * v0.y + v0.z * v0.z + v0.w * v0.w;
            ss += v1.x * v1.x + v1.y * v1.y + v1.z * v1.z + v1.w * v1.w;
            const float gg[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) u[e] = u[e] * gg[e];
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
        // across the block's four lanes by DPP quad permutations (no LDS round trip)
        m = fmaxf(m, vx_dpp<0xB1>(m));
        m = fmaxf(m, vx_dpp<0x4E>(m));
        nan += vx_dpp<0xB1>(nan);
        nan += vx_dpp<0x4E>(nan);
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
        if constexpr (G64) {
            // T: the block's integers summed exactly (|sum| <= 2^27), one rounding to fp32
            int xsum = 0;
#pragma unroll
            for (int e = 0; e < 8; ++e) xsum += (int)Y[e] - (int)kXOffset;
            xsum += __builtin_amdgcn_update_dpp(0, xsum, 0xB1, 0xF, 0xF, true);
            xsum += __builtin_amdgcn_update_dpp(0, xsum, 0x4E, 0xF, 0xF, true);
            if ((g & 3u) == 0u) tsum[g >> 2] = (float)xsum * vx_pow2f(-ex) + nan;
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
    if constexpr (NORM) {
        ss = vx_group_sum<64>(ss);
        if (lane == 0) red[wave] = ss;
    }
    __syncthreads();
    float inv_rms = 1.0f;
    if constexpr (NORM) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < W; ++w) t += red[w];
        inv_rms = 1.0f / sqrtf(t / (float)K + a.eps);
    }
    VX_TL_MARK(1);

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
        if constexpr (G64) {
            // the pair's slots: even lane (even block) s, odd lane m (padded pairs: both zero)
            const uint32_t other = (uint32_t)__builtin_amdgcn_update_dpp(0, (int)sbuf[u], 0xB1, 0xF, 0xF, true);
            const bool odd = (lane & 1) != 0;
            const float sc = vx_h2f(odd ? other : sbuf[u]), mn = vx_h2f(odd ? sbuf[u] : other);
            acc = fmaf(sc * unscale[b], dot, acc);
            acc = fmaf(fmaf(8.0f, sc, mn), tsum[b], acc);
        } else {
            acc = fmaf(vx_h2f(sbuf[u]) * unscale[b], dot, acc);
        }
        if (++ci == n_iter) {
            acc = vx_group_sum<S>(acc);
            if constexpr (NORM) acc *= inv_rms;
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

template <int S, int EPI, bool NORM, int GX, int SPL>
__global__ __launch_bounds__(64 * kGemvWaves) void vx_gemv_q4_kernel(VxGemvArgs a) {
    VX_TL_BEGIN(a, blockIdx.x);
    vx_gemv_tiled<VX_FMT_Q4, S, EPI, NORM, GX, SPL>(a);
}

template <int S, int EPI, bool NORM, int GX, int SPL>
__global__ __launch_bounds__(64 * kGemvWaves) void vx_gemv_g64_kernel(VxGemvArgs a) {
    vx_gemv_tiled<VX_FMT_G64, S, EPI, NORM, GX, SPL>(a);
}

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

// The kernel of a format (only the referenced one is instantiated).
template <int FMT, int S, int EPI, bool NORM, int GX, int SPL>
constexpr auto vx_gemv_kernel_of() {
    if constexpr (FMT == VX_FMT_G64) return &vx_gemv_g64_kernel<S, EPI, NORM, GX, SPL>;
    else return &vx_gemv_q4_kernel<S, EPI, NORM, GX, SPL>;
}

template <int FMT, int S, int EPI, bool NORM, int GX, int SPL>
hipError_t vx_gemv_launch_t(const VxGemvArgs& a, uint32_t max_wgs, hipStream_t st) {
    constexpr int W = kGemvWaves;
    constexpr auto kern = vx_gemv_kernel_of<FMT, S, EPI, NORM, GX, SPL>();
    const uint32_t nb = a.k >> 5;
    // K <= 32768: at most 102,464 bytes (106,560 with the group-64 sums)
    const size_t lds = (size_t)nb * (16u * kXDigits + (FMT == VX_FMT_G64 ? 8u : 4u)) + 64u;
    static size_t attr_lds = 64u * 1024u;
    if (lds > attr_lds) {
        if (hipFuncSetAttribute((const void*)kern,
                                hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        attr_lds = lds;
    }
    const uint32_t wgs = vx_gemv_wgs(a.n_tiles, max_wgs);
    VxGemvArgs ag = a;
    ag.wg_q = a.n_tiles / wgs;
    ag.wg_r = a.n_tiles % wgs;
    hipLaunchKernelGGL(kern, dim3(wgs), dim3(64 * W), lds, st, ag);
    return hipGetLastError();
}

// x register groups per thread: ceil(K / 8 / threads) rounded up to 1, 2 or 4 (larger K loops;
// merged attention partials must fit the registers)
template <int FMT, int S, int EPI, bool NORM, int SPL>
hipError_t vx_gemv_dispatch_gx(const VxGemvArgs& a, uint32_t max_wgs, hipStream_t st) {
    const uint32_t per = ((a.k >> 3) + 64u * kGemvWaves - 1u) / (64u * kGemvWaves);
    if (per <= 1u) return vx_gemv_launch_t<FMT, S, EPI, NORM, 1, SPL>(a, max_wgs, st);
    if (per <= 2u) return vx_gemv_launch_t<FMT, S, EPI, NORM, 2, SPL>(a, max_wgs, st);
    if (SPL > 0 && per > 4u) return hipErrorInvalidValue;
    return vx_gemv_launch_t<FMT, S, EPI, NORM, 4, SPL>(a, max_wgs, st);
}

template <int FMT, int EPI, bool NORM, int SPL>
hipError_t vx_gemv_dispatch_s(uint32_t s, const VxGemvArgs& a, uint32_t max_wgs, hipStream_t st) {
    switch (s) {
        case 4: return vx_gemv_dispatch_gx<FMT, 4, EPI, NORM, SPL>(a, max_wgs, st);
        case 8: return vx_gemv_dispatch_gx<FMT, 8, EPI, NORM, SPL>(a, max_wgs, st);
        case 16: return vx_gemv_dispatch_gx<FMT, 16, EPI, NORM, SPL>(a, max_wgs, st);
        case 32: return vx_gemv_dispatch_gx<FMT, 32, EPI, NORM, SPL>(a, max_wgs, st);
        case 64:
            if constexpr (EPI != VX_EPI_SWIGLU) return vx_gemv_dispatch_gx<FMT, 64, EPI, NORM, SPL>(a, max_wgs, st);
            return hipErrorInvalidValue;
        default: return hipErrorInvalidValue;
    }
}

template <int FMT, int EPI>
hipError_t vx_gemv_dispatch_norm(uint32_t s, const VxGemvArgs& a, uint32_t max_wgs, hipStream_t st) {
    if constexpr (EPI == VX_EPI_RESID) {
        if (a.gain) return hipErrorInvalidValue;  // the residual epilogue takes raw activations
        if (!a.part_o) return vx_gemv_dispatch_s<FMT, EPI, false, 0>(s, a, max_wgs, st);
        // o_proj over split-K attention partials: 8-element groups must not straddle heads
        if (!a.part_ml || a.att_d == 0 || (a.att_d & 7u) || a.k % a.att_d) return hipErrorInvalidValue;
        switch (a.att_splits) {
            case 1: return vx_gemv_dispatch_s<FMT, EPI, false, 1>(s, a, max_wgs, st);
            case 2: return vx_gemv_dispatch_s<FMT, EPI, false, 2>(s, a, max_wgs, st);
            case 4: return vx_gemv_dispatch_s<FMT, EPI, false, 4>(s, a, max_wgs, st);
            case 8: return vx_gemv_dispatch_s<FMT, EPI, false, 8>(s, a, max_wgs, st);
            default: return hipErrorInvalidValue;
        }
    } else {
        if (a.part_o) return hipErrorInvalidValue;
        return a.gain ? vx_gemv_dispatch_s<FMT, EPI, true, 0>(s, a, max_wgs, st)
                      : vx_gemv_dispatch_s<FMT, EPI, false, 0>(s, a, max_wgs, st);
    }
}

// The tiled GEMV of matrix m in format FMT (VX_FMT_Q4 or VX_FMT_G64).
template <int FMT>
hipError_t vx_launch_gemv_tiled(const VxMat& m, const VxGemvArgs& a0, int epi, uint32_t max_wgs, hipStream_t st) {
    VxGemvArgs a = a0;
    a.codes = m.codes;
    a.scales = m.scales;
    a.n = m.n;
    a.k = m.k;
    a.n_tiles = m.n_tiles;
    a.n_iter = m.n_iter;
    if (m.k == 0 || (m.k & (FMT == VX_FMT_G64 ? 63u : 31u)) != 0) return hipErrorInvalidValue;
    if (FMT == VX_FMT_G64 && (m.s & 1u)) return hipErrorInvalidValue;
    if ((epi == VX_EPI_SWIGLU) != (m.paired != 0)) return hipErrorInvalidValue;
    switch (epi) {
        case VX_EPI_STORE: return vx_gemv_dispatch_norm<FMT, VX_EPI_STORE>(m.s, a, max_wgs, st);
        case VX_EPI_RESID: return vx_gemv_dispatch_norm<FMT, VX_EPI_RESID>(m.s, a, max_wgs, st);
        case VX_EPI_SWIGLU: return vx_gemv_dispatch_norm<FMT, VX_EPI_SWIGLU>(m.s, a, max_wgs, st);
        case VX_EPI_ARGMAX: return vx_gemv_dispatch_norm<FMT, VX_EPI_ARGMAX>(m.s, a, max_wgs, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace
