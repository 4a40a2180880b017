// vx_qkv_attn.hip -- the single-sequence decode step's QKV GEMV and decode attention in one launch.
//
// The reference runs them as two kernels (src/codegen.rs:1104-2582; the q/k/v projection, then
// RoPE, the KV append and attention, src/runtime.rs:745-831). Here one grid holds both:
//   * GEMV workgroups: the RMSNorm-prologue Q4_0 GEMV of vx_gemv_q4.h (STORE epilogue, bias),
//     with the rows of KV head g (its G q heads, its k and its v) dealt to workgroups b = g mod 8,
//     which all run on one XCD: the dispatcher deals a launch's workgroups to the 8 XCDs
//     round-robin, workgroup b to XCD (b + o) mod 8 with o where the previous launch left off
//     (checked on each device before the library uses this kernel, vx_xcd_roundrobin_ok, and by
//     every launch, below). A workgroup stores its rows, waits for their acknowledgements, then adds
//     1 + 2^(8 + 7 x) to its head's 64-bit counter (x: its XCD), once.
//   * Attention workgroups (the first hkv x A of the grid, so they are dispatched first): split sp
//     of KV head g, on the same XCD. Each reads the position, prefetches its first K/V chunk and
//     waits for the head's counter to count its P GEMV workgroups, all P on its own XCD (the 7-bit
//     field of its XCD holds P; else it sets error bit 1); the head's q/k/v rows are then
//     in this XCD's L2 (plain stores, acknowledged before the count), and the workgroup reads them
//     there, applies RoPE, appends the new K/V row (split 0) and attends over its 32-position chunks
//     (chunk c belongs to split c % A), writing the (m, l, o) partials the o_proj GEMV merges.
// This removes one kernel boundary per layer and lets the attention's first loads overlap the GEMV.
// No workgroup waits on anything but its own head's GEMV workgroups, which wait on nothing, so the
// wait always ends; it is bounded anyway (an expired wait sets the error word and writes no
// partials).
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <cstdio>
#include <mutex>
#include <string>

#include "vx_common.h"
#include "vx_gemv_q4.h"

namespace {

typedef __bf16 vq_bf8 __attribute__((ext_vector_type(8)));
typedef float vq_af4 __attribute__((ext_vector_type(4)));

constexpr int kQaWaves = 8;               // both roles: 8-wave workgroups
constexpr uint32_t kQaSpinMax = 1u << 18; // polls before a wait is declared expired (0.1-0.3 s)

__device__ __forceinline__ uint32_t vq_xcc_id() {
    uint32_t id;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(id));
    return id & 15u;
}

// Rotate-half RoPE of one pair (src/runtime.rs:761-764), unfused like the reference's Rust.
__device__ __forceinline__ float2 vq_rope_pair(float x1, float x2, float2 cs) {
#pragma clang fp contract(off)
    return make_float2(x1 * cs.x - x2 * cs.y, x2 * cs.x + x1 * cs.y);
}

// KV head g's rows of the fused [q; k; v] matrix, in tiles of R rows: its G q heads, then its k
// head, then its v head.
struct VxQkvTileMap {
    uint32_t tq, tk, qb, kb, vb;
    __device__ __forceinline__ uint32_t operator()(uint32_t t) const {
        return t < tq ? qb + t : (t < tq + tk ? kb + (t - tq) : vb + (t - tq - tk));
    }
};

template <int D, int G>
constexpr int vq_hrows() { return G <= 4 ? 4 : 8; }

template <int D, int G>
constexpr size_t vq_attn_lds() {
    return (size_t)3 * 16 * (D + 8) * 2 + (size_t)2 * D * 2 + (size_t)4 * 32 * 4 + 16 * 4 +
           (size_t)4 * vq_hrows<D, G>() * D * 4;
}

// Attention workgroup (kv head g, split sp): 4 wave pairs; the two waves of a pair take the same
// 32-position chunks (both form the chunk's scores), each accumulating P.V over one half of the
// dimensions, which keeps a wave within 128 VGPRs (two 8-wave workgroups per CU for the GEMV role).
// The arithmetic is vx_attn_kernel's: scores S^T = K Q^T on v_mfma_f32_16x16x32_bf16 with q as
// three exact bf16 terms (fp32 products), online softmax in the log2 domain, P as two bf16 terms.
template <int D, int G>
__device__ __forceinline__ void vq_attention(const VxQkvAttnArgs& f, uint32_t g, uint32_t sp, unsigned char* smem) {
    constexpr int W = kQaWaves, NPAIR = W / 2, HALF = D / 2, NT = 64 * W, NC = D / 32, NBH = D / 32;
    constexpr int HR = vq_hrows<D, G>(), QP = D + 8;
    constexpr float kLog2e = 1.4426950408889634f;
    static_assert(G >= 1 && G <= 8 && D % 64 == 0, "q heads in MFMA columns 0..G-1");
    const VxAttnArgs& a = f.at;
    uint16_t* qt_s = (uint16_t*)smem;          // [3][16][QP] bf16 terms of the pre-scaled q
    uint16_t* kn_s = qt_s + 3 * 16 * QP;       // the new position's k (RoPE'd) and v, bf16
    uint16_t* vn_s = kn_s + D;
    float* ml_s = (float*)(vn_s + D);          // [pair][2][16]: m, l per head
    float* sn_s = ml_s + NPAIR * 32;           // [16]: q_h . k_new
    float* o_s = sn_s + 16;                    // [pair][HR][D]
    __shared__ uint32_t s_go;
    const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int pair = wave >> 1, hv = wave & 1, col = lane & 15, grp = lane >> 4;
    const uint32_t A = a.splits;
    uint16_t* Kc = a.kv + (size_t)g * a.s_cap * D;
    uint16_t* Vc = a.kv + ((size_t)a.hkv + g) * a.s_cap * D;
    auto uniform = [](uint32_t v) { return (uint32_t)__builtin_amdgcn_readfirstlane(v); };

    // ---- the position, the RoPE row of the step, then the first chunk of this pair ----
    const uint64_t step = __hip_atomic_load((uint64_t*)&a.state[0].step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    constexpr int NP = (G + 1) * HALF, RP = (NP + NT - 1) / NT;
    float2 rcs[RP];
#pragma unroll
    for (int i = 0; i < RP; ++i) rcs[i] = a.rope_cur[min(tid + i * NT, NP - 1) % HALF];
    if ((a.active_mask & 1ULL) == 0ULL) return;  // uniform: the GEMV workgroups skip this step too
    const uint32_t pos = uniform(step < (uint64_t)a.s_max ? (uint32_t)step : a.s_max - 1u);
    const uint32_t nch = (pos + 31u) >> 5;        // chunks holding cached positions [0, pos)
    const uint32_t last_blk = a.s_cap / 32u - 1u; // clamp: every load stays inside the planes

    vq_bf8 kf[2][NC], vf[NBH];
    auto load_chunk = [&](uint32_t c) {
        const uint32_t cb = 32u * min(c, last_blk);
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int cc = 0; cc < NC; ++cc)
                kf[b][cc] = *(const vq_bf8*)(Kc + (size_t)(cb + 16u * b + (uint32_t)col) * D + 32 * cc + 8 * grp);
        const uint16_t* vb = Vc + (size_t)(cb >> 5) * D * 32;
#pragma unroll
        for (int nb = 0; nb < NBH; ++nb)
            vf[nb] = *(const vq_bf8*)(vb + (HALF * hv + 16 * nb + col) * 32 + 8 * grp);
    };
    uint32_t c = sp + A * (uint32_t)pair;  // this pair's chunks: c, c + 4 A, ...
    if (c < nch) load_chunk(c);  // (uniform; a pair with no chunk reads nothing)

    // ---- wait for the head's GEMV workgroups (their q/k/v rows are then in this XCD's L2) ----
    uint64_t* cnt = (uint64_t*)(f.sync + (size_t)g * 64u);
    uint32_t* done = f.sync + ((size_t)a.hkv + g) * 64u;
    if (tid == 0) {
        uint32_t n = 0;
        uint64_t v = 0;
        while (((v = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) & 0xFFu) < f.p &&
               ++n < kQaSpinMax)
            __builtin_amdgcn_s_sleep(1);
        const bool ok = n < kQaSpinMax;
        if (ok) {
            // every count from this XCD, or the rows are not all in its L2
            if (((v >> (8u + 7u * vq_xcc_id())) & 0x7Fu) != f.p) atomicOr(f.sync + 2u * a.hkv * 64u, 1u);
            // the head's last split to get here re-arms both counters for the next launch (every
            // GEMV workgroup has counted, every split has stopped reading the counter)
            if (__hip_atomic_fetch_add(done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == A - 1u) {
                __hip_atomic_store(cnt, 0ull, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_store(done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
        } else {
            atomicOr(f.sync + 2u * a.hkv * 64u, 2u);
        }
        s_go = ok ? 1u : 0u;
    }
    __syncthreads();
    VX_TL_MARK(1);
    if (!s_go) return;

    // ---- q heads and the new k/v of this head, RoPE, bf16 staging ----
    const float* q = a.qkv + (size_t)g * G * D;
    const float* k = a.qkv + (size_t)a.hq * D + (size_t)g * D;
    const float* v = a.qkv + ((size_t)a.hq + a.hkv) * D + (size_t)g * D;
    float r1[RP], r2[RP];
#pragma unroll
    for (int i = 0; i < RP; ++i) {
        const int p = min(tid + i * NT, NP - 1);
        const int hh = p / HALF, j = p % HALF;
        const float* src = hh < G ? q + (size_t)hh * D : k;
        r1[i] = src[j];
        r2[i] = src[j + HALF];
    }
    const float vnew = v[min(tid, D - 1)];
    const float qscale = a.scale * kLog2e;  // scores in the log2 domain
    for (int i = tid; i < 3 * (16 - G) * QP / 2; i += NT) {  // q rows G..15 of every term: zero
        const int t = i / ((16 - G) * QP / 2), r = i % ((16 - G) * QP / 2);
        ((uint32_t*)(qt_s + (t * 16 + G) * QP))[r] = 0u;
    }
#pragma unroll
    for (int i = 0; i < RP; ++i) {
        const int p = tid + i * NT;
        const float2 o = vq_rope_pair(r1[i], r2[i], rcs[i]);
        if (p < NP) {
            const int hh = p / HALF, j = p % HALF;
            if (hh < G) {
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
    if (sp == 0) {  // the bf16 K/V append (read by later steps only: this step folds it in below)
        const uint16_t* vblk = Vc + (size_t)(pos >> 5) * D * 32 + vx_vslot(pos & 31u);
        for (int d = tid; d < D; d += NT) {
            Kc[(size_t)pos * D + d] = kn_s[d];
            ((uint16_t*)vblk)[d * 32] = vn_s[d];
        }
    }
    const bool has_new = (pos >> 5) % A == sp;  // the split owning pos's chunk adds the new position
    if (has_new && wave == W - 1) {
        for (int h = 0; h < G; ++h) {
            float sn = 0.0f;
#pragma unroll
            for (int d = lane; d < D; d += 64) {
                float qv = 0.0f;
#pragma unroll
                for (int t = 0; t < 3; ++t) qv += __uint_as_float((uint32_t)qt_s[(t * 16 + h) * QP + d] << 16);
                sn += qv * __uint_as_float((uint32_t)kn_s[d] << 16);
            }
#pragma unroll
            for (int off = 32; off > 0; off >>= 1) sn += __shfl_xor(sn, off);
            if (lane == 0) sn_s[h] = sn;
        }
    }

    // ---- this pair's chunks ----
    float m_run = -INFINITY, l_run = 0.0f;
    vq_af4 o_acc[NBH];
#pragma unroll
    for (int nb = 0; nb < NBH; ++nb) o_acc[nb] = vq_af4{0.f, 0.f, 0.f, 0.f};
    const uint32_t cstep = 4u * A;
    for (; c < nch; c += cstep) {
        const uint32_t cb = 32u * c;
        vq_af4 sc[2] = {vq_af4{0.f, 0.f, 0.f, 0.f}, vq_af4{0.f, 0.f, 0.f, 0.f}};
        // the q operands are read from LDS at each use (an opaque base per chunk: held across the
        // loop they would take 48 more VGPRs)
        uint32_t qoff = (uint32_t)(col * QP + 8 * grp) * 2u;
        asm volatile("" : "+v"(qoff));
        const unsigned char* qb = (const unsigned char*)qt_s + qoff;
#pragma unroll
        for (int cc = 0; cc < NC; ++cc)
#pragma unroll
            for (int t = 0; t < 3; ++t) {
                const vq_bf8 qop = *(const vq_bf8*)(qb + ((t * 16) * QP + 32 * cc) * 2);
                sc[0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[0][cc], qop, sc[0], 0, 0, 0);
                sc[1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[1][cc], qop, sc[1], 0, 0, 0);
            }
        float pr[8];
        float mx = -INFINITY;
#pragma unroll
        for (int b = 0; b < 2; ++b)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const uint32_t p = cb + 16u * b + 4u * grp + i;
                pr[4 * b + i] = p < pos ? sc[b][i] : -INFINITY;
                mx = fmaxf(mx, pr[4 * b + i]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 16));
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = m_run == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_run - m_new);
        float lt = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            pr[e] = pr[e] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(pr[e] - m_new);
            lt += pr[e];
        }
        l_run = l_run * alpha + lt;
        m_run = m_new;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float ai = __shfl(alpha, 4 * grp + i);
#pragma unroll
            for (int nb = 0; nb < NBH; ++nb) o_acc[nb][i] *= ai;
        }
        // P as two bf16 terms (truncations of the exact remainders)
        vq_bf8 pop[2];
        {
            float rr[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) rr[e] = pr[e];
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                uint32_t w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const uint32_t x0 = __float_as_uint(rr[2 * e]) & 0xFFFF0000u, x1 = __float_as_uint(rr[2 * e + 1]) & 0xFFFF0000u;
                    w[e] = (x0 >> 16) | x1;
                    rr[2 * e] -= __uint_as_float(x0);
                    rr[2 * e + 1] -= __uint_as_float(x1);
                }
                pop[t] = __builtin_bit_cast(vq_bf8, w);
            }
        }
#pragma unroll
        for (int nb = 0; nb < NBH; ++nb)
#pragma unroll
            for (int t = 0; t < 2; ++t) o_acc[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pop[t], vf[nb], o_acc[nb], 0, 0, 0);
        if (c + cstep < nch) load_chunk(c + cstep);
    }

    VX_TL_MARK(3);
    // ---- merge the pairs (and the new position) into this split's partial ----
    l_run += __shfl_xor(l_run, 16);
    l_run += __shfl_xor(l_run, 32);
    if (hv == 0 && lane < 16) {
        ml_s[pair * 32 + lane] = m_run;
        ml_s[pair * 32 + 16 + lane] = l_run;
    }
    if (grp < HR / 4) {
#pragma unroll
        for (int nb = 0; nb < NBH; ++nb)
#pragma unroll
            for (int i = 0; i < 4; ++i) o_s[(pair * HR + 4 * grp + i) * D + HALF * hv + 16 * nb + col] = o_acc[nb][i];
    }
    __syncthreads();
    VX_TL_MARK(4);
    for (int idx = tid; idx < G * D; idx += NT) {
        const int h = idx / D, d = idx % D;
        const float sn = has_new ? sn_s[h] : -INFINITY;
        float M = sn;
#pragma unroll
        for (int p = 0; p < NPAIR; ++p) M = fmaxf(M, ml_s[p * 32 + h]);
        float o = 0.0f, l = 0.0f;
        if (has_new) {
            const float wt = __builtin_amdgcn_exp2f(sn - M);
            o = wt * __uint_as_float((uint32_t)vn_s[d] << 16);
            l = wt;
        }
#pragma unroll
        for (int p = 0; p < NPAIR; ++p) {
            const float mp = ml_s[p * 32 + h];
            const float wt = mp == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mp - M);
            o += wt * o_s[(p * HR + h) * D + d];
            l += wt * ml_s[p * 32 + 16 + h];
        }
        const size_t hs = ((size_t)g * G + (size_t)h) * A + sp;
        a.part_o[hs * D + d] = o;
        if (d == 0) {
            a.part_ml[hs * 2] = M;
            a.part_ml[hs * 2 + 1] = l;
        }
    }
}

}  // namespace

template <int S, int GX, int G>
__global__ __launch_bounds__(64 * kQaWaves) __attribute__((amdgpu_waves_per_eu(4)))
void vx_qkv_attn_kernel(VxQkvAttnArgs f) {
    constexpr int D = 128;
    extern __shared__ __align__(16) unsigned char vx_smem[];
    VX_TL_BEGIN(f.g, blockIdx.x);
    const uint32_t bid = blockIdx.x;
    if (bid < f.na) {  // attention: split (bid / 8) % A of head 8 ((bid / 8) / A) + bid % 8
        const uint32_t i = bid >> 3, A = f.at.splits;
        vq_attention<D, G>(f, (bid & 7u) + 8u * (i / A), i % A, vx_smem);
    } else {
        // GEMV workgroup j of head g, on the head's XCD (na is a multiple of 8)
        const uint32_t b = bid - f.na, i = b >> 3;
        const uint32_t g = (b & 7u) + 8u * (i / f.p), j = i % f.p;
        const VxQkvTileMap tm{f.tq, f.tk, g * f.tq, f.k_base + g * f.tk, f.v_base + g * f.tk};
        vx_gemv_tiled<VX_FMT_Q4, S, VX_EPI_STORE, true, GX, 0>(f.g, j, tm);
        if ((f.g.active_mask & 1ULL) != 0ULL) {
            // this workgroup's rows are stored: wait for every wave's store acknowledgements (from
            // this XCD's L2), then count the workgroup in once
            __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
            __syncthreads();
            if (threadIdx.x == 0)
                __hip_atomic_fetch_add((uint64_t*)(f.sync + (size_t)g * 64u), 1ull + (1ull << (8u + 7u * vq_xcc_id())),
                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
    }
}

// Records the XCD each workgroup ran on.
__global__ __launch_bounds__(64) void vx_xcc_probe_kernel(uint32_t* out) {
    if (threadIdx.x == 0) out[blockIdx.x] = vq_xcc_id();
}

namespace {

template <int S, int GX, int G>
hipError_t vq_launch(const VxQkvAttnArgs& f, uint32_t grid, hipStream_t st) {
    constexpr auto kern = &vx_qkv_attn_kernel<S, GX, G>;
    const size_t lds_g = (size_t)(f.g.k >> 5) * (16u * kXDigits + 4u) + 64u;
    const size_t lds_a = vq_attn_lds<128, G>();
    const size_t lds = lds_g > lds_a ? lds_g : lds_a;
    static size_t attr_lds = 64u * 1024u;
    if (lds > attr_lds) {
        if (hipFuncSetAttribute((const void*)kern, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) {
            (void)hipGetLastError();
            return hipErrorInvalidValue;
        }
        attr_lds = lds;
    }
    hipLaunchKernelGGL(kern, dim3(grid), dim3(64 * kQaWaves), lds, st, f);
    return hipGetLastError();
}

template <int S, int G>
hipError_t vq_launch_gx(const VxQkvAttnArgs& f, uint32_t grid, hipStream_t st) {
    const uint32_t per = ((f.g.k >> 3) + 64u * kQaWaves - 1u) / (64u * kQaWaves);
    if (per <= 1u) return vq_launch<S, 1, G>(f, grid, st);
    if (per <= 2u) return vq_launch<S, 2, G>(f, grid, st);
    return vq_launch<S, 4, G>(f, grid, st);
}

template <int G>
hipError_t vq_launch_s(uint32_t s, const VxQkvAttnArgs& f, uint32_t grid, hipStream_t st) {
    switch (s) {
        case 16: return vq_launch_gx<16, G>(f, grid, st);
        case 32: return vq_launch_gx<32, G>(f, grid, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

bool vx_qkv_attn_supported(const VxMat& m, uint32_t hq, uint32_t hkv, uint32_t d) {
    if (m.fmt != VX_FMT_Q4 || m.paired || d != 128 || hkv == 0 || hkv % 8u || hq % hkv) return false;
    const uint32_t G = hq / hkv, R = 64u / m.s;
    if (G != 4 && G != 8) return false;
    if (m.s != 16 && m.s != 32) return false;
    return d % R == 0 && m.n == (hq + 2u * hkv) * d && m.k <= 32768u;
}

// The fused launch: f.g carries the QKV GEMV's arguments (x, gain, eps, bias, y = the q/k/v
// buffer, active_mask), f.at the attention's (qkv = f.g.y, kv, rope_cur, state, part_o, part_ml,
// hq, hkv, s_max, s_cap, scale, splits = A <= 8), f.sync the zeroed words of the counters.
hipError_t vx_launch_qkv_attn(const VxMat& m, const VxQkvAttnArgs& f0, uint32_t p, hipStream_t st) {
    const VxAttnArgs& a = f0.at;
    if (!vx_qkv_attn_supported(m, a.hq, a.hkv, 128u) || !f0.sync || !a.state || !a.rope_cur || !a.part_o ||
        !a.part_ml || a.splits == 0 || a.splits > 8 || p == 0 || a.s_max == 0 || (a.s_cap & 31u) || a.s_cap < a.s_max ||
        a.qkv != f0.g.y || !f0.g.gain)
        return hipErrorInvalidValue;
    const uint32_t G = a.hq / a.hkv, R = 64u / m.s;
    VxQkvAttnArgs f = f0;
    f.g.codes = m.codes;
    f.g.scales = m.scales;
    f.g.n = m.n;
    f.g.k = m.k;
    f.g.n_tiles = m.n_tiles;
    f.g.n_iter = m.n_iter;
    f.tq = G * 128u / R;
    f.tk = 128u / R;
    f.k_base = a.hq * 128u / R;
    f.v_base = (a.hq + a.hkv) * 128u / R;
    const uint32_t th = f.tq + 2u * f.tk;  // tiles per KV head
    f.p = p;
    f.g.wg_q = th / p;
    f.g.wg_r = th % p;
    f.na = a.hkv * a.splits;
    const uint32_t grid = f.na + a.hkv * p;
    return G == 4 ? vq_launch_s<4>(m.s, f, grid, st) : vq_launch_s<8>(m.s, f, grid, st);
}

// Workgroup b of a launch runs on XCD (b + o) % 8, o fixed per launch (256 CUs in 8 XCDs, dealt
// round-robin from where the previous launch left off): checked on the current device over several
// grid sizes, synchronously (never under graph capture), once per device.
bool vx_xcd_roundrobin_ok() {
    static std::mutex mu;
    static int known[64];  // 0 unknown, 1 yes, 2 no (a failed HIP call leaves it unknown)
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return false;
    std::lock_guard<std::mutex> lock(mu);
    if (known[dev]) return known[dev] == 1;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, dev) != hipSuccess) return false;
    if (std::string(p.gcnArchName).rfind("gfx950", 0) != 0 || p.multiProcessorCount != 256) {
        std::fprintf(stderr, "velox_hip: device %s with %d CUs: the fused QKV + attention launch stays off\n",
                     p.gcnArchName, p.multiProcessorCount);
        known[dev] = 2;
        return false;
    }
    constexpr uint32_t kMax = 2048;
    uint32_t* d = nullptr;
    if (hipMalloc((void**)&d, kMax * 4) != hipSuccess) {
        std::fprintf(stderr, "velox_hip: XCD check: hipMalloc failed\n");
        return false;
    }
    static uint32_t h[kMax];
    bool api_ok = true, mapped = true;
    for (uint32_t grid : {8u, 64u, 416u, 600u, 2048u}) {
        (void)hipGetLastError();  // an earlier call's error is not this launch's
        hipLaunchKernelGGL(vx_xcc_probe_kernel, dim3(grid), dim3(64), 0, 0, d);
        const hipError_t e1 = hipGetLastError();
        const hipError_t e2 = e1 == hipSuccess ? hipMemcpy(h, d, grid * 4, hipMemcpyDeviceToHost) : e1;
        if (e2 != hipSuccess) {
            std::fprintf(stderr, "velox_hip: XCD check: launch/copy failed (%d)\n", (int)e2);
            api_ok = false;
            break;
        }
        for (uint32_t b = 0; b < grid && mapped; ++b) {
            mapped = h[b] == ((h[0] + b) & 7u);
            if (!mapped)
                std::fprintf(stderr,
                             "velox_hip: workgroup %u of a %u-workgroup launch ran on XCD %u, not %u: the fused QKV + "
                             "attention launch stays off on this device\n",
                             b, grid, h[b], (h[0] + b) & 7u);
        }
        if (!mapped) break;
    }
    (void)hipFree(d);
    if (!api_ok) return false;
    known[dev] = mapped ? 1 : 2;
    return mapped;
}
