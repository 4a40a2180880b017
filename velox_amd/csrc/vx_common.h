// vx_common.h -- types and helpers shared by the HIP kernels (device) and the planner/runner (host).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "velox_hip.h"

#define VX_HD __host__ __device__ __forceinline__

// ---------------------------------------------------------------------------------------------
// Seeded synthetic-model recipe (counter-based, identical on host and device):
//   stream = mix64(seed ^ mix64(tag + C0)); h(i) = mix64(stream + (i+1) * golden)
//   normal(i) = (float)(2 * sum of the eight 16-bit words of h(2i), h(2i+1) - 524280) * coef
// An Irwin-Hall(8) approximation of N(0, sigma) computed with one exact int->float conversion and
// one IEEE multiply, so host and device produce the same bits.
// ---------------------------------------------------------------------------------------------
VX_HD uint64_t vx_mix64(uint64_t z) {
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
    return z ^ (z >> 31);
}
VX_HD uint64_t vx_stream(uint64_t seed, uint64_t tag) { return vx_mix64(seed ^ vx_mix64(tag + 0x632BE59BD9B4E019ULL)); }
VX_HD uint64_t vx_hash(uint64_t stream, uint64_t idx) { return vx_mix64(stream + (idx + 1ULL) * 0x9E3779B97F4A7C15ULL); }
VX_HD int32_t vx_normal_int(uint64_t stream, uint64_t idx) {
    const uint64_t a = vx_hash(stream, 2ULL * idx), b = vx_hash(stream, 2ULL * idx + 1ULL);
    const int64_t s = (int64_t)(a & 0xFFFF) + (int64_t)((a >> 16) & 0xFFFF) + (int64_t)((a >> 32) & 0xFFFF) +
                      (int64_t)(a >> 48) + (int64_t)(b & 0xFFFF) + (int64_t)((b >> 16) & 0xFFFF) +
                      (int64_t)((b >> 32) & 0xFFFF) + (int64_t)(b >> 48);
    return (int32_t)(2 * s - 524280);
}
VX_HD uint32_t vx_uniform_u32(uint64_t stream, uint64_t idx, uint32_t n) {
    return (uint32_t)(((vx_hash(stream, idx) >> 32) * (uint64_t)n) >> 32);
}
inline float vx_normal_coef(float sigma) { return (float)((double)sigma / (131072.0 * 0.81649658092772603)); }
// Value idx of a seeded N(mean, sigma) stream (coef = vx_normal_coef(sigma)), unfused.
VX_HD float vx_normal_value(uint64_t stream, uint64_t idx, float coef, float mean) {
#pragma clang fp contract(off)
    return mean + (float)vx_normal_int(stream, idx) * coef;
}
VX_HD uint64_t vx_tag(uint32_t layer, uint32_t kind) { return (uint64_t)layer * 256ULL + kind; }
#define VX_TAG_PROMPT 16u
#define VX_TAG_KV_K 17u
#define VX_TAG_KV_V 18u

// IEEE fp32 -> fp16 bits, round to nearest even (integer form, host == device).
VX_HD uint16_t vx_f32_to_f16_bits(float f) {
    const uint32_t x = __builtin_bit_cast(uint32_t, f);
    const uint32_t sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax >= 0x7F800000u) return (uint16_t)(sign | (ax == 0x7F800000u ? 0x7C00u : (0x7E00u | ((ax >> 13) & 0x3FFu))));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) {
        if (ax < 0x33000000u) return (uint16_t)sign;
        const uint32_t e = ax >> 23, mant = (ax & 0x7FFFFFu) | 0x800000u, sh = 126u - e;
        uint32_t q = mant >> sh;
        const uint32_t rem = mant & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) q++;
        return (uint16_t)(sign | q);
    }
    uint32_t h = (((ax >> 23) - 112u) << 10) | ((ax & 0x7FFFFFu) >> 13);
    const uint32_t rem = ax & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
    return (uint16_t)(sign | h);
}
VX_HD float vx_f16_bits_to_f32(uint16_t h) {
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16, e = ((uint32_t)h >> 10) & 0x1Fu;
    uint32_t m = (uint32_t)h & 0x3FFu, x;
    if (e == 0) {
        if (m == 0) {
            x = sign;
        } else {
            uint32_t sh = 0;
            while (!(m & 0x400u)) { m <<= 1; sh++; }
            x = sign | ((113u - sh) << 23) | ((m & 0x3FFu) << 13);
        }
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    return __builtin_bit_cast(float, x);
}
VX_HD uint16_t vx_f32_to_bf16_bits(float f) {
    uint32_t x = __builtin_bit_cast(uint32_t, f);
    if ((x & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7FFFu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}
VX_HD float vx_bf16_bits_to_f32(uint16_t h) { return __builtin_bit_cast(float, (uint32_t)h << 16); }

// V cache blocks hold 32 positions dimension-major; slot of position r (0..31) of a block: the P.V
// MFMA's lane group j supplies, as its 8 K-elements, positions 4j..4j+3 and 16+4j..16+4j+3 (where
// the K.Q^T MFMA leaves the scores), so slot 8j + 4 half + i holds position 16 half + 4j + i.
VX_HD uint32_t vx_vslot(uint32_t r) { return 8u * ((r & 15u) >> 2) + 4u * (r >> 4) + (r & 3u); }

// ---------------------------------------------------------------------------------------------
// Device-side views
// ---------------------------------------------------------------------------------------------
// Weight formats of a VxMat: GGML Q4_0 or the reference's group-64 format (quant_mode 2) in the
// tiled layout, or the reference's unquantized rows (quant_mode 0 fp32, 1 fp16), row-major
// [rows][k] (paired: n gate rows, then n up rows), n_tiles = ceil(n / 4) tiles of 4 logical rows,
// no scales.
enum { VX_FMT_Q4 = 0, VX_FMT_F32 = 1, VX_FMT_F16 = 2, VX_FMT_G64 = 3 };
constexpr uint32_t kVxFloatMaxK = 32768;  // fp32 activations of a float-row GEMV in LDS (128 KiB)

// Timeline build (-DVX_TIMELINE; velox_amd.build --timeline): the decode step's GEMV and attention
// launches stamp s_memrealtime (100 MHz) per workgroup into a host-set buffer, 8 words per workgroup
// at tl + 8 (tl_slot + workgroup): [0] start, [1] activations staged (GEMV) or first barrier
// (attention), [2] end, [3] attention's chunk loop done, [4] its merge barrier. The product build
// has neither the fields nor the stamps.
#ifdef VX_TIMELINE
#define VX_TIMELINE_FIELDS \
    unsigned long long* tl;  \
    uint32_t tl_slot;
#if defined(__HIP__)
__device__ __forceinline__ unsigned long long& vx_tl_mark(int i) {
    __shared__ unsigned long long m[5];
    return m[i];
}
struct VxTimelineWg {
    unsigned long long* e;
    __device__ VxTimelineWg(unsigned long long* tl, uint32_t slot, uint32_t wg) : e(tl ? tl + 8ull * (slot + wg) : nullptr) {
        if (threadIdx.x == 0) {
            vx_tl_mark(0) = __builtin_amdgcn_s_memrealtime();
            vx_tl_mark(1) = vx_tl_mark(3) = vx_tl_mark(4) = 0ull;
        }
    }
    // every thread of the workgroup leaves through one (uniform) return
    __device__ ~VxTimelineWg() {
        __syncthreads();
        if (e && threadIdx.x == 0) {
            e[0] = vx_tl_mark(0);
            e[1] = vx_tl_mark(1) ? vx_tl_mark(1) : vx_tl_mark(0);
            e[2] = __builtin_amdgcn_s_memrealtime();
            e[3] = vx_tl_mark(3);
            e[4] = vx_tl_mark(4);
        }
    }
};
#define VX_TL_BEGIN(args, wg) VxTimelineWg vx_tl_wg_((args).tl, (args).tl_slot, (wg))
#define VX_TL_MARK(i) \
    do {                                                                    \
        if (threadIdx.x == 0) vx_tl_mark(i) = __builtin_amdgcn_s_memrealtime(); \
    } while (0)
#endif
#else
#define VX_TIMELINE_FIELDS
#define VX_TL_BEGIN(args, wg) \
    do {                      \
    } while (0)
#define VX_TL_MARK(i) \
    do {              \
    } while (0)
#endif

struct VxMat {
    const uint4* codes;
    const uint16_t* scales;
    uint32_t n, k, s, n_tiles, n_iter, paired;
    uint32_t fmt;
};

struct VxGemvArgs {
    const uint4* codes;
    const uint16_t* scales;
    uint32_t n, k, n_tiles, n_iter;
    // tiled GEMV grid (set by the launcher): workgroup b owns tiles [b q + min(b, r), + q + (b < r))
    uint32_t wg_q, wg_r;
    const float* x;
    const float* gain;
    float eps;
    const float* bias;
    const float* res;
    float* y;
    // fused argmax (LM head)
    float* cand_v;
    uint32_t* cand_i;
    uint32_t* counter;
    VeloxDecodeState* state;
    uint32_t* ring;
    const uint32_t* prompt;
    const uint32_t* prompt_len;
    uint32_t* token_out;
    uint64_t active_mask;
    // x from split-K attention partials instead of `x` (o_proj): x[h*d + e] is the LSE merge of
    // part_o[h][s][e] with (m, l) = part_ml[h][s] over att_splits splits
    const float* part_o;
    const float* part_ml;
    uint32_t att_splits, att_d;
    VX_TIMELINE_FIELDS
};

struct VxAttnArgs {
    const float* qkv;
    uint16_t* kv;            // layer base, bf16: K [hkv][s_cap][d], then V [hkv][s_cap / 32][d][32] (vx_vslot)
    const float2* rope;      // [s_max][d/2] (cos, sin)
    const VeloxDecodeState* state;
    uint32_t fixed_pos;      // used when state == nullptr
    float* part_o;           // [hq][splits][d]
    float* part_ml;          // [hq][splits][2]
    uint32_t* counters;      // [hkv]
    float* out;              // [hq*d]
    uint32_t hq, hkv, s_max, splits;
    uint32_t s_cap;          // KV plane capacity in positions: s_max rounded up to 32
    uint32_t prefill;        // 1: the rows are positions of one sequence whose K/V rows (its own
                             // included) are already in the cache: attend over [0, pos], no append
    float scale;
    uint64_t active_mask;
    uint32_t partials_only;  // 1: always write (m, l, o) partials; the consumer merges them
    // batched decode: sequence b = blockIdx.z uses state[b], kv + b * kv_bstride (elements),
    // qkv + b * qkv_bstride, and partials offset by b * hq * splits * (d or 2)
    uint32_t batch;
    uint64_t kv_bstride;
    uint32_t qkv_bstride;
    // q/k/v as the K-split partials of the batched QKV GEMM (qkv_nparts > 0): element c of row b is
    // sum_{p < qkv_nparts} qkv_part[p * qkv_pstride + b * qkv_bstride + c] (+ qkv_bias[c]), summed in
    // split order as the partial-sum kernel would; qkv is then unused
    const float* qkv_part;
    const float* qkv_bias;
    uint64_t qkv_pstride;
    uint32_t qkv_nparts;
    uint32_t max_len;        // > 0: no row attends past this many positions (a prefill chunk's end); 0 unknown
    // one split and x16 set (batched steps): the normalized output goes straight to the fp16 operand
    // of the o_proj GEMM, element c of row b at x16[b * x_ld + (c / 32) * x_bs + c % 32] (the
    // batched merge kernel's output: fp16((1 / l) o)), and no partials are written
    uint16_t* x16;
    uint32_t x_ld, x_bs;
    // single-sequence decode (batch <= 1, state set): the RoPE row of the state's position, which the
    // step's embedding kernel copied there; the kernel then issues every load before it waits for the
    // position. NULL: the row is read from `rope` at the position.
    const float2* rope_cur;
    uint32_t chunk;  // set by vx_launch_attention: positions per split, ceil(s_max / splits) rounded up to 32
    VX_TIMELINE_FIELDS
};

// The single-sequence decode step's QKV GEMV and attention in one launch (vx_qkv_attn.hip): the
// GEMV's arguments (its own grid fields set by the launcher), the attention's (splits = A splits
// per KV head), and the synchronisation words: [g * 64] (64-bit) workgroups of head g counted in
// (low 8 bits; 7 bits per XCD above), [(hkv + g) * 64] its splits past their wait, [2 hkv * 64]
// error bits (1: a head's workgroups on two XCDs, 2: an expired wait), zero between launches.
struct VxQkvAttnArgs {
    VxGemvArgs g;
    VxAttnArgs at;
    uint32_t* sync;
    uint32_t na, p;               // attention workgroups (hkv x A); GEMV workgroups per KV head
    uint32_t tq, tk;              // row tiles of a KV head's q heads, and of its k (= of its v)
    uint32_t k_base, v_base;      // first row tile of the k heads, of the v heads
};
constexpr uint32_t kVxQkvSyncWords(uint32_t hkv) { return (2u * hkv + 1u) * 64u; }

// Batched (B <= 32 sequences) Q4_0 GEMM: Y[m][n] = sum_k X[m][k] W[n][k] for fp16 activations
// X (row stride ldx elements), through MFMA, with the same epilogues as the GEMV.
struct VxBGemmArgs {
    const uint4* codes;
    const uint16_t* scales;
    uint32_t n, k, n_tiles, n_iter, batch;
    // fp16 activations: element k of row m at x16[m * ldx + (k / 32) * xbs + k % 32] -- row-major
    // with xbs = 32, or block-major ([k / 32][rows][32]) with ldx = 32 and xbs = 32 * rows
    const uint16_t* x16;
    uint32_t ldx, xbs;
    const float* bias;     // STORE: + bias[n]
    float* y;              // STORE / ARGMAX: y[m][n] = ...; RESID: y[m][n] += ...   (row stride ldy)
    uint32_t ldy;
    uint16_t* out16;       // SWIGLU: out16[m * ldo + (j / 32) * obs + j % 32] = fp16(silu(gate) * up)
    uint32_t ldo, obs;
    float* cand_v;         // ARGMAX: per (m, workgroup) candidates, [batch][gridDim.x]
    uint32_t* cand_i;
    uint64_t active_mask;
    // RESID split over K: ksplit > 1 workgroup rows each cover n_iter / ksplit items and store
    // their sums to part[ks * pstride + m * ldy + n] instead of adding to y; the next batched
    // RMSNorm adds the ksplit partials to y in split order (vx_launch_bnorm's parts)
    uint32_t ksplit;
    float* part;
    uint64_t pstride;
};

// A Q4_0 matrix in the MFMA operand layout of the batched GEMM (vx_mgemm.hip), a second copy of a
// tiled matrix: 16-row tiles (paired: gate tile u at 2u, up tile u at 2u + 1) x groups of 4 blocks;
// per (tile, group) 64 16-byte words, lane l = row (l % 16), dword l / 16 of blocks 4j .. 4j+3;
// fp16 scales [tile][group][row][4].
struct VxMMat {
    const uint4* codes;
    const uint2* scales;
    uint32_t n, k, n_tiles, n_grp, paired;
};
void vx_mmat_shape(uint32_t n, uint32_t k, uint32_t paired, VxMMat& m);  // fills n, k, paired, n_tiles, n_grp
uint64_t vx_mmat_code_bytes(const VxMMat& m);
uint64_t vx_mmat_scale_bytes(const VxMMat& m);
uint32_t vx_mgemm_grid(uint32_t n_tiles);  // workgroups of one grid row (also the ARGMAX candidate count)
uint32_t vx_pgemm_grid(uint32_t n_tiles);  // the same for the 17-128-row GEMM (8 tiles per workgroup)
hipError_t vx_launch_mlayout(const VxMat& src, const VxMMat& dst, hipStream_t st);
// The batched Q4_0 GEMM over an MFMA-layout copy (codes/scales/n/k from `w`), epilogues as the
// GEMV's; ksplit > 1 (STORE or RESID) stores K-split partials, which vx_launch_msum (STORE, + bias)
// or the next batched RMSNorm (RESID) sums in split order.
hipError_t vx_launch_mgemm(const VxMMat& w, const VxBGemmArgs& a, int epi, hipStream_t st);
hipError_t vx_launch_msum(const float* part, uint32_t nparts, uint64_t pstride, const float* bias, float* y,
                          uint32_t n, uint32_t ldy, uint32_t batch, uint32_t accumulate, uint64_t mask,
                          hipStream_t st);

// fp8 (e4m3fn) block-scaled GEMM of up to 32 rows of activations, on MFMA (vx_mla.hip). Weights
// in 16-row x 64-column tiles of 1 KiB: lane l of tile (rt, kt) holds row 16 rt + l % 16, columns
// 64 kt + 16 (l / 16) .. + 15; scales per (16-row tile, 128-column block). grid (ceil(n_rt / 4),
// ksplit, groups): group g uses codes + g * w_gstride (16-byte units), scales + g * s_gstride,
// x + g * x_gstride, y + g * y_gstride (elements); ksplit > 1 stores split ks at y + ks * pstride.
struct VxF8GemmArgs {
    const uint4* codes;
    const float* scales;
    uint32_t n_rt, n_kt, n_kb, batch;
    const void* x;          // [batch][ldx] fp16 (x_f32 == 0) or fp32
    uint32_t ldx, x_f32;
    float* y;               // [batch][ldy]
    uint16_t* y16;          // != nullptr (ksplit 1): fp16 output [batch][ldy] in place of y
    uint32_t ldy, ksplit;
    uint32_t add_y;         // 1 (batch 1, ksplit 1, fp32 y): y += the product (a residual epilogue)
    const float* gain;      // != nullptr (batch 1, fp32 x): x := RMSNorm(x) * gain over its whole row first
    float eps;
    uint64_t w_gstride, s_gstride, x_gstride, y_gstride, pstride;
    uint64_t active_mask;
    // != nullptr (batch 1, fp32 x, ksplit 1, no gain): group g's activation row is the LSE merge of
    // its m_splits split partials -- fp16 o_j / l_j at m_part_o[(g m_splits + j) n_kt 64 + c] and
    // (m_j, l_j) at m_part_ml[2 (g m_splits + j)] -- in split order, as vx_mla_merge_kernel forms ctx;
    // x is then unused
    const uint16_t* m_part_o;
    const float* m_part_ml;
    uint32_t m_splits;
    // x_nparts > 1 (batch 1, fp32 x, with gain): the activation row is the sum of x_nparts K-split
    // partials x[s * x_pstride + k] (in split order), as the MLA prep kernel folded them
    uint32_t x_nparts;
    uint64_t x_pstride;
};

// vx_mla.hip launchers (absorbed MLA layer), used by vx_mla_host.cpp.
struct VxF8Dest;
struct VxMlaPrepArgs;
struct VxMlaAttnArgs;
hipError_t vx_launch_f8gemm(const VxF8GemmArgs& a, uint32_t groups, hipStream_t st);
uint32_t vx_f8gemm_rows_per_wave(uint32_t batch);  // 16-row tiles per wave of the fp8 GEMM
int vx_record_error(hipError_t e);  // vx_host.cpp: the first error of a step, read by velox_hip_last_error

// Launch helpers implemented in vx_kernels.hip, used by vx_host.cpp.
enum { VX_EPI_STORE = 0, VX_EPI_RESID = 1, VX_EPI_SWIGLU = 2, VX_EPI_ARGMAX = 3 };
hipError_t vx_launch_gemv(const VxMat& m, const VxGemvArgs& a, int epi, uint32_t max_wgs, hipStream_t st);
// The float-row GEMV (vx_gemv_f.hip) that vx_launch_gemv runs for VX_FMT_F32 / VX_FMT_F16 matrices,
// on `wgs` workgroups (vx_gemv_grid of the matrix's tiles).
hipError_t vx_launch_gemv_f(const VxMat& m, const VxGemvArgs& a, int epi, uint32_t wgs, hipStream_t st);
hipError_t vx_launch_attention(const VxAttnArgs& a, uint32_t d, hipStream_t st);
// vx_qkv_attn.hip: whether matrix m (the fused [q; k; v] rows) and the head shape take the fused
// QKV + attention launch; the launch with p GEMV workgroups per KV head; and the device check that
// workgroup b of a launch runs on XCD b % 8 (synchronous, once per device).
bool vx_qkv_attn_supported(const VxMat& m, uint32_t hq, uint32_t hkv, uint32_t d);
hipError_t vx_launch_qkv_attn(const VxMat& m, const VxQkvAttnArgs& f, uint32_t p, hipStream_t st);
bool vx_xcd_roundrobin_ok();
// vx_gemv_g64.hip: the reference's group-64 format (quant_mode 2) in the tiled layout -- the GEMV
// that vx_launch_gemv runs for VX_FMT_G64 matrices, fp32 rows (device) or seeded weights converted
// into rows [row0, row0 + rows) of part pair_part, and the reference's own packed output layout
hipError_t vx_launch_gemv_g64(const VxMat& m, const VxGemvArgs& a, int epi, uint32_t max_wgs, hipStream_t st);
hipError_t vx_launch_g64_from_rows(const float* rows_dev, uint32_t rows, uint32_t row0, uint32_t pair_part,
                                   const VxMat& m, hipStream_t st);
hipError_t vx_launch_synth_g64(const VxMat& m, uint32_t rows, uint32_t row0, uint32_t pair_part, uint64_t stream,
                               float coef, hipStream_t st);
hipError_t vx_launch_g64_quantize_ref(const float* src, uint64_t n_groups, uint32_t* packed, uint16_t* scale_min,
                                      hipStream_t st);
// vx_batch.hip
// Batched prefill (vx_batch.hip): row r of a chunk is position p0 + r of the one sequence.
hipError_t vx_launch_prefill_rows(VeloxDecodeState* rows, uint32_t n_rows, uint64_t p0, const uint32_t* prompt,
                                  uint64_t mask, hipStream_t st);
// qkv rows ldq apart; nparts > 0: qkv holds nparts K-split partials pstride apart (+ bias), summed here
hipError_t vx_launch_kv_append_rows(const float* qkv, uint32_t ldq, uint32_t nparts, uint64_t pstride,
                                    const float* bias, uint32_t hq, uint32_t hkv, uint32_t d,
                                    const VeloxDecodeState* rows, uint32_t n_rows, const float2* rope, uint32_t s_max,
                                    uint32_t s_cap, uint16_t* kv, uint64_t mask, hipStream_t st);
hipError_t vx_launch_prefill_finalize(const float* cand_v, const uint32_t* cand_i, uint32_t n,
                                      const VeloxDecodeState* rows, uint32_t n_rows, uint32_t* ring,
                                      VeloxDecodeState* state, const uint32_t* prompt, const uint32_t* plen,
                                      uint64_t mask, hipStream_t st);
hipError_t vx_launch_bembed(const VxMat& m, const VeloxDecodeState* states, uint32_t batch, float* h, uint32_t ldh,
                            uint64_t mask, hipStream_t st);
// parts != nullptr: h[b] += sum over s < nparts of parts[s * pstride + b * ldh] first (written back)
hipError_t vx_launch_bnorm(float* h, uint32_t ldh, const float* parts, uint32_t nparts, uint64_t pstride, const float* g,
                           uint32_t k, float eps, uint16_t* x16, uint32_t ldx, uint32_t xbs, uint32_t batch,
                           uint64_t mask, hipStream_t st);
bool vx_x_layout_ok(uint32_t k, uint32_t ldx, uint32_t xbs, uint32_t batch);  // activation operand layout check
hipError_t vx_launch_bmerge(const float* part_o, const float* part_ml, uint32_t hq, uint32_t d, uint32_t splits,
                            uint16_t* x16, uint32_t ldx, uint32_t xbs, uint32_t batch, uint64_t mask, hipStream_t st);
hipError_t vx_launch_bfinalize(const float* cand_v, const uint32_t* cand_i, uint32_t n, VeloxDecodeState* states,
                               uint32_t* rings, const uint32_t* prompts, const uint32_t* plens, uint32_t prompt_stride,
                               uint32_t batch, uint64_t mask, hipStream_t st);
hipError_t vx_launch_embed(const VxMat& m, const VeloxDecodeState* state, uint32_t fixed_token, float* h,
                           uint64_t mask, hipStream_t st, const float2* rope = nullptr, float2* rope_cur = nullptr,
                           uint32_t half = 0, uint32_t s_max = 0);
hipError_t vx_launch_set_state(VeloxDecodeState* state, uint64_t step, uint32_t token, hipStream_t st);
hipError_t vx_launch_repack(const void* blocks, uint32_t rows, uint32_t row0, uint32_t pair_part, const VxMat& m,
                            hipStream_t st);
hipError_t vx_launch_synth_q4(const VxMat& m, uint32_t rows, uint32_t row0, uint32_t pair_part, uint64_t stream,
                              float coef, hipStream_t st);
hipError_t vx_launch_fill_normal(float* out, uint64_t n, uint64_t stream, float coef, float mean, hipStream_t st);
hipError_t vx_launch_fill_normal_f16(uint16_t* out, uint64_t n, uint64_t stream, float coef, float mean, hipStream_t st);
// Fills K/V of one layer, positions [0, n_pos): element (t, g, d) draws index (t*hkv + g)*D + d,
// the [S][hkv*D] order of the reference's cache (src/runtime.rs:1358-1361).
hipError_t vx_launch_fill_kv(uint16_t* layer_base, uint32_t hkv, uint32_t s_cap, uint32_t d, uint32_t n_pos,
                             uint64_t stream_k, uint64_t stream_v, float coef, hipStream_t st);
hipError_t vx_launch_dequant(const VxMat& m, float* out, hipStream_t st);
hipError_t vx_launch_quantize(const float* x, uint32_t rows, uint32_t k, void* blocks, hipStream_t st);
// Element types of checkpoint tensors (safetensors F32 / F16 / BF16) for vx_launch_convert.
enum { VX_DT_F32 = 0, VX_DT_F16 = 1, VX_DT_BF16 = 2 };
hipError_t vx_launch_convert(const void* src, uint32_t src_dt, void* dst, uint32_t dst_dt, uint64_t n, hipStream_t st);
hipError_t vx_launch_rmsnorm(const float* x, const float* w, uint32_t n, float eps, float* y, hipStream_t st);
hipError_t vx_launch_argmax(const float* x, uint32_t n, uint32_t* out, hipStream_t st);
uint32_t vx_gemv_max_wgs_default();
uint32_t vx_gemv_grid(uint32_t n_tiles, uint32_t max_wgs);
hipError_t vx_launch_argmax_finalize(const float* cand_v, const uint32_t* cand_i, uint32_t n, VeloxDecodeState* state,
                                     uint32_t* ring, const uint32_t* prompt, const uint32_t* prompt_len,
                                     uint32_t* token_out, uint64_t mask, hipStream_t st);
