// vx_mla.h -- argument blocks and launchers of the absorbed MLA layer kernels (vx_mla.hip),
// shared with the host planner (vx_mla_host.cpp).
#pragma once

#include "vx_common.h"

// A destination fp8 matrix (groups x rows x cols in the tiled layout) reads element (g, r, k) of a
// logical source matrix [src_rows][src_cols] (the checkpoint's row-major tensor, or the seeded
// N(0, sigma) of the oracle's vxo_fp8_synth_matrix) at
//   DIRECT:  (row_off + r, k)                     -- q_a / kv_a / q_b / o (row_off: fused rows)
//   UK_T:    (g (dn + dv) + k, r)                 -- W_uk[g]^T, the absorption operand
//   UV:      (g (dn + dv) + dn + r, k)            -- W_uv[g]
enum { VX_MAP_DIRECT = 0, VX_MAP_UKT = 1, VX_MAP_UV = 2 };

struct VxF8Dest {
    uint4* codes;               // tiles of this destination (rows row_tile0.. of the matrix)
    float* scales;              // [g][n_rt_total][n_kb]
    uint32_t groups, rows, cols, n_rt_total, n_kt, n_kb, row_tile0;
    uint32_t map, row_off, dn, dv;
    uint32_t src_rows, src_cols;
    const uint8_t* src_codes;   // row-major source codes, or nullptr: synthesize
    const float* src_scales;    // source block scales [ceil(src_rows/128)][ceil(src_cols/128)]
    uint64_t stream;            // synthesis stream
    float coef;
    uint64_t w_gstride, s_gstride;
};

struct VxMlaPrepArgs {
    const float* parts;         // [nparts][batch][na] K-split partials of [W_qa; W_kva] x
    uint32_t nparts, na, q_part;  // q_part: leading q outputs (q_lora, or n_heads * (d_nope + d_rope))
    uint64_t pstride;
    uint32_t q_lora, lr, dr, kv_norm;
    const float* g_qa;          // q_lora RMSNorm gain
    const float* g_kva;         // latent RMSNorm gain
    float eps;
    const VeloxDecodeState* states;
    uint32_t s_max;
    const float2* rope;         // [s_max][dr / 2]
    uint16_t* cache;            // bf16 [batch][s_cap][lr + dr]
    uint64_t cache_bstride;
    uint16_t* q16;              // q_lora > 0: fp16 [batch][ldq16] normalized q latent
    uint32_t ldq16;
    float* q32;                 // q_lora == 0: fp32 [batch][q_part] q
    uint64_t active_mask;
};

struct VxMlaAttnArgs {
    const float* qabs;          // [batch][nh][LR] absorbed q
    const float* q32;           // [batch][nh * dq]: q_rope of head h at h * dq + dn
    uint32_t nh, dq, dn;
    const VeloxDecodeState* states;
    uint32_t s_max, s_cap, splits;
    const float2* rope;         // [s_max][DR / 2]
    float qscale;               // softmax scale * log2(e)
    const uint16_t* cache;      // bf16 [batch][s_cap][LR + DR]
    uint64_t cache_bstride;
    uint16_t* part_o;           // fp16 [batch][nh][splits][LR]: each split's output divided by its l
    float* part_ml;             // [batch][nh][splits][2]
    uint64_t active_mask;
};

hipError_t vx_launch_f8_synth_scales(float* scales, uint32_t rows, uint32_t cols, uint64_t stream, float coef,
                                     hipStream_t st);
hipError_t vx_launch_f8_pack(const VxF8Dest& d, hipStream_t st);
hipError_t vx_launch_mla_prep(const VxMlaPrepArgs& a, uint32_t batch, hipStream_t st);
// one sequence: W_qb's GEMV (x: the q-latent partials, with gain) and, in one more workgroup, the new
// latent row of p (the prep kernel's latent half)
hipError_t vx_launch_f8gemv_prep(const VxF8GemmArgs& a, const VxMlaPrepArgs& p, hipStream_t st);
hipError_t vx_launch_mla_attn(const VxMlaAttnArgs& a, uint32_t lr, uint32_t dr, uint32_t batch, hipStream_t st);
hipError_t vx_launch_mla_merge(const uint16_t* part_o, const float* part_ml, uint32_t nh, uint32_t splits, uint32_t lr,
                               float* ctx, uint32_t batch, uint64_t mask, hipStream_t st);
hipError_t vx_launch_mla_resid(float* h, const float* parts, uint32_t nparts, uint64_t pstride, uint32_t n,
                               uint32_t batch, uint64_t mask, hipStream_t st);
hipError_t vx_launch_mla_fill_cache(uint16_t* dst, uint64_t n, uint64_t stream, float coef, hipStream_t st);
hipError_t vx_launch_mla_advance(VeloxDecodeState* states, uint32_t batch, uint64_t mask, hipStream_t st);
