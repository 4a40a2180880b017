// vx_noalloc.hip -- the fused RMSNorm + LM head + greedy argmax for callers that cannot allocate
// device memory (code under hipGraph capture, tight serving loops, harnesses that forbid hipMalloc).
//
// velox_hip_lm_head_argmax needs one (value, index) candidate per GEMV workgroup and allocates
// that buffer per call. The variant here keeps it in a file-scope device array instead, so the
// call allocates nothing: every call on one GPU shares that GPU's copy of the array.
#include <hip/hip_runtime.h>

#include <mutex>

#include "vx_common.h"

// Candidate capacity: the GEMV grid never exceeds 512 workgroups (vx_gemv_grid), so 512
// (value, index) pairs -- 4 KiB per GPU, held until the process ends -- cover every matrix shape.
#define VX_NOALLOC_CANDIDATES 512u

// fp32 candidate values [0, 512) then uint32 candidate indices [512, 1024). In host code this name
// is only a stand-in for the symbol: its device address comes from hipGetSymbolAddress below.
static __device__ __align__(256) uint32_t scratch[2u * VX_NOALLOC_CANDIDATES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of the current device's scratch copy, looked up once per device with that device
// current.
hipError_t vx_scratch_ptr(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return e;
        if (!p) return hipErrorInvalidSymbol;
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return hipSuccess;
}

}  // namespace

extern "C" int velox_hip_lm_head_argmax_noalloc(const VeloxHipQ4Matrix* m, const float* d_x, const float* d_gain,
                                                float eps, float* d_logits, uint32_t* d_token, hipStream_t st) {
    if (!m || !d_x || !d_logits || !d_token || m->paired || m->k == 0 || (m->k & 31u)) return VELOX_HIP_EINVAL;
    const uint32_t wgs = vx_gemv_max_wgs_default(), n = vx_gemv_grid(m->n_tiles, wgs);
    if (n == 0 || n > VX_NOALLOC_CANDIDATES) return VELOX_HIP_EINVAL;  // more candidates than the array holds
    void* p = nullptr;
    hipError_t e = vx_scratch_ptr(&p);
    if (e != hipSuccess) return (int)e;
    VxMat w;
    w.codes = (const uint4*)m->codes;
    w.scales = (const uint16_t*)m->scales;
    w.n = m->n;
    w.k = m->k;
    w.s = m->s_lanes;
    w.n_tiles = m->n_tiles;
    w.n_iter = m->n_iter;
    w.paired = 0;
    // format 0: GGML Q4_0 blocks; VELOX_QUANT_Q4_GROUP64: group-64 pairs; others are refused
    if (m->format != 0 && m->format != VELOX_QUANT_Q4_GROUP64) return VELOX_HIP_EINVAL;
    w.fmt = m->format == 0 ? VX_FMT_Q4 : VX_FMT_G64;
    VxGemvArgs g = {};
    g.x = d_x;
    g.gain = d_gain;
    g.eps = eps;
    g.y = d_logits;
    // every workgroup writes its candidate before the finalize kernel reads it: nothing to clear
    g.cand_v = (float*)p;
    g.cand_i = (uint32_t*)p + VX_NOALLOC_CANDIDATES;
    g.active_mask = 1;
    e = vx_launch_gemv(w, g, VX_EPI_ARGMAX, wgs, st);
    if (e == hipSuccess)
        e = vx_launch_argmax_finalize(g.cand_v, g.cand_i, n, nullptr, nullptr, nullptr, nullptr, d_token, 1, st);
    return (int)e;
}
