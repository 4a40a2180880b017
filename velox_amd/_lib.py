"""ctypes bindings of the C ABI in include/velox_hip.h (libvelox_hip.so, built in-tree).

The product path has no fallback: if the HIP library is missing, load() raises.
"""
from __future__ import annotations

import ctypes as C
import os
import re

PKG = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(PKG)
LIB_PATH = os.path.join(PKG, "lib", "libvelox_hip.so")
HEADER = os.path.join(ROOT, "include", "velox_hip.h")

# quant_mode: the reference's fp32 / fp16 rows and group-64 format, GGML Q4_0
QUANT_F32, QUANT_F16, QUANT_G64, QUANT_GGML_Q4_0 = 0, 1, 2, 5
GEMV_STORE, GEMV_RESIDUAL, GEMV_SWIGLU = 0, 1, 2
EINVAL, ENOMEM, ESHAPE, ENOTLOADED, ETENSOR, EDTYPE = -1, -2, -3, -4, -5, -6
DT_F32, DT_F16, DT_BF16 = 0, 1, 2
T_EMBED, T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN = 1, 2, 3, 4, 5, 6, 7, 8
T_ATTN_NORM, T_MLP_NORM, T_FINAL_NORM, T_HEAD, T_BQ, T_BK, T_BV = 9, 10, 11, 12, 13, 14, 15
RING_SIZE = 1024


class ModelConfig(C.Structure):
    _fields_ = [
        ("name", C.c_char * 32),
        ("vocab_size", C.c_uint32), ("hidden_dim", C.c_uint32), ("intermediate_dim", C.c_uint32),
        ("num_layers", C.c_uint32), ("num_heads", C.c_uint32), ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("max_seq_len", C.c_uint32),
        ("rms_norm_eps", C.c_float), ("rope_theta", C.c_float),
        ("qkv_bias", C.c_uint32), ("tied_lm_head", C.c_uint32), ("quant_mode", C.c_uint32),
        ("attn_splits", C.c_uint32), ("vram_budget_bytes", C.c_uint64),
        ("max_batch", C.c_uint32), ("prefill_chunk", C.c_uint32),
    ]

    def as_dict(self) -> dict:
        d = {f: getattr(self, f) for f, _ in self._fields_}
        d["name"] = self.name.decode()
        return d


class Arena(C.Structure):
    _fields_ = [
        ("weight_arena", C.c_void_p), ("kv_cache_pool", C.c_void_p), ("activation_arena", C.c_void_p),
        ("host_pinned_ring", C.POINTER(C.c_uint32)), ("norm_weight_arena", C.c_void_p),
        ("weight_scales", C.c_void_p), ("quant_mode", C.c_uint32), ("tied_lm_head", C.c_uint32),
    ]


class DecodeState(C.Structure):
    _fields_ = [("step", C.c_uint64), ("token", C.c_uint32), ("reserved", C.c_uint32)]


class Q4Matrix(C.Structure):
    _fields_ = [
        ("codes", C.c_void_p), ("scales", C.c_void_p), ("n", C.c_uint32), ("k", C.c_uint32),
        ("s_lanes", C.c_uint32), ("n_tiles", C.c_uint32), ("n_iter", C.c_uint32),
        ("paired", C.c_uint32), ("format", C.c_uint32),
    ]


class RunOptions(C.Structure):
    _fields_ = [
        ("model", C.c_char_p), ("max_seq_len", C.c_uint32), ("prompt_len", C.c_uint32),
        ("warmup", C.c_uint32), ("steps", C.c_uint32), ("seed", C.c_uint64), ("sigma", C.c_float),
        ("norm_sigma", C.c_float), ("use_graph", C.c_uint32), ("num_layers", C.c_uint32),
        ("kernel_passes", C.c_uint32), ("verbose", C.c_uint32), ("prompt_tokens", C.POINTER(C.c_uint32)),
        ("context_len", C.c_uint32), ("batch", C.c_uint32), ("weights_path", C.c_char_p),
        ("prefill_chunk", C.c_uint32), ("model_file", C.c_char_p), ("unquantized", C.c_uint32),
        ("model_config", C.POINTER(ModelConfig)), ("decode_step", C.c_void_p), ("attn_splits", C.c_uint32),
    ]


class RunReport(C.Structure):
    _fields_ = [
        ("load_ms", C.c_double), ("prefill_ms", C.c_double), ("decode_ms", C.c_double),
        ("tok_per_s", C.c_double), ("bytes_per_step", C.c_double), ("hbm_gbps", C.c_double),
        ("wall_ms", C.c_double), ("kernel_us", C.c_double), ("kernel_bytes", C.c_double),
        ("kernel_launches", C.c_uint32), ("n_tokens", C.c_uint32), ("first_token", C.c_uint32), ("status", C.c_int),
        ("first_position", C.c_uint32),
        ("step_p50_ms", C.c_double), ("step_p99_ms", C.c_double), ("step_max_ms", C.c_double),
    ]


class VlxTarget(C.Structure):
    _fields_ = [("device", C.c_char * 64), ("vram_capacity_bytes", C.c_uint64), ("safety_factor", C.c_double),
                ("safe_budget_bytes", C.c_uint64), ("system_reserve_bytes", C.c_uint64), ("b_max", C.c_uint32),
                ("s_max", C.c_uint32), ("weights_file", C.c_char * 256)]


class MlaConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("hidden_dim", "num_heads", "q_lora_rank", "kv_lora_rank", "qk_nope_dim",
                                          "qk_rope_dim", "v_head_dim", "num_layers", "max_seq_len", "max_batch",
                                          "kv_norm", "attn_splits")] + \
               [("rms_norm_eps", C.c_float), ("rope_theta", C.c_float), ("softmax_scale", C.c_float),
                ("reserved", C.c_uint32), ("vram_budget_bytes", C.c_uint64)]


class MlaBuffers(C.Structure):
    _fields_ = [("hidden", C.c_void_p), ("latent_cache", C.c_void_p), ("states", C.c_void_p), ("s_cap", C.c_uint32),
                ("splits", C.c_uint32), ("weight_bytes", C.c_uint64), ("cache_bytes", C.c_uint64),
                ("act_bytes", C.c_uint64)]


class MlaRunReport(C.Structure):
    _fields_ = [(n, C.c_double) for n in ("us_per_layer", "bytes_per_layer", "hbm_gbps", "attn_us", "attn_bytes",
                                          "wall_ms")] + [("status", C.c_int)]


MLA_Q_A, MLA_Q_B, MLA_KV_A, MLA_KV_B, MLA_O, MLA_NORM, MLA_Q_A_NORM, MLA_KV_A_NORM = range(1, 9)


def header_exports(path: str = HEADER) -> list[str]:
    """Names of every function declared in include/velox_hip.h."""
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(velox_\w+)\s*\(", text)))


_lib = None

_P = C.c_void_p
_U32, _U64, _F, _I = C.c_uint32, C.c_uint64, C.c_float, C.c_int

_SIGS = {
    "velox_hip_last_error": (_I, []),
    "velox_hip_set_fused_attention": (None, [_I]),
    "velox_hip_fused_attention_status": (_I, [C.POINTER(Arena), C.POINTER(_U32), C.POINTER(_U32)]),
    "velox_hip_builtin_config": (_I, [C.c_char_p, _U32, C.POINTER(ModelConfig)]),
    "velox_hip_vlx_config": (_I, [C.c_char_p, _U32, C.POINTER(ModelConfig), C.POINTER(VlxTarget)]),
    "velox_hip_vlx_load": (_I, [C.c_char_p, _U32, C.POINTER(ModelConfig), C.POINTER(VlxTarget)]),
    "velox_hip_model_create": (_I, [C.POINTER(ModelConfig), C.POINTER(_P)]),
    "velox_hip_model_destroy": (None, [_P]),
    "velox_hip_model_config": (_I, [_P, C.POINTER(ModelConfig)]),
    "velox_hip_model_arena_bytes": (_I, [_P] + [C.POINTER(_U64)] * 5),
    "velox_hip_model_step_bytes": (_U64, [_P, _U64]),
    "velox_hip_model_logits_offset": (_U64, [_P]),
    "velox_hip_model_hidden_offset": (_U64, [_P]),
    "velox_hip_arena_create": (_I, [_P, C.POINTER(Arena)]),
    "velox_hip_arena_destroy": (_I, [C.POINTER(Arena)]),
    "velox_hip_arena_bind": (_I, [_P, C.POINTER(Arena)]),
    "velox_hip_arena_model": (_P, [C.POINTER(Arena)]),
    "velox_hip_load_q4_0": (_I, [C.POINTER(Arena), _I, _U32, _P, _U64, _P]),
    "velox_hip_load_rows": (_I, [C.POINTER(Arena), _I, _U32, _P, _U64, _P]),
    "velox_hip_load_f32": (_I, [C.POINTER(Arena), _I, _U32, _P, _U64, _P]),
    "velox_hip_load_tensor": (_I, [C.POINTER(Arena), _I, _U32, _P, _U64, _U32, _P]),
    "velox_hip_st_open": (_I, [C.c_char_p, C.POINTER(_P)]),
    "velox_hip_st_close": (None, [_P]),
    "velox_hip_st_tensor_count": (_U64, [_P]),
    "velox_hip_st_tensor_info": (_I, [_P, _U64, C.c_char_p, _U32, C.c_char_p, C.POINTER(_U64), C.POINTER(_U32),
                                      C.POINTER(_U64), C.POINTER(_U64)]),
    "velox_hip_st_find": (_I, [_P, C.c_char_p, C.POINTER(_U64)]),
    "velox_hip_st_tensor_data": (_I, [_P, C.c_char_p, C.c_char_p, C.POINTER(_P), C.POINTER(_U64)]),
    "velox_hip_st_config": (_I, [_P, _U32, C.POINTER(ModelConfig)]),
    "velox_hip_st_check": (_I, [_P, C.POINTER(ModelConfig)]),
    "velox_hip_st_load": (_I, [C.POINTER(Arena), _P, _P]),
    "velox_hip_synthesize_model": (_I, [C.POINTER(Arena), _U64, _F, _F, _P]),
    "velox_hip_fill_kv": (_I, [C.POINTER(Arena), _U32, _U32, _U64, _F, _P]),
    "velox_hip_set_prompt": (_I, [C.POINTER(Arena), C.POINTER(_U32), _U32, _P]),
    "velox_hip_set_state": (_I, [C.POINTER(Arena), _U64, _U32, _P]),
    "velox_hip_get_state": (_I, [C.POINTER(Arena), C.POINTER(DecodeState), _P]),
    "velox_hip_decode_graph_step": (None, [C.POINTER(Arena), _U64, _P]),
    "velox_hip_model_batch_layout": (_I, [_P, C.POINTER(_U32), C.POINTER(_U64), C.POINTER(_U64)]),
    "velox_hip_model_batch_step_bytes": (_U64, [_P, _U32, _U64]),
    "velox_hip_batch_set_prompt": (_I, [C.POINTER(Arena), _U32, _P, _U32, _P]),
    "velox_hip_batch_set_state": (_I, [C.POINTER(Arena), _U32, _U64, _U32, _P]),
    "velox_hip_batch_get_state": (_I, [C.POINTER(Arena), _U32, C.POINTER(DecodeState), _P]),
    "velox_hip_fill_kv_seq": (_I, [C.POINTER(Arena), _U32, _U32, _U32, _U64, _F, _P]),
    "velox_hip_decode_batch_graph_step": (None, [C.POINTER(Arena), _U32, _U64, _P]),
    "velox_hip_prefill_batch": (_I, [C.POINTER(Arena), _U64, _U32, _U64, _P]),
    "velox_hip_decode": (None, [C.POINTER(Arena), _U32, C.c_size_t, _U64, _P]),
    "velox_hip_prefill_graph_step": (None, [C.POINTER(Arena), _U64, _P]),
    "velox_hip_prefill": (None, [C.POINTER(Arena), _U32, C.c_size_t, _U64, _P]),
    "velox_hip_arena_matrix": (_I, [C.POINTER(Arena), _I, _U32, C.POINTER(Q4Matrix), C.POINTER(_U32)]),
    "velox_hip_arena_vector": (_I, [C.POINTER(Arena), _I, _U32, C.POINTER(_P), C.POINTER(_U64)]),
    "velox_hip_q4_layout": (_I, [_U32, _U32, _U32, _U32, C.POINTER(Q4Matrix), C.POINTER(_U64), C.POINTER(_U64)]),
    "velox_hip_q4_0_repack": (_I, [_P, _U32, _U32, _U32, C.POINTER(Q4Matrix), _P]),
    "velox_hip_q4_0_dequant": (_I, [C.POINTER(Q4Matrix), _P, _P]),
    "velox_hip_q4_0_quantize": (_I, [_P, _U32, _U32, _P, _P]),
    "velox_hip_g64_quantize": (_I, [_P, _U64, _P, _P, _P]),
    "velox_hip_g64_pack": (_I, [_P, _U32, _U32, _U32, C.POINTER(Q4Matrix), _P]),
    "velox_hip_fill_normal": (_I, [_P, _U64, _U64, _U64, _F, _F, _P]),
    "velox_hip_gemv_q4_0": (_I, [C.POINTER(Q4Matrix), _P, _P, _F, _P, _P, _P, _I, _P]),
    "velox_hip_gemm_q4_0_batch": (_I, [C.POINTER(Q4Matrix), _P, _U32, _U32, _P, _P, _U32, _P, _U32, _I, _P]),
    "velox_hip_q4_mlayout_bytes": (_I, [C.POINTER(Q4Matrix), C.POINTER(_U64), C.POINTER(_U64)]),
    "velox_hip_q4_mlayout": (_I, [C.POINTER(Q4Matrix), _P, _P, _P]),
    "velox_hip_gemm_q4_0_batch_m": (_I, [C.POINTER(Q4Matrix), _P, _P, _P, _U32, _U32, _U32, _P, _P, _U32, _P, _U32,
                                         _U32, _I, _U32, _P, _P]),
    "velox_hip_lm_head_argmax": (_I, [C.POINTER(Q4Matrix), _P, _P, _F, _P, _P, _P]),
    "velox_hip_lm_head_argmax_noalloc": (_I, [C.POINTER(Q4Matrix), _P, _P, _F, _P, _P, _P]),
    "velox_hip_argmax_f32": (_I, [_P, _U32, _P, _P]),
    "velox_hip_rmsnorm": (_I, [_P, _P, _U32, _F, _P, _P]),
    "velox_hip_attention_decode": (_I, [_P, _P, _U32, _U32, _U32, _U32, _U32, _F, _U32, _P, _P]),
    "velox_hip_run": (_I, [C.POINTER(RunOptions), C.POINTER(_U32), _U32, C.POINTER(RunReport)]),
    "velox_hip_gguf_open": (_I, [C.c_char_p, C.POINTER(_P)]),
    "velox_hip_gguf_close": (None, [_P]),
    "velox_hip_gguf_tensor_count": (_U64, [_P]),
    "velox_hip_gguf_tensor_info": (_I, [_P, _U64, C.c_char_p, _U32, C.POINTER(_U32), C.POINTER(_U32),
                                        C.POINTER(_U64), C.POINTER(_U64)]),
    "velox_hip_gguf_config": (_I, [_P, _U32, C.POINTER(ModelConfig)]),
    "velox_hip_gguf_load": (_I, [C.POINTER(Arena), _P, _P]),
    "velox_hip_mla_builtin_config": (_I, [C.c_char_p, _U32, _U32, C.POINTER(MlaConfig)]),
    "velox_hip_vlx_mla_config": (_I, [C.c_char_p, _U32, _U32, C.POINTER(MlaConfig), C.POINTER(VlxTarget)]),
    "velox_hip_mla_create": (_I, [C.POINTER(MlaConfig), C.POINTER(_P)]),
    "velox_hip_mla_destroy": (None, [_P]),
    "velox_hip_mla_buffers": (_I, [_P, C.POINTER(MlaBuffers)]),
    "velox_hip_mla_load_fp8": (_I, [_P, _I, _U32, _P, _P, _P]),
    "velox_hip_mla_load_f32": (_I, [_P, _I, _U32, _P, _U64, _P]),
    "velox_hip_mla_synthesize": (_I, [_P, _U64, _F, _F, _P]),
    "velox_hip_mla_fill_cache": (_I, [_P, _U32, _U32, _U32, _U64, _F, _P]),
    "velox_hip_mla_set_position": (_I, [_P, _U32, _U64, _P]),
    "velox_hip_mla_layer_step": (None, [_P, _U32, _U32, _U64, _P]),
    "velox_hip_mla_decode_step": (None, [_P, _U32, _U64, _P]),
    "velox_hip_mla_step_bytes": (C.c_double, [_P, _U32, _U64]),
    "velox_hip_mla_run": (_I, [C.c_char_p, _U32, _U32, _U32, _U32, _U32, _U64, C.POINTER(MlaRunReport)]),
    "velox_hip_mla_plan": (_I, [C.POINTER(MlaConfig), C.POINTER(_P)]),
    "velox_hip_mla_arena_bytes": (_I, [_P] + [C.POINTER(_U64)] * 5),
    "velox_hip_mla_arena": (_I, [_P, C.POINTER(Arena)]),
    "velox_hip_mla_arena_bind": (_I, [_P, C.POINTER(Arena)]),
    "velox_hip_mla_arena_mla": (_P, [C.POINTER(Arena)]),
    "velox_hip_mla_arena_check": (_I, [C.POINTER(Arena), C.POINTER(MlaConfig)]),
    "velox_hip_mla_graph_step": (None, [C.POINTER(Arena), _U64, _P]),
    "velox_hip_mla_decode": (None, [C.POINTER(Arena), _U32, C.c_size_t, _U64, _P]),
    "velox_hip_arena_check": (_I, [C.POINTER(Arena), C.POINTER(ModelConfig)]),
    "velox_hip_record_error": (None, [_I]),
    "velox_hip_decode": (None, [C.POINTER(Arena), _U32, C.c_size_t, _U64, _P]),
    "velox_hip_decode_graph_step": (None, [C.POINTER(Arena), _U64, _P]),
}


def bind_entry_points(lib: C.CDLL, model: str) -> None:
    """Argument types of a model's four named entry points (velox_<model>_{decode,prefill}
    {_graph_step,}_hip) in `lib` (the HIP library, or a module velox_amd.build generated)."""
    for phase in ("decode", "prefill"):
        g = getattr(lib, f"velox_{model}_{phase}_graph_step_hip")
        g.restype, g.argtypes = None, [C.POINTER(Arena), _U64, _P]
        f = getattr(lib, f"velox_{model}_{phase}_hip")
        f.restype, f.argtypes = None, [C.POINTER(Arena), _U32, C.c_size_t, _U64, _P]


def load() -> C.CDLL:
    """Loads libvelox_hip.so; raises if it was not built (there is no CPU fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"HIP backend not built: {LIB_PATH} missing (run velox_amd.build.build())")
    L = C.CDLL(LIB_PATH)
    for name, (res, args) in _SIGS.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    for model in ("SmolLM_135M", "Llama3_8B", "Qwen2_5_7B", "Qwen2_72B", "DeepSeek_V3_MLA"):
        bind_entry_points(L, model)
    _lib = L
    return L


def check(rc: int, what: str = "") -> None:
    if rc != 0:
        raise RuntimeError(f"velox_hip call {what} failed with status {rc}")


def builtin_config(name: str, max_seq_len: int = 0) -> ModelConfig:
    c = ModelConfig()
    check(load().velox_hip_builtin_config(name.encode(), max_seq_len, C.byref(c)), "builtin_config")
    return c


# ---------------------------------------------------------------------------------------------
# HIP runtime plumbing for host<->device copies of arena regions (libamdhip64 is the runtime the
# library itself links; no compute goes through it).
# ---------------------------------------------------------------------------------------------
_hip = None


def hip() -> C.CDLL:
    global _hip
    if _hip is None:
        _hip = C.CDLL("libamdhip64.so")
        _hip.hipMemcpy.restype = C.c_int
        _hip.hipMemcpy.argtypes = [_P, _P, C.c_size_t, C.c_int]
        _hip.hipDeviceSynchronize.restype = C.c_int
        _hip.hipStreamSynchronize.restype = C.c_int
        _hip.hipStreamSynchronize.argtypes = [_P]
    return _hip


def memcpy_dtoh(dst_host_ptr: int, src_dev_ptr: int, nbytes: int) -> None:
    rc = hip().hipMemcpy(dst_host_ptr, src_dev_ptr, nbytes, 2)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy DtoH failed: {rc}")


def memcpy_htod(dst_dev_ptr: int, src_host_ptr: int, nbytes: int) -> None:
    rc = hip().hipMemcpy(dst_dev_ptr, src_host_ptr, nbytes, 1)
    if rc != 0:
        raise RuntimeError(f"hipMemcpy HtoD failed: {rc}")


def device_copy_calibration(nbytes: int, reps: int = 3) -> None:
    """hipMemcpy device->device of `nbytes`, `reps` times: a plain copy kernel of known size
    (reads and writes nbytes per dispatch), the yardstick for the HBM byte counters under
    rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE."""
    h = hip()
    h.hipMalloc.restype = C.c_int
    h.hipMalloc.argtypes = [C.POINTER(_P), C.c_size_t]
    h.hipFree.restype = C.c_int
    h.hipFree.argtypes = [_P]
    h.hipMemset.restype = C.c_int
    h.hipMemset.argtypes = [_P, C.c_int, C.c_size_t]
    src, dst = _P(), _P()
    if h.hipMalloc(C.byref(src), nbytes) or h.hipMalloc(C.byref(dst), nbytes):
        raise RuntimeError("hipMalloc failed")
    try:
        if h.hipMemset(src, 1, nbytes):
            raise RuntimeError("hipMemset failed")
        for _ in range(reps):
            if h.hipMemcpy(dst, src, nbytes, 3):
                raise RuntimeError("hipMemcpy DtoD failed")
        if h.hipDeviceSynchronize():
            raise RuntimeError("hipDeviceSynchronize failed")
    finally:
        h.hipFree(src)
        h.hipFree(dst)
