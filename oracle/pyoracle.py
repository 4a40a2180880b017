"""ctypes bindings for the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg import this module:
the oracle is the checker and the timed CPU baseline, never part of the product path.
The C sources (velox_oracle.c) cite the reference functions they restate.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "build", "libvelox_oracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libvelox_ref_smollm.so")

# tensor kinds (velox_oracle.h)
T_EMBED, T_Q, T_K, T_V, T_O, T_GATE, T_UP, T_DOWN = 1, 2, 3, 4, 5, 6, 7, 8
T_ATTN_NORM, T_MLP_NORM, T_FINAL_NORM, T_HEAD, T_BQ, T_BK, T_BV, T_PROMPT = 9, 10, 11, 12, 13, 14, 15, 16


class VxoConfig(C.Structure):
    _fields_ = [
        ("vocab_size", C.c_uint32), ("hidden_dim", C.c_uint32), ("intermediate_dim", C.c_uint32),
        ("num_layers", C.c_uint32), ("num_heads", C.c_uint32), ("num_kv_heads", C.c_uint32),
        ("head_dim", C.c_uint32), ("max_seq_len", C.c_uint32), ("rms_norm_eps", C.c_float),
        ("rope_theta", C.c_float), ("qkv_bias", C.c_uint32), ("tied_lm_head", C.c_uint32),
        ("q4_0", C.c_uint32), ("kv_bf16", C.c_uint32), ("w_f16", C.c_uint32), ("w_g64", C.c_uint32),
    ]


class VxoMlaConfig(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("hidden", "n_heads", "q_lora", "kv_lora", "d_nope", "d_rope", "d_v",
                                          "kv_norm", "max_seq")] + \
               [(n, C.c_float) for n in ("eps", "rope_theta", "scale")]


class VxoMlaWeights(C.Structure):
    _fields_ = [(n, C.POINTER(C.c_float)) for n in ("norm", "q_a", "q_a_norm", "q_b", "kv_a", "kv_a_norm", "kv_b",
                                                    "o")]


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE], check=True)


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        fp = C.POINTER(C.c_float)
        u8p = C.POINTER(C.c_uint8)
        L.vxo_mix64.restype = C.c_uint64
        L.vxo_mix64.argtypes = [C.c_uint64]
        L.vxo_stream.restype = C.c_uint64
        L.vxo_stream.argtypes = [C.c_uint64, C.c_uint64]
        L.vxo_normal.restype = C.c_float
        L.vxo_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_float]
        L.vxo_normal_coef.restype = C.c_float
        L.vxo_normal_coef.argtypes = [C.c_float]
        L.vxo_uniform_u32.restype = C.c_uint32
        L.vxo_uniform_u32.argtypes = [C.c_uint64, C.c_uint64, C.c_uint32]
        L.vxo_fill_normal.argtypes = [fp, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, C.c_float]
        L.vxo_tag.restype = C.c_uint64
        L.vxo_tag.argtypes = [C.c_uint32, C.c_uint32]
        L.vxo_f32_to_f16.restype = C.c_uint16
        L.vxo_f32_to_f16.argtypes = [C.c_float]
        L.vxo_f16_to_f32.restype = C.c_float
        L.vxo_f16_to_f32.argtypes = [C.c_uint16]
        L.vxo_f32_to_bf16.restype = C.c_uint16
        L.vxo_f32_to_bf16.argtypes = [C.c_float]
        L.vxo_bf16_to_f32.restype = C.c_float
        L.vxo_bf16_to_f32.argtypes = [C.c_uint16]
        L.vxo_q4_0_quantize_row.argtypes = [fp, C.c_uint64, u8p]
        L.vxo_q4_0_dequant_row.argtypes = [u8p, C.c_uint64, fp]
        L.vxo_g64_quantize.argtypes = [fp, C.c_uint64, C.POINTER(C.c_uint32), C.POINTER(C.c_uint16)]
        L.vxo_g64_dequant.argtypes = [C.POINTER(C.c_uint32), C.POINTER(C.c_uint16), C.c_uint64, fp]
        L.vxo_rmsnorm.argtypes = [fp, fp, fp, C.c_uint64, C.c_float]
        L.vxo_matmul_transposed.argtypes = [fp, fp, fp, C.c_uint64, C.c_uint64]
        L.vxo_matmul_q4_0.argtypes = [fp, fp, u8p, C.c_uint64, C.c_uint64, C.c_int]
        L.vxo_rope_rotate_half.argtypes = [fp, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float]
        L.vxo_gqa_attention_step.argtypes = [fp, fp, fp, fp, fp, C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64]
        L.vxo_swiglu_act.argtypes = [fp, fp, C.c_uint64]
        L.vxo_argmax.restype = C.c_uint32
        L.vxo_argmax.argtypes = [fp, C.c_uint64]
        L.vxo_mla_absorbed_step.argtypes = [fp, fp, fp, fp, fp, fp, fp, C.c_uint64, C.c_uint64,
                                            C.c_uint64, C.c_uint64, C.c_float]
        L.vxo_f32_to_e4m3.restype = C.c_uint8
        L.vxo_f32_to_e4m3.argtypes = [C.c_float]
        L.vxo_e4m3_to_f32.restype = C.c_float
        L.vxo_e4m3_to_f32.argtypes = [C.c_uint8]
        L.vxo_fp8_quantize.argtypes = [fp, C.c_uint64, C.c_uint64, u8p, fp]
        L.vxo_fp8_dequant.argtypes = [u8p, fp, C.c_uint64, C.c_uint64, fp]
        L.vxo_fp8_synth_matrix.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.c_uint64, C.c_float, u8p, fp, fp]
        L.vxo_mla_layer_step.argtypes = [C.POINTER(VxoMlaConfig), C.POINTER(VxoMlaWeights), fp, C.c_int, fp, fp,
                                         C.c_uint64]
        L.vxo_engine_create.restype = C.c_void_p
        L.vxo_engine_create.argtypes = [C.POINTER(VxoConfig), C.c_uint64, C.c_float, C.c_float, C.c_uint32, C.c_int]
        L.vxo_engine_destroy.argtypes = [C.c_void_p]
        L.vxo_engine_forward.restype = C.c_uint32
        L.vxo_engine_forward.argtypes = [C.c_void_p, C.c_uint32, C.c_uint64, fp]
        L.vxo_engine_forward_layers.restype = C.c_uint32
        L.vxo_engine_forward_layers.argtypes = [C.c_void_p, C.c_uint32, C.c_uint64, C.c_uint32, fp]
        L.vxo_engine_reset.argtypes = [C.c_void_p]
        L.vxo_engine_set_threads.argtypes = [C.c_void_p, C.c_int]
        L.vxo_engine_tensor.restype = C.c_void_p
        L.vxo_engine_tensor.argtypes = [C.c_void_p, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint64)]
        L.vxo_engine_hidden.restype = fp
        L.vxo_engine_hidden.argtypes = [C.c_void_p]
        L.vxo_engine_k_cache.restype = fp
        L.vxo_engine_k_cache.argtypes = [C.c_void_p]
        L.vxo_engine_v_cache.restype = fp
        L.vxo_engine_v_cache.argtypes = [C.c_void_p]
        L.vxo_engine_force_kv.argtypes = [C.c_void_p, fp, fp, fp, fp]
        _lib = L
    return _lib


def fptr(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_float))


def u8ptr(a: np.ndarray):
    assert a.dtype == np.uint8 and a.flags.c_contiguous
    return a.ctypes.data_as(C.POINTER(C.c_uint8))


# ---------------------------------------------------------------------------------------------
# thin numpy wrappers
# ---------------------------------------------------------------------------------------------
def tag(layer: int, kind: int) -> int:
    return layer * 256 + kind


def fill_normal(n: int, seed: int, tg: int, sigma: float = 0.02, mean: float = 0.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().vxo_fill_normal(fptr(out), n, seed, tg, sigma, mean)
    return out


def prompt_tokens(seed: int, n: int, vocab: int) -> np.ndarray:
    L = lib()
    st = L.vxo_stream(seed, tag(0, T_PROMPT))
    return np.array([L.vxo_uniform_u32(st, i, vocab) for i in range(n)], np.uint32)


def q4_0_quantize(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    rows, k = x.shape
    out = np.empty((rows, (k // 32) * 18), np.uint8)
    for r in range(rows):
        lib().vxo_q4_0_quantize_row(fptr(x[r]), k, u8ptr(out[r]))
    return out


def q4_0_dequant(blocks: np.ndarray, k: int) -> np.ndarray:
    blocks = np.ascontiguousarray(blocks, np.uint8)
    rows = blocks.shape[0]
    out = np.empty((rows, k), np.float32)
    for r in range(rows):
        lib().vxo_q4_0_dequant_row(u8ptr(blocks[r]), k, fptr(out[r]))
    return out


def g64_quantize(x: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """The reference's group-64 codec over consecutive groups of 64 values: packed words
    [n_groups][8] uint32 and (s, m) fp16 bits [n_groups][2]."""
    x = np.ascontiguousarray(x, np.float32).ravel()
    ng = x.size // 64
    packed = np.empty((ng, 8), np.uint32)
    sm = np.empty((ng, 2), np.uint16)
    lib().vxo_g64_quantize(fptr(x), ng, packed.ctypes.data_as(C.POINTER(C.c_uint32)),
                           sm.ctypes.data_as(C.POINTER(C.c_uint16)))
    return packed, sm


def g64_dequant(packed: np.ndarray, sm: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, np.uint32)
    sm = np.ascontiguousarray(sm, np.uint16)
    out = np.empty(packed.size * 8, np.float32)
    lib().vxo_g64_dequant(packed.ctypes.data_as(C.POINTER(C.c_uint32)), sm.ctypes.data_as(C.POINTER(C.c_uint16)),
                          packed.size // 8, fptr(out))
    return out


def rmsnorm(x, w, eps):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty_like(x)
    lib().vxo_rmsnorm(fptr(out), fptr(x), fptr(w), x.size, eps)
    return out


def matmul_transposed(x, w):
    x = np.ascontiguousarray(x, np.float32)
    w = np.ascontiguousarray(w, np.float32)
    out = np.empty(w.shape[0], np.float32)
    lib().vxo_matmul_transposed(fptr(out), fptr(x), fptr(w), w.shape[1], w.shape[0])
    return out


def matmul_q4_0(x, blocks, k, threads=1):
    x = np.ascontiguousarray(x, np.float32)
    blocks = np.ascontiguousarray(blocks, np.uint8)
    out = np.empty(blocks.shape[0], np.float32)
    lib().vxo_matmul_q4_0(fptr(out), fptr(x), u8ptr(blocks), k, blocks.shape[0], threads)
    return out


def rope(t, num_heads, head_dim, pos, theta):
    t = np.array(t, np.float32, copy=True)
    lib().vxo_rope_rotate_half(fptr(t), num_heads, head_dim, pos, theta)
    return t


def attention(q, k_layer, v_layer, n_q, n_kv, head_dim, pos):
    q = np.ascontiguousarray(q, np.float32)
    k_layer = np.ascontiguousarray(k_layer, np.float32)
    v_layer = np.ascontiguousarray(v_layer, np.float32)
    out = np.empty(n_q * head_dim, np.float32)
    scores = np.empty(pos + 1, np.float32)
    lib().vxo_gqa_attention_step(fptr(out), fptr(scores), fptr(q), fptr(k_layer), fptr(v_layer),
                                 n_q, n_kv, head_dim, pos)
    return out


def swiglu(gate, up):
    g = np.array(gate, np.float32, copy=True)
    up = np.ascontiguousarray(up, np.float32)
    lib().vxo_swiglu_act(fptr(g), fptr(up), g.size)
    return g


def argmax(logits):
    logits = np.ascontiguousarray(logits, np.float32)
    return int(lib().vxo_argmax(fptr(logits), logits.size))


class Engine:
    """Whole-model oracle (src/runtime.rs VeloxStaticExecutionEngine restated)."""

    def __init__(self, cfg: dict, seed: int, sigma: float = 0.02, norm_sigma: float = 0.0,
                 q4_0: bool = True, kv_bf16: bool = True, layers_to_build: int | None = None,
                 threads: int = 1, w_f16: bool = False, w_g64: bool = False):
        self.cfg = dict(cfg)
        c = VxoConfig()
        c.vocab_size = cfg["vocab_size"]
        c.hidden_dim = cfg["hidden_dim"]
        c.intermediate_dim = cfg["intermediate_dim"]
        c.num_layers = cfg["num_layers"]
        c.num_heads = cfg["num_heads"]
        c.num_kv_heads = cfg["num_kv_heads"]
        c.head_dim = cfg["head_dim"]
        c.max_seq_len = cfg["max_seq_len"]
        c.rms_norm_eps = cfg["rms_norm_eps"]
        c.rope_theta = cfg["rope_theta"]
        c.qkv_bias = int(cfg.get("qkv_bias", 0))
        c.tied_lm_head = int(cfg.get("tied_lm_head", 0))
        c.q4_0 = int(q4_0)
        c.kv_bf16 = int(kv_bf16)
        c.w_f16 = int(w_f16)
        c.w_g64 = int(w_g64)
        self._c = c
        nl = cfg["num_layers"] if layers_to_build is None else layers_to_build
        self.layers = min(nl, cfg["num_layers"])
        self.h = lib().vxo_engine_create(C.byref(c), seed, sigma, norm_sigma, self.layers, threads)
        self.logits = np.zeros(cfg["vocab_size"], np.float32)

    def forward(self, token: int, pos: int, layers: int | None = None) -> int:
        if layers is None:
            return int(lib().vxo_engine_forward(self.h, token, pos, fptr(self.logits)))
        return int(lib().vxo_engine_forward_layers(self.h, token, pos, layers, fptr(self.logits)))

    def reset(self):
        lib().vxo_engine_reset(self.h)

    def set_threads(self, n: int):
        lib().vxo_engine_set_threads(self.h, n)

    def tensor(self, kind: int, layer: int = 0) -> np.ndarray:
        n = C.c_uint64(0)
        p = lib().vxo_engine_tensor(self.h, kind, layer, C.byref(n))
        if not p:
            raise KeyError((kind, layer))
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), shape=(n.value,)).copy()

    def tensor_view(self, kind: int, layer: int = 0) -> np.ndarray:
        """Writable uint8 view of a tensor's storage (tests plant closed-form weights through it)."""
        n = C.c_uint64(0)
        p = lib().vxo_engine_tensor(self.h, kind, layer, C.byref(n))
        if not p:
            raise KeyError((kind, layer))
        return np.ctypeslib.as_array(C.cast(p, C.POINTER(C.c_uint8)), shape=(n.value,))

    def hidden(self) -> np.ndarray:
        p = lib().vxo_engine_hidden(self.h)
        return np.ctypeslib.as_array(p, shape=(self.cfg["hidden_dim"],)).copy()

    def kv_cache(self, layer: int) -> tuple[np.ndarray, np.ndarray]:
        """Writable views of layer `layer`'s K and V caches, [max_seq_len][num_kv_heads * head_dim]
        fp32 (src/runtime.rs:1328-1451 keeps them per layer, position-major)."""
        kvd = self.cfg["num_kv_heads"] * self.cfg["head_dim"]
        n = self.cfg["max_seq_len"] * kvd
        views = []
        for fn in (lib().vxo_engine_k_cache, lib().vxo_engine_v_cache):
            base = np.ctypeslib.as_array(fn(self.h), shape=(self.cfg["num_layers"] * n,))
            views.append(base[layer * n:(layer + 1) * n].reshape(self.cfg["max_seq_len"], kvd))
        return views[0], views[1]

    def forward_forced(self, token: int, pos: int, k_rows: np.ndarray, v_rows: np.ndarray):
        """One step that attends with the given K/V rows ([layers][kv_heads * head_dim] fp32) at `pos`
        in place of its own; returns (token, the K rows, the V rows it computed)."""
        k_rows = np.ascontiguousarray(k_rows, np.float32)
        v_rows = np.ascontiguousarray(v_rows, np.float32)
        kvd = self.cfg["num_kv_heads"] * self.cfg["head_dim"]
        assert k_rows.shape == v_rows.shape == (self.layers, kvd)
        seen_k, seen_v = np.zeros_like(k_rows), np.zeros_like(v_rows)
        lib().vxo_engine_force_kv(self.h, fptr(k_rows), fptr(v_rows), fptr(seen_k), fptr(seen_v))
        t = int(lib().vxo_engine_forward(self.h, token, pos, fptr(self.logits)))
        return t, seen_k, seen_v

    def close(self):
        if self.h:
            lib().vxo_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class RefSmolLM:
    """The reference's emitted C99 SmolLM module compiled in place (oracle/_ref)."""

    def __init__(self, seed: int, sigma: float = 0.02, norm_sigma: float = 0.0):
        if not os.path.exists(REF_PATH):
            raise FileNotFoundError(REF_PATH)
        L = C.CDLL(REF_PATH)
        L.vxr_smollm_init.restype = C.c_int
        L.vxr_smollm_init.argtypes = [C.c_uint64, C.c_float, C.c_float]
        L.vxr_smollm_step.restype = C.c_uint32
        L.vxr_smollm_step.argtypes = [C.c_uint32, C.c_uint64, C.POINTER(C.c_float)]
        L.vxr_smollm_free.argtypes = []
        self.L = L
        if L.vxr_smollm_init(seed, sigma, norm_sigma) != 0:
            raise MemoryError("reference arena allocation failed")
        self.logits = np.zeros(49152, np.float32)

    def step(self, token: int, pos: int) -> int:
        return int(self.L.vxr_smollm_step(token, pos, fptr(self.logits)))

    def close(self):
        self.L.vxr_smollm_free()


# ---- fp8 e4m3fn block format and the absorbed MLA layer (benchmark configuration 4) ----
MLA_TAGS = dict(norm=32, q_a=33, q_a_norm=34, q_b=35, kv_a=36, kv_a_norm=37, kv_b=38, o=39, hidden=40, cache=41)


def e4m3_encode(x: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.vxo_f32_to_e4m3(float(v)) for v in np.asarray(x, np.float32).ravel()], np.uint8)


def e4m3_decode(b: np.ndarray) -> np.ndarray:
    L = lib()
    return np.array([L.vxo_e4m3_to_f32(int(v)) for v in np.asarray(b, np.uint8).ravel()], np.float32)


def fp8_quantize(w: np.ndarray):
    """w [rows][cols] fp32 -> (codes uint8 [rows][cols], scales [ceil(rows/128)][ceil(cols/128)])."""
    w = np.ascontiguousarray(w, np.float32)
    rows, cols = w.shape
    codes = np.zeros((rows, cols), np.uint8)
    scales = np.zeros(((rows + 127) // 128, (cols + 127) // 128), np.float32)
    lib().vxo_fp8_quantize(fptr(w), rows, cols, u8ptr(codes), fptr(scales))
    return codes, scales


def fp8_dequant(codes: np.ndarray, scales: np.ndarray) -> np.ndarray:
    codes = np.ascontiguousarray(codes, np.uint8)
    rows, cols = codes.shape
    out = np.zeros((rows, cols), np.float32)
    lib().vxo_fp8_dequant(u8ptr(codes), fptr(np.ascontiguousarray(scales, np.float32)), rows, cols, fptr(out))
    return out


def fp8_synth_matrix(seed: int, tg: int, rows: int, cols: int, sigma: float):
    """Seeded N(0, sigma) matrix as fp8 blocks: (codes, scales, dequantized fp32)."""
    codes = np.zeros((rows, cols), np.uint8)
    scales = np.zeros(((rows + 127) // 128, (cols + 127) // 128), np.float32)
    deq = np.zeros((rows, cols), np.float32)
    lib().vxo_fp8_synth_matrix(seed, tg, rows, cols, sigma, u8ptr(codes), fptr(scales), fptr(deq))
    return codes, scales, deq


def mla_config(hidden, n_heads, q_lora, kv_lora, d_nope, d_rope, d_v, kv_norm=1, max_seq=64, eps=1e-6,
               rope_theta=10000.0, scale=None) -> VxoMlaConfig:
    if scale is None:
        scale = 1.0 / np.sqrt(np.float32(d_nope + d_rope))
    return VxoMlaConfig(hidden, n_heads, q_lora, kv_lora, d_nope, d_rope, d_v, kv_norm, max_seq, eps, rope_theta,
                        float(scale))


def mla_layer_step(cfg: VxoMlaConfig, w: dict, cache: np.ndarray, h: np.ndarray, pos: int,
                   cache_bf16: bool = True) -> np.ndarray:
    """One absorbed-MLA decode step (vxo_mla_layer_step); cache [max_seq][kv_lora + d_rope] is updated."""
    keep = {k: np.ascontiguousarray(v, np.float32) for k, v in w.items() if v is not None}
    nul = C.POINTER(C.c_float)()
    ws = VxoMlaWeights(*[fptr(keep[n]) if n in keep else nul for n in
                         ("norm", "q_a", "q_a_norm", "q_b", "kv_a", "kv_a_norm", "kv_b", "o")])
    h = np.ascontiguousarray(h, np.float32)
    out = np.zeros_like(h)
    assert cache.dtype == np.float32 and cache.flags.c_contiguous
    lib().vxo_mla_layer_step(C.byref(cfg), C.byref(ws), fptr(cache), int(cache_bf16), fptr(h), fptr(out), pos)
    return out


def mla_synth_weights(cfg: VxoMlaConfig, seed: int, sigma: float = 0.02, norm_sigma: float = 0.0, layer: int = 0):
    """The seeded fp8 MLA layer (device synthesizer's recipe): dequantized fp32 weights by name."""
    H, nh, ql, lr = cfg.hidden, cfg.n_heads, cfg.q_lora, cfg.kv_lora
    dq, R = cfg.d_nope + cfg.d_rope, cfg.kv_lora + cfg.d_rope
    t = lambda k: tag(layer, MLA_TAGS[k])
    w = {}
    w["q_a"] = fp8_synth_matrix(seed, t("q_a"), ql, H, sigma)[2] if ql else None
    w["q_b"] = fp8_synth_matrix(seed, t("q_b"), nh * dq, ql if ql else H, sigma)[2]
    w["kv_a"] = fp8_synth_matrix(seed, t("kv_a"), R, H, sigma)[2]
    w["kv_b"] = fp8_synth_matrix(seed, t("kv_b"), nh * (cfg.d_nope + cfg.d_v), lr, sigma)[2]
    w["o"] = fp8_synth_matrix(seed, t("o"), H, nh * cfg.d_v, sigma)[2]
    vec = lambda k, n: (fill_normal(n, seed, t(k), norm_sigma, 1.0) if norm_sigma else np.ones(n, np.float32))
    w["norm"] = vec("norm", H)
    w["q_a_norm"] = vec("q_a_norm", ql) if ql else None
    w["kv_a_norm"] = vec("kv_a_norm", lr) if cfg.kv_norm else None
    return w
