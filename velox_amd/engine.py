"""Host-side mirror of the reference's engine interface over the HIP decode backend.

``HipDecodeEngine`` offers the call surface of ``VeloxStaticExecutionEngine``
(src/runtime.rs:1229-1502): ``forward_step(token, pos) -> next token`` with ``logits`` filled,
and ``generate_greedy_into(prompt, n)``; underneath, every step is one launch sequence of the
hand-written gfx950 kernels behind include/velox_hip.h (optionally replayed as a hipGraph, as the
reference runner does, src/runners/velox_cuda_runner.cu:471-540). Weights are the seeded synthetic
Q4_0 model synthesized on the device.
"""
from __future__ import annotations

import ctypes as C

import numpy as np

from . import _lib as L


def gguf_config(path: str, max_seq_len: int = 0) -> L.ModelConfig:
    """The model configuration a GGUF checkpoint's metadata defines (velox_hip_gguf_config)."""
    lib = L.load()
    g = C.c_void_p()
    L.check(lib.velox_hip_gguf_open(path.encode(), C.byref(g)), "gguf_open")
    try:
        cfg = L.ModelConfig()
        L.check(lib.velox_hip_gguf_config(g, max_seq_len, C.byref(cfg)), "gguf_config")
    finally:
        lib.velox_hip_gguf_close(g)
    return cfg


class Safetensors:
    """A memory-mapped safetensors checkpoint (velox_hip_st_*): the reference runner's --weights format."""

    def __init__(self, path: str):
        self.lib = L.load()
        self.handle = C.c_void_p()
        L.check(self.lib.velox_hip_st_open(path.encode(), C.byref(self.handle)), f"st_open {path}")

    def config(self, max_seq_len: int = 0) -> L.ModelConfig:
        cfg = L.ModelConfig()
        L.check(self.lib.velox_hip_st_config(self.handle, max_seq_len, C.byref(cfg)), "st_config")
        return cfg

    def names(self) -> list[str]:
        out = []
        buf = C.create_string_buffer(256)
        for i in range(int(self.lib.velox_hip_st_tensor_count(self.handle))):
            L.check(self.lib.velox_hip_st_tensor_info(self.handle, i, buf, 256, None, None, None, None, None))
            out.append(buf.value.decode())
        return out

    def close(self) -> None:
        if self.handle:
            self.lib.velox_hip_st_close(self.handle)
            self.handle = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


def safetensors_config(path: str, max_seq_len: int = 0) -> L.ModelConfig:
    """The model a safetensors checkpoint holds (velox_hip_st_config)."""
    with Safetensors(path) as st:
        return st.config(max_seq_len)


def vlx_config(path: str, max_seq_len: int = 0) -> tuple[L.ModelConfig, L.VlxTarget]:
    """The model configuration and target a .vlx model source declares (velox_hip_vlx_load)."""
    lib = L.load()
    cfg, tgt = L.ModelConfig(), L.VlxTarget()
    L.check(lib.velox_hip_vlx_load(path.encode(), max_seq_len, C.byref(cfg), C.byref(tgt)), f"vlx_load {path}")
    return cfg, tgt


def make_config(model, max_seq_len: int = 0, num_layers: int = 0, attn_splits: int = 0,
                max_batch: int = 0, prefill_chunk: int = 0, quant_mode: int | None = None) -> L.ModelConfig:
    """A builtin config by name, a GGUF file (path ending in .gguf), a safetensors checkpoint (path
    ending in .safetensors), a .vlx model source (path ending in .vlx, read by velox_hip_vlx_load), or a
    dict of ModelConfig fields (custom shapes for tests).
    `quant_mode` overrides the weight format (L.QUANT_F32 / L.QUANT_F16 rows, L.QUANT_GGML_Q4_0)."""
    if isinstance(model, str) and model.endswith(".gguf"):
        cfg = gguf_config(model, max_seq_len)
    elif isinstance(model, str) and model.endswith(".safetensors"):
        cfg = safetensors_config(model, max_seq_len)
    elif isinstance(model, str) and model.endswith(".vlx"):
        cfg = vlx_config(model, max_seq_len)[0]
    elif isinstance(model, str):
        cfg = L.builtin_config(model, max_seq_len)
    else:
        cfg = L.ModelConfig()
        d = dict(model)
        cfg.name = d.pop("name", "custom").encode()
        cfg.quant_mode = L.QUANT_GGML_Q4_0
        for k, v in d.items():
            setattr(cfg, k, v)
        if max_seq_len:
            cfg.max_seq_len = max_seq_len
    if num_layers:
        cfg.num_layers = num_layers
    if attn_splits:
        cfg.attn_splits = attn_splits
    if max_batch:
        cfg.max_batch = max_batch
    if prefill_chunk:
        cfg.prefill_chunk = prefill_chunk
    if quant_mode is not None:
        cfg.quant_mode = quant_mode
    return cfg


def set_fused_attention(enable: bool) -> None:
    """Process-wide: steps recorded afterwards run QKV and attention as one launch per layer where
    the plan allows it (the default), or always as two."""
    L.load().velox_hip_set_fused_attention(1 if enable else 0)


class HipDecodeEngine:
    def __init__(self, model, seed: int = 0, sigma: float = 0.02, norm_sigma: float = 0.0,
                 max_seq_len: int = 0, num_layers: int = 0, attn_splits: int = 0, synthesize: bool = True,
                 max_batch: int = 0, prefill_chunk: int = 0, quant_mode: int | None = None):
        self.lib = L.load()
        self.cfg = make_config(model, max_seq_len, num_layers, attn_splits, max_batch, prefill_chunk, quant_mode)
        self._model = C.c_void_p()
        L.check(self.lib.velox_hip_model_create(C.byref(self.cfg), C.byref(self._model)), "model_create")
        self.arena = L.Arena()
        L.check(self.lib.velox_hip_arena_create(self._model, C.byref(self.arena)), "arena_create")
        self.vocab = self.cfg.vocab_size
        self.logits_off = self.lib.velox_hip_model_logits_offset(self._model)
        self.hidden_off = self.lib.velox_hip_model_hidden_offset(self._model)
        self.logits = np.zeros(self.vocab, np.float32)
        self._graph = None
        if isinstance(model, str) and model.endswith(".gguf"):
            g = C.c_void_p()
            L.check(self.lib.velox_hip_gguf_open(model.encode(), C.byref(g)), "gguf_open")
            try:
                L.check(self.lib.velox_hip_gguf_load(C.byref(self.arena), g, None), "gguf_load")
            finally:
                self.lib.velox_hip_gguf_close(g)
        elif isinstance(model, str) and model.endswith(".safetensors"):
            self.load_safetensors(model)
        elif synthesize:
            L.check(self.lib.velox_hip_synthesize_model(C.byref(self.arena), seed, sigma, norm_sigma, None),
                    "synthesize_model")

    # -- plan ---------------------------------------------------------------------------------
    def step_bytes(self, pos: int) -> int:
        return int(self.lib.velox_hip_model_step_bytes(self._model, pos))

    def arena_bytes(self) -> dict:
        v = [C.c_uint64() for _ in range(5)]
        L.check(self.lib.velox_hip_model_arena_bytes(self._model, *[C.byref(x) for x in v]))
        return dict(zip(["weights", "scales", "norms", "kv", "activations"], [x.value for x in v]))

    # -- loaders ------------------------------------------------------------------------------
    def load_q4_0(self, kind: int, layer: int, blocks: np.ndarray) -> None:
        blocks = np.ascontiguousarray(blocks, np.uint8)
        L.check(self.lib.velox_hip_load_q4_0(C.byref(self.arena), kind, layer, blocks.ctypes.data, blocks.nbytes,
                                             None), "load_q4_0")

    def load_safetensors(self, path: str) -> None:
        """Every tensor of a safetensors checkpoint, converted on the device to this arena's format."""
        with Safetensors(path) as st:
            L.check(self.lib.velox_hip_st_load(C.byref(self.arena), st.handle, None), f"st_load {path}")

    def load_f32(self, kind: int, layer: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data, np.float32)
        L.check(self.lib.velox_hip_load_f32(C.byref(self.arena), kind, layer, data.ctypes.data, data.size, None),
                "load_f32")

    def fill_kv(self, layer: int, n_pos: int, seed: int, sigma: float = 1.0) -> None:
        L.check(self.lib.velox_hip_fill_kv(C.byref(self.arena), layer, n_pos, seed, sigma, None), "fill_kv")

    # -- state --------------------------------------------------------------------------------
    def set_prompt(self, tokens) -> None:
        arr = (C.c_uint32 * len(tokens))(*[int(t) for t in tokens])
        L.check(self.lib.velox_hip_set_prompt(C.byref(self.arena), arr, len(tokens), None), "set_prompt")

    def set_state(self, step: int, token: int) -> None:
        L.check(self.lib.velox_hip_set_state(C.byref(self.arena), step, token, None), "set_state")

    def state(self) -> tuple[int, int]:
        s = L.DecodeState()
        L.check(self.lib.velox_hip_get_state(C.byref(self.arena), C.byref(s), None), "get_state")
        return int(s.step), int(s.token)

    def sync(self) -> None:
        rc = L.hip().hipDeviceSynchronize()
        if rc != 0:
            raise RuntimeError(f"hipDeviceSynchronize failed: {rc}")
        err = self.lib.velox_hip_last_error()
        if err != 0:
            raise RuntimeError(f"decode step launch failed: {err}")

    # -- the step -----------------------------------------------------------------------------
    def forward_step(self, token: int, pos: int) -> int:
        """src/runtime.rs:1328-1451: one token at position pos; fills self.logits."""
        self.lib.velox_hip_decode(C.byref(self.arena), int(token), int(pos), 1, None)
        self.sync()
        self.read_logits()
        return int(self.arena.host_pinned_ring[pos & (L.RING_SIZE - 1)])

    def prefill_batch(self, pos0: int, n_tokens: int) -> None:
        """Positions [pos0, pos0 + n_tokens) of the staged prompt as batched chunks of
        cfg.prefill_chunk rows (the token-by-token prefill of velox_cuda_runner.cu:493-512 in one
        weight pass per chunk); leaves the state where that many prefill steps would."""
        L.check(self.lib.velox_hip_prefill_batch(C.byref(self.arena), int(pos0), int(n_tokens), 1, None),
                "prefill_batch")
        self.sync()

    def chunk_logits(self, n_rows: int) -> np.ndarray:
        """The last prefill chunk's logits, one row per position."""
        lo = C.c_uint64()
        L.check(self.lib.velox_hip_model_batch_layout(self._model, None, C.byref(lo), None))
        out = np.empty((n_rows, self.vocab), np.float32)
        L.memcpy_dtoh(out.ctypes.data, self.arena.activation_arena + lo.value, out.nbytes)
        return out

    def fused_status(self) -> tuple[int, int]:
        """(attention splits per KV head of the fused QKV + attention launch, 0 when the step
        launches the two apart; the fused launches' error bits, 0 after correct steps)."""
        used, err = C.c_uint32(), C.c_uint32()
        L.check(self.lib.velox_hip_fused_attention_status(C.byref(self.arena), C.byref(used), C.byref(err)),
                "fused_attention_status")
        return int(used.value), int(err.value)

    def graph_step(self) -> None:
        """One decode step driven by the device state (no host round trip)."""
        self.lib.velox_hip_decode_graph_step(C.byref(self.arena), 1, None)

    def read_logits(self) -> np.ndarray:
        L.memcpy_dtoh(self.logits.ctypes.data, self.arena.activation_arena + self.logits_off, self.logits.nbytes)
        return self.logits

    def read_hidden(self) -> np.ndarray:
        h = np.empty(self.cfg.hidden_dim, np.float32)
        L.memcpy_dtoh(h.ctypes.data, self.arena.activation_arena + self.hidden_off, h.nbytes)
        return h

    def ring(self, pos: int) -> int:
        return int(self.arena.host_pinned_ring[pos & (L.RING_SIZE - 1)])

    def generate_greedy_into(self, prompt, num_new_tokens: int) -> list[int]:
        """src/runtime.rs:1456-1490: prefill token by token, then greedy decode."""
        pos = 0
        nxt = int(prompt[0])
        for tok in prompt:
            nxt = self.forward_step(int(tok), pos)
            pos += 1
        out = []
        if num_new_tokens == 0:
            return out
        out.append(nxt)
        for _ in range(1, num_new_tokens):
            nxt = self.forward_step(nxt, pos)
            pos += 1
            out.append(nxt)
        return out

    def close(self) -> None:
        if getattr(self, "_model", None) and self._model.value:
            self.lib.velox_hip_arena_destroy(C.byref(self.arena))
            self.lib.velox_hip_model_destroy(self._model)
            self._model = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class HipBatchEngine(HipDecodeEngine):
    """Batched decode of up to 32 independent sequences (src/runners/velox_cuda_runner_k2.cu:
    553-1088 batched kernels): each sequence keeps its own KV cache, decode state, prompt and ring;
    one step advances all of them, reading the weights once (MFMA GEMMs)."""

    def __init__(self, model, max_batch: int, **kw):
        super().__init__(model, max_batch=max_batch, **kw)
        mb, lo, ho = C.c_uint32(), C.c_uint64(), C.c_uint64()
        L.check(self.lib.velox_hip_model_batch_layout(self._model, C.byref(mb), C.byref(lo), C.byref(ho)))
        self.max_batch, self.blogits_off, self.bhidden_off = mb.value, lo.value, ho.value

    def fill_kv_seq(self, layer: int, seq: int, n_pos: int, seed: int, sigma: float = 1.0) -> None:
        L.check(self.lib.velox_hip_fill_kv_seq(C.byref(self.arena), layer, seq, n_pos, seed, sigma, None))

    def set_prompt_seq(self, seq: int, tokens) -> None:
        arr = (C.c_uint32 * max(1, len(tokens)))(*[int(t) for t in tokens])
        L.check(self.lib.velox_hip_batch_set_prompt(C.byref(self.arena), seq, arr, len(tokens), None))

    def set_state_seq(self, seq: int, step: int, token: int) -> None:
        L.check(self.lib.velox_hip_batch_set_state(C.byref(self.arena), seq, step, token, None))

    def state_seq(self, seq: int) -> tuple[int, int]:
        s = L.DecodeState()
        L.check(self.lib.velox_hip_batch_get_state(C.byref(self.arena), seq, C.byref(s), None))
        return int(s.step), int(s.token)

    def batch_step(self, batch: int) -> None:
        self.lib.velox_hip_decode_batch_graph_step(C.byref(self.arena), batch, 1, None)

    def logits_seq(self, seq: int) -> np.ndarray:
        out = np.empty(self.vocab, np.float32)
        L.memcpy_dtoh(out.ctypes.data, self.arena.activation_arena + self.blogits_off + seq * self.vocab * 4,
                      out.nbytes)
        return out

    def ring_seq(self, seq: int, pos: int) -> int:
        return int(self.arena.host_pinned_ring[seq * L.RING_SIZE + (pos & (L.RING_SIZE - 1))])

    def step_bytes_batch(self, batch: int, pos: int) -> int:
        return int(self.lib.velox_hip_model_batch_step_bytes(self._model, batch, pos))


def run(model: str = "llama3_8b", prompt_len: int = 128, warmup: int = 5, steps: int = 251, seed: int = 1234,
        sigma: float = 0.02, norm_sigma: float = 0.0, use_graph: bool = True, num_layers: int = 0,
        max_seq_len: int = 0, max_tokens: int = 1024, kernel_passes: int = 0,
        prompt: list[int] | None = None, context_len: int = 0, batch: int = 1,
        prefill_chunk: int = 0, model_file: str | None = None, unquantized: int = 0,
        attn_splits: int = 0) -> tuple[dict, list[int]]:
    """The C++ runner flow (velox_hip_run): synthesize, capture, prefill, timed decode. `prompt`
    replaces the seeded random prompt of `prompt_len` ids; `context_len` > 0 starts from a seeded
    context of that many positions already in the KV cache (then prompt_len must be 1). Returned
    tokens are ring entries, ring[p] = argmax after position p, for the last positions run.
    `prefill_chunk` > 1 prefills the prompt as batched chunks of that many positions. `model_file`
    reads the model from a .vlx source instead of the builtin `model`. `unquantized` 1 / 2 / 3 runs the
    reference's fp32 weights as fp32 rows, fp16 rows or quantized to group-64 (quant_mode 0 / 1 / 2)
    instead of GGML Q4_0."""
    lib = L.load()
    ptoks = None
    if prompt is not None:
        prompt_len = len(prompt)
        ptoks = (C.c_uint32 * prompt_len)(*prompt)
    opt = L.RunOptions(model.encode(), max_seq_len, prompt_len, warmup, steps, seed, sigma, norm_sigma,
                       int(use_graph), num_layers, kernel_passes, 0, ptoks, context_len, batch, None,
                       prefill_chunk, model_file.encode() if model_file else None, unquantized, None, None,
                       attn_splits)
    rep = L.RunReport()
    toks = (C.c_uint32 * max_tokens)()
    rc = lib.velox_hip_run(C.byref(opt), toks, max_tokens, C.byref(rep))
    L.check(rc, "velox_hip_run")
    d = {f: getattr(rep, f) for f, _ in rep._fields_}
    return d, [int(toks[i]) for i in range(rep.n_tokens)]


class MlaEngine:
    """The absorbed multi-head latent attention layer (benchmark configuration 4) behind the C ABI: the
    full form of the reference's ``mla_absorbed_step_f32`` (src/runtime.rs:845-1044), for up to
    32 sequences, with fp8 block-scaled weights and a bf16 latent cache on the device."""

    def __init__(self, cfg: dict | str = "deepseek_v3_mla", max_seq_len: int = 64, max_batch: int = 1,
                 num_layers: int = 1, seed: int = 1, sigma: float = 0.02, norm_sigma: float = 0.0,
                 attn_splits: int = 0, synthesize: bool = True):
        self.lib = L.load()
        c = L.MlaConfig()
        if isinstance(cfg, str):
            L.check(self.lib.velox_hip_mla_builtin_config(cfg.encode(), max_seq_len, max_batch, C.byref(c)), cfg)
        else:
            for k, v in cfg.items():
                setattr(c, k, v)
            c.max_seq_len, c.max_batch = max_seq_len, max_batch
            if not c.rms_norm_eps:
                c.rms_norm_eps = 1e-6
            if not c.rope_theta:
                c.rope_theta = 10000.0
        c.num_layers = num_layers
        c.attn_splits = attn_splits
        self.cfg = c
        self._m = C.c_void_p()
        L.check(self.lib.velox_hip_mla_create(C.byref(c), C.byref(self._m)), "mla_create")
        self.arena = L.Arena()  # the plan's regions as the emitted-runner arena (velox_hip_mla_arena)
        L.check(self.lib.velox_hip_mla_arena(self._m, C.byref(self.arena)), "mla_arena")
        self.buf = L.MlaBuffers()
        L.check(self.lib.velox_hip_mla_buffers(self._m, C.byref(self.buf)), "mla_buffers")
        self.R = c.kv_lora_rank + c.qk_rope_dim
        if synthesize:
            L.check(self.lib.velox_hip_mla_synthesize(self._m, seed, sigma, norm_sigma, None), "mla_synthesize")

    def fill_cache(self, layer: int, seq: int, n_pos: int, seed: int, sigma: float = 1.0) -> None:
        L.check(self.lib.velox_hip_mla_fill_cache(self._m, layer, seq, n_pos, seed, sigma, None), "mla_fill_cache")

    def set_position(self, seq: int, pos: int) -> None:
        L.check(self.lib.velox_hip_mla_set_position(self._m, seq, pos, None), "mla_set_position")

    def set_hidden(self, h: np.ndarray) -> None:
        h = np.ascontiguousarray(h, np.float32)
        L.memcpy_htod(self.buf.hidden, h.ctypes.data, h.nbytes)

    def hidden(self, batch: int) -> np.ndarray:
        out = np.zeros((batch, self.cfg.hidden_dim), np.float32)
        L.memcpy_dtoh(out.ctypes.data, self.buf.hidden, out.nbytes)
        return out

    def cache(self, layer: int, seq: int, n_pos: int) -> np.ndarray:
        """Latent rows [0, n_pos) of one sequence as fp32 (from the bf16 cache)."""
        raw = np.zeros((n_pos, self.R), np.uint16)
        off = ((layer * self.cfg.max_batch + seq) * self.buf.s_cap) * self.R * 2
        L.memcpy_dtoh(raw.ctypes.data, self.buf.latent_cache + off, raw.nbytes)
        return (raw.astype(np.uint32) << 16).view(np.float32)

    def load_fp8(self, kind: int, layer: int, codes: np.ndarray, scales: np.ndarray) -> None:
        codes = np.ascontiguousarray(codes, np.uint8)
        scales = np.ascontiguousarray(scales, np.float32)
        L.check(self.lib.velox_hip_mla_load_fp8(self._m, kind, layer, codes.ctypes.data, scales.ctypes.data, None),
                "mla_load_fp8")

    def load_f32(self, kind: int, layer: int, data: np.ndarray) -> None:
        data = np.ascontiguousarray(data, np.float32)
        L.check(self.lib.velox_hip_mla_load_f32(self._m, kind, layer, data.ctypes.data, data.size, None), "mla_load_f32")

    def step(self, layer: int = 0, batch: int = 1) -> None:
        self.lib.velox_hip_mla_layer_step(self._m, layer, batch, 1, None)
        L.check(L.hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
        L.check(self.lib.velox_hip_last_error(), "mla_layer_step")

    def decode_step(self, batch: int = 1) -> None:
        """Every layer in order (velox_hip_mla_decode_step)."""
        self.lib.velox_hip_mla_decode_step(self._m, batch, 1, None)
        L.check(L.hip().hipDeviceSynchronize(), "hipDeviceSynchronize")
        L.check(self.lib.velox_hip_last_error(), "mla_decode_step")

    def step_bytes(self, batch: int, pos: int) -> float:
        return float(self.lib.velox_hip_mla_step_bytes(self._m, batch, pos))

    def close(self) -> None:
        if self._m:
            self.lib.velox_hip_mla_destroy(self._m)
            self._m = C.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def mla_run(which: str = "deepseek_v3_mla", batch: int = 1, context_len: int = 4096, warmup: int = 5,
            steps: int = 50, seed: int = 1234, layers: int = 1) -> dict:
    """velox_hip_mla_run: synthesize `layers` layers, seed the latent contexts, time graph-replayed
    steps (the decode step over the stack when layers > 1); us_per_layer = step time / layers."""
    rep = L.MlaRunReport()
    L.check(L.load().velox_hip_mla_run(which.encode(), batch, context_len, layers, warmup, steps, seed,
                                       C.byref(rep)), "velox_hip_mla_run")
    return {f: getattr(rep, f) for f, _ in rep._fields_}
