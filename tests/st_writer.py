"""Writes safetensors files for the tests: the reference's own test writer pattern
(MmapSafetensors::write_safetensors_file, src/runtime.rs:537-579) -- an 8-byte little-endian header
length, the JSON header padded with spaces to an 8-byte boundary, then the tensors back to back --
plus raw writers for malformed files, and the Hugging Face tensor names a model's checkpoint holds
(src/runtime.rs:1273-1300)."""
from __future__ import annotations

import json
import struct

import numpy as np

_NP = {"F32": np.float32, "F16": np.float16}


def to_dtype(a: np.ndarray, dtype: str) -> bytes:
    """fp32 values stored as F32, F16 (nearest even) or BF16 (nearest even, the top half of fp32)."""
    a = np.ascontiguousarray(a, np.float32)
    if dtype in _NP:
        return a.astype(_NP[dtype]).tobytes()
    if dtype == "BF16":
        u = a.view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        return r.tobytes()
    raise ValueError(dtype)


def from_bf16(raw: bytes) -> np.ndarray:
    return (np.frombuffer(raw, np.uint16).astype(np.uint32) << 16).view(np.float32)


def write(path: str, tensors: list[tuple[str, str, tuple, bytes]], metadata: dict | None = None) -> None:
    """tensors: (name, dtype, shape, data bytes) in file order."""
    header, off = {}, 0
    if metadata is not None:
        header["__metadata__"] = metadata
    for name, dt, shape, data in tensors:
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(data)]}
        off += len(data)
    h = json.dumps(header, separators=(",", ":"))
    while (8 + len(h)) % 8:
        h += " "
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h.encode())
        for _, _, _, data in tensors:
            f.write(data)


def write_raw(path: str, header: bytes | str, payload: bytes = b"", header_len: int | None = None) -> None:
    """A file with an arbitrary header (for malformed-input tests)."""
    hb = header.encode() if isinstance(header, str) else header
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(hb) if header_len is None else header_len))
        f.write(hb)
        f.write(payload)


def hf_names(cfg: dict) -> list[tuple[str, int, int, tuple]]:
    """(name, oracle tensor kind, layer, shape) of every tensor a decoder checkpoint holds."""
    from oracle import pyoracle as po

    H, F, D = cfg["hidden_dim"], cfg["intermediate_dim"], cfg["head_dim"]
    qd, kvd = cfg["num_heads"] * D, cfg["num_kv_heads"] * D
    out = [("model.embed_tokens.weight", po.T_EMBED, 0, (cfg["vocab_size"], H))]
    for li in range(cfg["num_layers"]):
        p = f"model.layers.{li}."
        out += [(p + "input_layernorm.weight", po.T_ATTN_NORM, li, (H,)),
                (p + "self_attn.q_proj.weight", po.T_Q, li, (qd, H)),
                (p + "self_attn.k_proj.weight", po.T_K, li, (kvd, H)),
                (p + "self_attn.v_proj.weight", po.T_V, li, (kvd, H))]
        if cfg.get("qkv_bias"):
            out += [(p + "self_attn.q_proj.bias", po.T_BQ, li, (qd,)),
                    (p + "self_attn.k_proj.bias", po.T_BK, li, (kvd,)),
                    (p + "self_attn.v_proj.bias", po.T_BV, li, (kvd,))]
        out += [(p + "self_attn.o_proj.weight", po.T_O, li, (H, qd)),
                (p + "post_attention_layernorm.weight", po.T_MLP_NORM, li, (H,)),
                (p + "mlp.gate_proj.weight", po.T_GATE, li, (F, H)),
                (p + "mlp.up_proj.weight", po.T_UP, li, (F, H)),
                (p + "mlp.down_proj.weight", po.T_DOWN, li, (H, F))]
    out.append(("model.norm.weight", po.T_FINAL_NORM, 0, (H,)))
    if not cfg.get("tied_lm_head"):
        out.append(("lm_head.weight", po.T_HEAD, 0, (cfg["vocab_size"], H)))
    return out


def write_oracle_model(path: str, ref, cfg: dict, dtype: str = "F32") -> None:
    """The oracle engine's fp32 weights (the build's seeded recipe) as a checkpoint, in `dtype`."""
    tensors = []
    for name, kind, layer, shape in hf_names(cfg):
        w = np.ascontiguousarray(ref.tensor(kind, layer)).view(np.float32).reshape(shape)
        tensors.append((name, dtype, shape, to_dtype(w, dtype)))
    write(path, tensors)
