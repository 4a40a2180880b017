"""Writes GGUF files (GGML's container, version 3: little-endian header, typed key/value metadata,
tensor directory, data at general.alignment) for the loader tests, and turns the oracle's
synthetic Q4_0 model into one with llama.cpp's tensor names.

llama.cpp stores llama's q/k projection rows permuted for its pairwise RoPE: within each head,
file row 2i + j holds rotate-half row j * D/2 + i. `model_to_gguf` writes them that way for
arch "llama" (and not for "qwen2"), so the loader's un-permutation is exercised."""
import struct

import numpy as np

GGUF_MAGIC = 0x46554747
T_U32, T_I32, T_F32, T_STR, T_ARR = 4, 5, 6, 8, 9
GT_F32, GT_F16, GT_Q4_0 = 0, 1, 2


def _s(text: str) -> bytes:
    b = text.encode()
    return struct.pack("<Q", len(b)) + b


def write_gguf(path, kv, tensors, alignment=32, version=3):
    """kv: [(key, type, value)] (arrays as (elem_type, values)); tensors: [(name, dims, type, bytes)]
    with dims in GGML order (dims[0] contiguous)."""
    out = bytearray(struct.pack("<IIQQ", GGUF_MAGIC, version, len(tensors), len(kv)))
    for key, t, v in kv:
        out += _s(key) + struct.pack("<I", t)
        if t == T_STR:
            out += _s(v)
        elif t == T_U32:
            out += struct.pack("<I", v)
        elif t == T_F32:
            out += struct.pack("<f", v)
        elif t == T_ARR:
            et, vals = v
            out += struct.pack("<IQ", et, len(vals))
            for x in vals:
                out += _s(x) if et == T_STR else struct.pack("<i", x)
        else:
            raise ValueError(t)
    offsets, off = [], 0
    for _, _, _, data in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offsets.append(off)
        off += len(data)
    for (name, dims, t, _), o in zip(tensors, offsets):
        out += _s(name) + struct.pack("<I", len(dims)) + b"".join(struct.pack("<Q", d) for d in dims)
        out += struct.pack("<IQ", t, o)
    start = (len(out) + alignment - 1) // alignment * alignment
    out += b"\0" * (start - len(out))
    for (_, _, _, data), o in zip(tensors, offsets):
        out += b"\0" * (start + o - len(out))
        out += bytes(data)
    with open(path, "wb") as f:
        f.write(out)
    return start


def llama_permute_rows(rows: np.ndarray, heads: int) -> np.ndarray:
    """Rotate-half row order -> llama.cpp's pairwise order (row 2i + j of a head <- row j*D/2 + i)."""
    n = rows.shape[0]
    d = n // heads
    r = rows.reshape(heads, 2, d // 2, *rows.shape[1:])
    return np.ascontiguousarray(np.swapaxes(r, 1, 2)).reshape(rows.shape)


def model_to_gguf(path, eng, cfg: dict, arch: str, context_length: int = 4096):
    """eng: an oracle Engine built with q4_0=True; cfg: its config dict."""
    H, F, V = cfg["hidden_dim"], cfg["intermediate_dim"], cfg["vocab_size"]
    nh, nkv, D = cfg["num_heads"], cfg["num_kv_heads"], cfg["head_dim"]
    L = cfg["num_layers"]
    row_q4 = lambda k: k // 32 * 18
    kv = [("general.architecture", T_STR, arch), ("general.alignment", T_U32, 32),
          (f"{arch}.embedding_length", T_U32, H), (f"{arch}.block_count", T_U32, L),
          (f"{arch}.feed_forward_length", T_U32, F), (f"{arch}.attention.head_count", T_U32, nh),
          (f"{arch}.attention.head_count_kv", T_U32, nkv),
          (f"{arch}.attention.layer_norm_rms_epsilon", T_F32, cfg["rms_norm_eps"]),
          (f"{arch}.rope.freq_base", T_F32, cfg["rope_theta"]), (f"{arch}.context_length", T_U32, context_length),
          ("tokenizer.ggml.tokens", T_ARR, (T_STR, [f"t{i}" for i in range(7)])),
          ("tokenizer.ggml.token_type", T_ARR, (T_I32, [1, 2, 3]))]
    perm = arch == "llama"
    q4 = lambda kind, layer, rows, k: eng.tensor(kind, layer).reshape(rows, row_q4(k))
    f32 = lambda kind, layer: eng.tensor(kind, layer).view(np.float32)
    tensors = [("token_embd.weight", [H, V], GT_Q4_0, q4(1, 0, V, H).tobytes())]
    for layer in range(L):
        p = f"blk.{layer}."
        wq, wk = q4(2, layer, nh * D, H), q4(3, layer, nkv * D, H)
        if perm:
            wq, wk = llama_permute_rows(wq, nh), llama_permute_rows(wk, nkv)
        tensors += [(p + "attn_q.weight", [H, nh * D], GT_Q4_0, wq.tobytes()),
                    (p + "attn_k.weight", [H, nkv * D], GT_Q4_0, wk.tobytes()),
                    (p + "attn_v.weight", [H, nkv * D], GT_Q4_0, q4(4, layer, nkv * D, H).tobytes()),
                    (p + "attn_output.weight", [nh * D, H], GT_Q4_0, q4(5, layer, H, nh * D).tobytes()),
                    (p + "ffn_gate.weight", [H, F], GT_Q4_0, q4(6, layer, F, H).tobytes()),
                    (p + "ffn_up.weight", [H, F], GT_Q4_0, q4(7, layer, F, H).tobytes()),
                    (p + "ffn_down.weight", [F, H], GT_Q4_0, q4(8, layer, H, F).tobytes()),
                    (p + "attn_norm.weight", [H], GT_F32, f32(9, layer).tobytes()),
                    # fp16 gains exercise the loader's conversion (the oracle's gains are exact in fp16)
                    (p + "ffn_norm.weight", [H], GT_F16, f32(10, layer).astype(np.float16).tobytes())]
        if cfg.get("qkv_bias"):
            bq, bk = f32(13, layer), f32(14, layer)
            if perm:
                bq, bk = llama_permute_rows(bq, nh), llama_permute_rows(bk, nkv)
            tensors += [(p + "attn_q.bias", [nh * D], GT_F32, bq.tobytes()),
                        (p + "attn_k.bias", [nkv * D], GT_F32, bk.tobytes()),
                        (p + "attn_v.bias", [nkv * D], GT_F32, f32(15, layer).tobytes())]
    tensors.append(("output_norm.weight", [H], GT_F32, f32(11, 0).tobytes()))
    if not cfg.get("tied_lm_head"):
        tensors.append(("output.weight", [H, V], GT_Q4_0, q4(12, 0, V, H).tobytes()))
    return write_gguf(path, kv, tensors)
