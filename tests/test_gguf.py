"""GGUF Q4_0 checkpoints (the container the reference's K2 runner reads,
src/runners/velox_cuda_runner_k2.cu:48-196): directory and configuration parsing and malformed
files on the CPU; on the GPU, a model loaded from a GGUF file written from the oracle's synthetic
weights decodes bit-identically to the same model synthesized on the device (llama's permuted q/k
rows, qwen2's biases and tied head), and the runner binary reads it with --weights."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

from velox_amd import _lib as L

from gguf_writer import GT_F16, GT_F32, GT_Q4_0, T_STR, T_U32, llama_permute_rows, model_to_gguf, write_gguf

TINY = dict(vocab_size=512, hidden_dim=128, intermediate_dim=256, num_layers=2, num_heads=2, num_kv_heads=1,
            head_dim=64, rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=0)


def _open(path):
    g = C.c_void_p()
    rc = L.load().velox_hip_gguf_open(str(path).encode(), C.byref(g))
    return rc, g


def test_llama_permutation_closed_form():
    """Row 2i + j of a head in the file is rotate-half row j * D/2 + i."""
    rows = np.arange(2 * 8).reshape(16, 1)
    p = llama_permute_rows(rows, 2).ravel()
    for h in range(2):
        for i in range(4):
            for j in range(2):
                assert p[h * 8 + 2 * i + j] == h * 8 + j * 4 + i


def test_gguf_directory_and_config(oracle, tmp_path):
    eng = oracle.Engine(dict(TINY, max_seq_len=64), seed=3, sigma=0.02, q4_0=True, kv_bf16=True)
    path = tmp_path / "tiny.gguf"
    model_to_gguf(path, eng, TINY, "llama", context_length=2048)
    eng.close()
    lib = L.load()
    rc, g = _open(path)
    assert rc == 0
    n = lib.velox_hip_gguf_tensor_count(g)
    assert n == 1 + 2 * 9 + 2
    name = C.create_string_buffer(128)
    t, nd, nb = C.c_uint32(), C.c_uint32(), C.c_uint64()
    dims = (C.c_uint64 * 4)()
    seen = {}
    for i in range(n):
        L.check(lib.velox_hip_gguf_tensor_info(g, i, name, 128, C.byref(t), C.byref(nd), dims, C.byref(nb)))
        seen[name.value.decode()] = (t.value, nd.value, tuple(dims[:nd.value]), nb.value)
    assert seen["token_embd.weight"] == (GT_Q4_0, 2, (128, 512), 512 * 4 * 18)
    assert seen["blk.1.ffn_down.weight"] == (GT_Q4_0, 2, (256, 128), 128 * 8 * 18)
    assert seen["blk.0.ffn_norm.weight"] == (GT_F16, 1, (128,), 256)
    assert seen["output_norm.weight"] == (GT_F32, 1, (128,), 512)
    cfg = L.ModelConfig()
    L.check(lib.velox_hip_gguf_config(g, 0, C.byref(cfg)))
    assert cfg.name == b"llama" and cfg.max_seq_len == 2048
    for k, v in TINY.items():
        assert getattr(cfg, k) == pytest.approx(v), k
    lib.velox_hip_gguf_close(g)


def test_gguf_rejects_malformed(tmp_path):
    good = tmp_path / "g.gguf"
    write_gguf(good, [("general.architecture", T_STR, "llama"), ("llama.block_count", T_U32, 1)],
               [("x.weight", [32, 2], GT_Q4_0, bytes(36))])
    assert _open(good)[0] == 0
    data = good.read_bytes()
    cases = {
        "magic": b"GGUX" + data[4:],
        "version": data[:4] + (9).to_bytes(4, "little") + data[8:],
        "truncated_header": data[:30],
        "truncated_data": data[:-10],
        "huge_kv_count": data[:16] + (1 << 40).to_bytes(8, "little") + data[24:],
        "empty": b"",
    }
    for label, blob in cases.items():
        p = tmp_path / f"{label}.gguf"
        p.write_bytes(blob)
        assert _open(p)[0] == L.ESHAPE, label
    assert _open(tmp_path / "missing.gguf")[0] == L.EINVAL


@pytest.mark.gpu
@pytest.mark.parametrize("arch,cfg", [
    ("llama", TINY),
    ("qwen2", dict(TINY, qkv_bias=1, tied_lm_head=1, num_heads=4, num_kv_heads=2, hidden_dim=256, head_dim=64,
                   rope_theta=1000000.0, rms_norm_eps=1e-6)),
])
def test_gguf_model_decodes_like_synthesized(oracle, tmp_path, arch, cfg):
    from velox_amd.engine import HipDecodeEngine
    seed = 21
    eng = oracle.Engine(dict(cfg, max_seq_len=64), seed=seed, sigma=0.02, q4_0=True, kv_bf16=True)
    path = str(tmp_path / f"{arch}.gguf")
    model_to_gguf(path, eng, cfg, arch)
    eng.close()
    a = HipDecodeEngine(cfg, seed=seed, max_seq_len=64)
    b = HipDecodeEngine(path, max_seq_len=64)
    assert b.cfg.vocab_size == cfg["vocab_size"] and b.cfg.qkv_bias == cfg["qkv_bias"]
    toks = oracle.prompt_tokens(seed, 6, cfg["vocab_size"])
    for pos, tok in enumerate(toks):
        ta = a.forward_step(int(tok), pos)
        tb = b.forward_step(int(tok), pos)
        assert ta == tb and np.array_equal(a.logits, b.logits), (arch, pos)
    a.close()
    b.close()


@pytest.mark.gpu
def test_runner_reads_gguf(oracle, tmp_path):
    """`velox_hip_runner --weights file.gguf` generates the same tokens as the synthesized model of
    the same seed (GGUF metadata defines the shapes)."""
    runner = os.path.join(os.path.dirname(L.LIB_PATH), "velox_hip_runner")
    cfg = dict(TINY, num_layers=2)
    eng = oracle.Engine(dict(cfg, max_seq_len=64), seed=1234, sigma=0.02, q4_0=True, kv_bf16=True)
    path = str(tmp_path / "r.gguf")
    model_to_gguf(path, eng, cfg, "llama")
    eng.close()
    out = subprocess.run([runner, "--weights", path, "--tokens", "5,9,2", "--steps", "6", "--warmup", "0"],
                         capture_output=True, text=True, timeout=120)
    assert out.returncode == 0, out.stderr
    got = [int(l.split(":")[1]) for l in out.stdout.splitlines() if l.startswith("[Step ")]
    from velox_amd.engine import HipDecodeEngine
    e = HipDecodeEngine(cfg, seed=1234, max_seq_len=64)
    want = []
    for pos, tok in enumerate([5, 9, 2]):
        t = e.forward_step(tok, pos)
    want.append(t)
    for pos in range(3, 3 + len(got) - 1):
        t = e.forward_step(t, pos)
        want.append(t)
    e.close()
    assert got == want
    assert "GGUF Q4_0" in out.stdout
