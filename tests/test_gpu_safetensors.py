"""safetensors checkpoints on the GPU: the reference runner's --weights path (src/cli.rs:653-654,
src/runners/velox_cuda_runner.cu:154-199, 390-393).

The checkpoints are written from the oracle's fp32 tensors (the build's seeded recipe) with the
reference's writer pattern (src/runtime.rs:537-579) and Hugging Face names (src/runtime.rs:1273-1300):
- loaded into every weight format (fp32 rows, fp16 rows, the reference's group-64 format, GGML
  Q4_0 quantized on the device), the model decodes bit for bit like the same model synthesized on
  the device (whose formats the other GPU tests pin to the oracle);
- F16 and BF16 files load like F32 files holding the same values;
- the fp32 SmolLM-135M checkpoint of the golden fixture (the reference's emitted C99 module's
  logits) reproduces its argmax and logits, through the engine and through the runner's own argv.
"""
import json
import os
import re
import subprocess

import numpy as np
import pytest

from velox_amd import _lib as L
from velox_amd.engine import HipDecodeEngine

import st_writer as W

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
RUNNER = os.path.join(os.path.dirname(HERE), "velox_amd", "lib", "velox_hip_runner")
SMOLLM = dict(vocab_size=49152, hidden_dim=576, intermediate_dim=1536, num_layers=30, num_heads=9, num_kv_heads=3,
              head_dim=64, rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=1)
# a Qwen-like decoder with QKV biases and a separate head
QWENISH = dict(vocab_size=1000, hidden_dim=256, intermediate_dim=512, num_layers=2, num_heads=4, num_kv_heads=2,
               head_dim=64, rms_norm_eps=1e-6, rope_theta=1e6, qkv_bias=1, tied_lm_head=0)
BF16_TOL = 2e-2


def _oracle(oracle, cfg, seed, norm_sigma, max_seq=16):
    return oracle.Engine(dict(cfg, max_seq_len=max_seq), seed=seed, sigma=0.02, norm_sigma=norm_sigma, q4_0=False,
                         kv_bf16=True, threads=8)


def _decode(eng, toks):
    out = []
    for pos, t in enumerate(toks):
        eng.forward_step(int(t), pos)
        out.append(eng.logits.copy())
    return out


@pytest.mark.parametrize("quant", [L.QUANT_F32, L.QUANT_F16, L.QUANT_G64, L.QUANT_GGML_Q4_0])
@pytest.mark.parametrize("shape", ["smollm2", "qwenish"])
def test_checkpoint_loads_like_the_synthesized_model(oracle, tmp_path, quant, shape):
    cfg = dict(SMOLLM, num_layers=2) if shape == "smollm2" else QWENISH
    if quant == L.QUANT_G64 and cfg["hidden_dim"] % 64:
        pytest.skip("group-64 needs widths divisible by 64")
    seed = 11
    ref = _oracle(oracle, cfg, seed, 0.1)
    path = str(tmp_path / "m.safetensors")
    W.write_oracle_model(path, ref, cfg, "F32")
    ref.close()
    synth = HipDecodeEngine(dict(cfg, quant_mode=quant), seed=seed, norm_sigma=0.1, max_seq_len=8)
    loaded = HipDecodeEngine(dict(cfg, quant_mode=quant), max_seq_len=8, synthesize=False)
    loaded.load_safetensors(path)
    toks = [7, 300, cfg["vocab_size"] - 1, 9]
    a, b = _decode(synth, toks), _decode(loaded, toks)
    for pos in range(len(toks)):
        assert np.array_equal(a[pos], b[pos]), (shape, quant, pos, float(np.max(np.abs(a[pos] - b[pos]))))
    synth.close()
    loaded.close()


@pytest.mark.parametrize("dtype", ["F16", "BF16"])
def test_half_precision_files_load_like_fp32_files_of_the_same_values(oracle, tmp_path, dtype):
    """Half-precision checkpoints widen exactly on the device: an F16 / BF16 file and an F32 file of
    the same (rounded) values give the same fp32-row and Q4_0 arenas."""
    cfg = dict(SMOLLM, num_layers=2)
    ref = _oracle(oracle, cfg, 5, 0.1)
    half, full = str(tmp_path / "h.safetensors"), str(tmp_path / "f.safetensors")
    t_half, t_full = [], []
    for name, kind, layer, shp in W.hf_names(cfg):
        w = ref.tensor(kind, layer).view(np.float32).reshape(shp)
        raw = W.to_dtype(w, dtype)
        t_half.append((name, dtype, shp, raw))
        r = np.frombuffer(raw, np.float16).astype(np.float32) if dtype == "F16" else W.from_bf16(raw)
        t_full.append((name, "F32", shp, r.tobytes()))
    ref.close()
    W.write(half, t_half)
    W.write(full, t_full)
    for quant in (L.QUANT_F32, L.QUANT_GGML_Q4_0):
        e1 = HipDecodeEngine(dict(cfg, quant_mode=quant), max_seq_len=8, synthesize=False)
        e2 = HipDecodeEngine(dict(cfg, quant_mode=quant), max_seq_len=8, synthesize=False)
        e1.load_safetensors(half)
        e2.load_safetensors(full)
        for x, y in zip(_decode(e1, [3, 40000, 5]), _decode(e2, [3, 40000, 5])):
            assert np.array_equal(x, y), (dtype, quant)
        e1.close()
        e2.close()


def test_golden_checkpoint_through_the_engine_and_the_runner(oracle, tmp_path):
    """The fp32 SmolLM-135M of the golden fixture (the reference's emitted C99 decode step) as a
    checkpoint: the engine's fp32-row arena loaded from it matches the fixture's argmax at every
    position and its logits to the bf16 bar (the GPU keeps K/V in bf16), and the runner, called with
    the CLI's argv (--weights FILE --tokens ... --steps N --verbose), emits the fixture's argmax after
    the last prompt position."""
    with open(os.path.join(HERE, "golden", "smollm_ref_fp32.json")) as f:
        g = json.load(f)
    ref = oracle.Engine(dict(SMOLLM, max_seq_len=64), seed=g["seed"], sigma=g["sigma"], norm_sigma=g["norm_sigma"],
                        q4_0=False, kv_bf16=True, threads=8)
    path = str(tmp_path / "smollm-135m.safetensors")
    W.write_oracle_model(path, ref, SMOLLM, "F32")
    ref.close()
    eng = HipDecodeEngine(path, max_seq_len=64)
    assert eng.cfg.quant_mode == L.QUANT_F32 and eng.cfg.num_layers == 30
    for st in g["steps"]:
        tok = eng.forward_step(st["token_in"], st["pos"])
        head = np.array(st["logits_head"], np.float32)
        d = max(float(np.max(np.abs(eng.logits[:16] - head))),
                max(abs(float(eng.logits[i]) - v) for i, v in st["top5"]))
        print(f"[safetensors golden] pos={st['pos']} token={tok} golden={st['argmax']} max-abs={d:.3e}", flush=True)
        assert tok == st["argmax"] and d < BF16_TOL
    eng.close()
    toks = [st["token_in"] for st in g["steps"]]
    r = subprocess.run([RUNNER, "--weights", path, "--tokens", ",".join(map(str, toks)), "--steps", "3", "--verbose"],
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    steps = [int(t) for _, t in re.findall(r"^\[Step (\d+)\] Token: (\d+)$", r.stdout, re.M)]
    assert len(steps) == 3 and steps[0] == g["steps"][-1]["argmax"], r.stdout
    assert "safetensors, fp32 rows" in r.stdout


@pytest.mark.parametrize("quantize,synth_args", [
    (None, ["--unquantized", "f32"]),
    ("f16", ["--unquantized", "f16"]),
    ("q4_0", ["--quantize", "q4_0"]),
    ("ggml_q4_0", []),
])
def test_runner_checkpoint_matches_the_synthetic_model(oracle, tmp_path, quantize, synth_args):
    """The runner on a 2-layer checkpoint of the seeded weights, in each --quantize mode, emits the
    tokens of the same model synthesized on the device (`--model smollm_135m --layers 2`)."""
    seed = 23
    cfg = dict(SMOLLM, num_layers=2)
    ref = _oracle(oracle, cfg, seed, 0.0)
    path = str(tmp_path / "w.safetensors")
    W.write_oracle_model(path, ref, cfg, "F32")
    ref.close()
    prompt = "5,1000,49151,77"
    q = ["--quantize", quantize] if quantize else []
    a = subprocess.run([RUNNER, "--weights", path, "--tokens", prompt, "--steps", "6", *q],
                       capture_output=True, text=True, timeout=300)
    b = subprocess.run([RUNNER, "--model", "smollm_135m", "--layers", "2", "--seed", str(seed), "--tokens", prompt,
                        "--steps", "6", *synth_args], capture_output=True, text=True, timeout=300)
    assert a.returncode == 0 and b.returncode == 0, (a.stderr, b.stderr)
    ta = re.findall(r"^\[Step \d+\] Token: (\d+)$", a.stdout, re.M)
    tb = re.findall(r"^\[Step \d+\] Token: (\d+)$", b.stdout, re.M)
    assert len(ta) == 6 and ta == tb, (quantize, ta, tb)
