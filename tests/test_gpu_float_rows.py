"""The reference's unquantized weight formats on the GPU: quant_mode 0 (fp32 rows) and 1 (fp16 rows),
run by the float-row GEMV (vx_gemv_f.hip) behind the same decode step.

Benchmark configuration 1, the fp32 SmolLM-135M, against the reference's own output: the golden
fixture holds logits of its emitted C99 decode step (tinystories_smollm.c:532) for four positions.
The GPU keeps K/V in bf16 where that module keeps fp32, so its logits are held to the bf16 bar
(2e-2) against the fixture, and to the fp32-accumulation bar (1e-3) against the oracle recomputing
each step on the GPU's own bf16 K/V rows (the two sides' bf16 roundings of a value at a rounding
boundary part otherwise, by one bf16 step)."""
import ctypes as C
import json
import os

import numpy as np
import pytest

from velox_amd import _lib as L
from velox_amd.engine import HipDecodeEngine

from test_gpu_configs import _device_kv

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
SMOLLM = dict(vocab_size=49152, hidden_dim=576, intermediate_dim=1536, num_layers=30, num_heads=9, num_kv_heads=3,
              head_dim=64, rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=1)
BF16_TOL, F32_TOL = 2e-2, 1e-3


def _golden():
    with open(os.path.join(HERE, "golden", "smollm_ref_fp32.json")) as f:
        return json.load(f)


def _shared_kv_step(ref, gpu, token, pos, max_seq):
    """The oracle's step at `pos` on the GPU's bf16 K/V rows [0, pos] of every layer."""
    hkv, d, nl = SMOLLM["num_kv_heads"], SMOLLM["head_dim"], ref.layers
    kv = [_device_kv(gpu.arena, layer, hkv, max_seq, d, pos + 1) for layer in range(nl)]
    for layer in range(nl):
        kr, vr = ref.kv_cache(layer)
        kr[:pos], vr[:pos] = kv[layer][0][:pos], kv[layer][1][:pos]
    ref.forward_forced(token, pos, np.stack([kv[layer][0][pos] for layer in range(nl)]),
                       np.stack([kv[layer][1][pos] for layer in range(nl)]))


def test_config1_smollm_fp32_matches_reference_golden(oracle):
    g = _golden()
    gpu = HipDecodeEngine(dict(SMOLLM, quant_mode=L.QUANT_F32), seed=g["seed"], sigma=g["sigma"],
                          norm_sigma=g["norm_sigma"], max_seq_len=64)
    ref = oracle.Engine(dict(SMOLLM, max_seq_len=64), seed=g["seed"], sigma=g["sigma"], norm_sigma=g["norm_sigma"],
                        q4_0=False, kv_bf16=True, threads=8)
    for st in g["steps"]:
        tok = gpu.forward_step(st["token_in"], st["pos"])
        _shared_kv_step(ref, gpu, st["token_in"], st["pos"], 64)
        head = np.array(st["logits_head"], np.float32)
        top = [(int(i), float(v)) for i, v in st["top5"]]
        d_gold = max(float(np.max(np.abs(gpu.logits[:16] - head))),
                     max(abs(float(gpu.logits[i]) - v) for i, v in top))
        d_ref = float(np.max(np.abs(gpu.logits - ref.logits)))
        print(f"[smollm fp32 rows] pos={st['pos']} token={tok} golden argmax={st['argmax']} "
              f"vs golden {d_gold:.2e}, vs the oracle on the GPU's K/V rows {d_ref:.2e}", flush=True)
        assert tok == st["argmax"] == oracle.argmax(gpu.logits)
        assert d_gold < BF16_TOL and d_ref < F32_TOL, (st["pos"], d_gold, d_ref)
    gpu.close()
    ref.close()


def test_config1_smollm_fp32_prompt_and_greedy_decode(oracle):
    """The configuration as stated: a 32-token uniform-random prompt, then 64 greedy steps. The oracle
    with the reference's fp32 K/V cache, teacher-forced with the GPU's tokens, stays within the bf16
    bar at every position; a second oracle recomputes sampled steps on the GPU's K/V rows within the
    fp32-accumulation bar."""
    seed, P, steps = 11, 32, 64
    n = P + steps
    gpu = HipDecodeEngine(dict(SMOLLM, quant_mode=L.QUANT_F32), seed=seed, norm_sigma=0.1, max_seq_len=n + 1)
    ref = oracle.Engine(dict(SMOLLM, max_seq_len=n + 1), seed=seed, sigma=0.02, norm_sigma=0.1, q4_0=False,
                        kv_bf16=False, threads=8)
    toks = [int(t) for t in oracle.prompt_tokens(seed, P, SMOLLM["vocab_size"])]
    got, worst = [], 0.0
    for pos in range(n):
        tg = gpu.forward_step(toks[pos], pos)
        assert tg == oracle.argmax(gpu.logits), pos
        got.append(gpu.logits.copy())
        t_ref = ref.forward(toks[pos], pos)
        worst = max(worst, float(np.max(np.abs(gpu.logits - ref.logits))))
        srt = np.sort(ref.logits)
        if srt[-1] - srt[-2] > 2 * BF16_TOL:
            assert tg == t_ref, pos
        if pos + 1 >= P:
            toks.append(tg)
    ref.close()
    shared = oracle.Engine(dict(SMOLLM, max_seq_len=n + 1), seed=seed, sigma=0.02, norm_sigma=0.1, q4_0=False,
                           kv_bf16=True, threads=8)
    worst_shared = 0.0
    for pos in (0, 1, 31, 32, 63, n - 1):
        _shared_kv_step(shared, gpu, toks[pos], pos, n + 1)
        worst_shared = max(worst_shared, float(np.max(np.abs(got[pos] - shared.logits))))
    print(f"[smollm fp32 rows, {n} positions] worst logits maxabs vs the oracle with the reference's fp32 K/V "
          f"{worst:.2e}; on the GPU's K/V rows {worst_shared:.2e}", flush=True)
    assert worst < BF16_TOL and worst_shared < F32_TOL
    gpu.close()
    shared.close()


def test_fp16_rows_match_the_oracle(oracle):
    """quant_mode 1: the seeded weights rounded to fp16 on both sides; 4 layers, 8 positions."""
    seed, layers, n = 5, 4, 8
    gpu = HipDecodeEngine(dict(SMOLLM, quant_mode=L.QUANT_F16), seed=seed, norm_sigma=0.1, max_seq_len=16,
                          num_layers=layers)
    ref = oracle.Engine(dict(SMOLLM, num_layers=layers, max_seq_len=16), seed=seed, sigma=0.02, norm_sigma=0.1,
                        q4_0=False, kv_bf16=True, w_f16=True, threads=8)
    for pos, tok in enumerate(oracle.prompt_tokens(seed, n, SMOLLM["vocab_size"])):
        tg = gpu.forward_step(int(tok), pos)
        _shared_kv_step(ref, gpu, int(tok), pos, 16)
        d = float(np.max(np.abs(gpu.logits - ref.logits)))
        assert tg == oracle.argmax(gpu.logits) and d < F32_TOL, (pos, d)
    gpu.close()
    ref.close()


@pytest.mark.parametrize("quant", [L.QUANT_F32, L.QUANT_F16])
def test_rows_loader_matches_synthesis(oracle, quant):
    """velox_hip_load_rows: the oracle's weights loaded row by row (the QKV parts at their row
    offsets, gate and up as the pair's halves) decode with logits bit-identical to the device-
    synthesized model; a Q4_0 upload into a row arena is refused."""
    seed, layers = 3, 2
    cfg = dict(SMOLLM, num_layers=layers, quant_mode=quant)
    a = HipDecodeEngine(cfg, seed=seed, norm_sigma=0.1, max_seq_len=8)
    b = HipDecodeEngine(cfg, max_seq_len=8, synthesize=False)
    ref = oracle.Engine(dict(SMOLLM, num_layers=layers, max_seq_len=8), seed=seed, sigma=0.02, norm_sigma=0.1,
                        q4_0=False, kv_bf16=True, w_f16=quant == L.QUANT_F16, threads=8)
    lib = b.lib

    def rows(kind, layer):
        w = ref.tensor(kind, layer).view(np.float32)
        return w.astype(np.float16) if quant == L.QUANT_F16 else w  # exact: the oracle's values are fp16's

    x = rows(oracle.T_EMBED, 0)
    L.check(lib.velox_hip_load_rows(C.byref(b.arena), L.T_EMBED, 0, x.ctypes.data, x.nbytes, None), "embed")
    for layer in range(layers):
        for kind in (oracle.T_Q, oracle.T_K, oracle.T_V, oracle.T_O, oracle.T_GATE, oracle.T_UP, oracle.T_DOWN):
            x = rows(kind, layer)
            L.check(lib.velox_hip_load_rows(C.byref(b.arena), kind, layer, x.ctypes.data, x.nbytes, None), kind)
        for kind in (oracle.T_ATTN_NORM, oracle.T_MLP_NORM):
            v = ref.tensor(kind, layer).view(np.float32)
            L.check(lib.velox_hip_load_f32(C.byref(b.arena), kind, layer, v.ctypes.data, v.size, None), kind)
    v = ref.tensor(oracle.T_FINAL_NORM, 0).view(np.float32)
    L.check(lib.velox_hip_load_f32(C.byref(b.arena), L.T_FINAL_NORM, 0, v.ctypes.data, v.size, None), "final")
    blocks = np.zeros(576 * 18, np.uint8)
    assert lib.velox_hip_load_q4_0(C.byref(b.arena), L.T_O, 0, blocks.ctypes.data, blocks.nbytes, None) == -1
    for pos, tok in enumerate((7, 300, 41000, 9)):
        a.forward_step(tok, pos)
        b.forward_step(tok, pos)
        assert np.array_equal(a.logits, b.logits), pos
    a.close()
    b.close()
    ref.close()


def test_runner_unquantized_fp32_matches_the_engine(oracle):
    """velox_hip_runner --unquantized f32 (the reference's build without --quantize) decodes the seeded
    fp32-row SmolLM: its tokens equal the engine's own decode of the same prompt, and the first of
    them the oracle's greedy token after the prompt."""
    import re
    import subprocess

    from velox_amd.engine import run

    root = os.path.dirname(HERE)
    runner = os.path.join(root, "velox_amd", "lib", "velox_hip_runner")
    prompt = [int(t) for t in oracle.prompt_tokens(17, 6, SMOLLM["vocab_size"])]
    r = subprocess.run([runner, "--model", "smollm_135m", "--unquantized", "f32", "--tokens", ",".join(map(str, prompt)),
                        "--steps", "5", "--seed", "17"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    steps = [int(t) for _, t in re.findall(r"^\[Step (\d+)\] Token: (\d+)$", r.stdout, re.M)]
    _, toks = run("smollm_135m", prompt=prompt, warmup=0, steps=4, seed=17, unquantized=1)
    assert steps == toks[len(prompt) - 1:len(prompt) - 1 + 5]
    ref = oracle.Engine(dict(SMOLLM, max_seq_len=16), seed=17, sigma=0.02, norm_sigma=0.0, q4_0=False, kv_bf16=True,
                        threads=8)
    for pos, t in enumerate(prompt):
        t_ref = ref.forward(t, pos)
    srt = np.sort(ref.logits)
    if srt[-1] - srt[-2] > 2 * BF16_TOL:
        assert steps[0] == t_ref
    ref.close()


@pytest.mark.parametrize("quant", [L.QUANT_F32, L.QUANT_F16])
@pytest.mark.parametrize("ffn", [16384, 29568])
def test_wide_rows_past_64k_of_lds(oracle, quant, ffn):
    """The float-row GEMV holds a row's fp32 activations in LDS: the down projection's 16384-wide rows
    take 65,600 bytes and Qwen2-72B's 29568-wide ones 118,336, past the 64 KiB default the launch
    raises. One layer of that width decodes within the fp32-accumulation bar of the oracle on the
    GPU's own K/V rows."""
    cfg = dict(vocab_size=512, hidden_dim=256, intermediate_dim=ffn, num_layers=1, num_heads=4, num_kv_heads=2,
               head_dim=64, rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=1)
    gpu = HipDecodeEngine(dict(cfg, quant_mode=quant), seed=9, norm_sigma=0.1, max_seq_len=8)
    ref = oracle.Engine(dict(cfg, max_seq_len=8), seed=9, sigma=0.02, norm_sigma=0.1, q4_0=False, kv_bf16=True,
                        w_f16=quant == L.QUANT_F16, threads=8)
    for pos, tok in enumerate((3, 500, 17)):
        tg = gpu.forward_step(tok, pos)
        kv = _device_kv(gpu.arena, 0, 2, 8, 64, pos + 1)
        kr, vr = ref.kv_cache(0)
        kr[:pos], vr[:pos] = kv[0][:pos], kv[1][:pos]
        ref.forward_forced(tok, pos, kv[0][pos][None], kv[1][pos][None])
        d = float(np.max(np.abs(gpu.logits - ref.logits)))
        print(f"[float rows K={ffn} quant={quant}] pos={pos} max-abs {d:.2e}", flush=True)
        assert tg == oracle.argmax(gpu.logits) and d < F32_TOL, (pos, d)
    gpu.close()
    ref.close()
