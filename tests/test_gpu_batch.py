"""Batched decode of independent sequences (src/runners/velox_cuda_runner_k2.cu:553-997 batched
Q4 kernels): the MFMA GEMM against fp64 with exactly its fp16 activations, and
the batched decode step against one oracle engine per sequence."""
import ctypes as C

import numpy as np
import pytest

from velox_amd import _lib as L

from test_gpu_kernels import TiledQ4, _weights

pytestmark = pytest.mark.gpu

rms = lambda a: float(np.sqrt(np.mean(np.square(a, dtype=np.float64))))


def _x16(rng, batch, k, ldx):
    x = np.zeros((batch, ldx), np.float16)
    x[:, :k] = rng.standard_normal((batch, k)).astype(np.float16)
    return x


@pytest.mark.parametrize("n,k,batch,s", [(4608, 3584, 8, 0), (3584, 18944, 32, 0), (960, 576, 5, 0),
                                         (4096, 4096, 16, 0), (123, 4096, 17, 0), (200, 1536, 1, 8),
                                         (64, 4096, 32, 4)])
def test_gemm_batch_store_and_residual(hiplib, oracle, dev, n, k, batch, s):
    rng = np.random.default_rng(n + k + batch)
    blocks = _weights(oracle, n, k, 500 + batch)
    t = TiledQ4(hiplib, dev, blocks, n, k, s)
    deq = oracle.q4_0_dequant(blocks, k).astype(np.float64)
    ldx, ldy = k + 8, n + 3
    x = _x16(rng, batch, k, ldx)
    bias = (0.1 * rng.standard_normal(n)).astype(np.float32)
    dx, db = dev.put(x.view(np.int16)), dev.put(bias)
    dy = dev.put(np.full((batch, ldy), 7.0, np.float32))
    L.check(hiplib.velox_hip_gemm_q4_0_batch(C.byref(t.m), dx.data_ptr(), batch, ldx, db.data_ptr(), dy.data_ptr(),
                                             ldy, None, 0, L.GEMV_STORE, None))
    got = dev.get(dy).reshape(batch, ldy)
    want = x[:, :k].astype(np.float64) @ deq.T + bias
    # exact products (fp16 x, integer codes), fp32 sums and fp32 block scales: only accumulation
    # rounding remains, as in the single-sequence GEMV
    assert rms(got[:, :n] - want) < 1e-5 * rms(want) * max(1.0, np.sqrt(k / 4096))
    assert np.all(got[:, n:] == 7.0)  # padding columns untouched
    # residual: y += W x
    y0 = rng.standard_normal((batch, ldy)).astype(np.float32)
    dy = dev.put(y0)
    L.check(hiplib.velox_hip_gemm_q4_0_batch(C.byref(t.m), dx.data_ptr(), batch, ldx, None, dy.data_ptr(), ldy, None,
                                             0, L.GEMV_RESIDUAL, None))
    got = dev.get(dy).reshape(batch, ldy)
    want = y0[:, :n].astype(np.float64) + x[:, :k].astype(np.float64) @ deq.T
    assert rms(got[:, :n] - want) < 1e-5 * rms(want - y0[:, :n]) * max(1.0, np.sqrt(k / 4096))


@pytest.mark.parametrize("F,H,batch", [(1536, 576, 3), (2048, 3584, 32), (100, 576, 9)])
def test_gemm_batch_swiglu(hiplib, oracle, dev, F, H, batch):
    rng = np.random.default_rng(F + batch)
    g = _weights(oracle, F, H, 21)
    u = _weights(oracle, F, H, 22)
    t = TiledQ4(hiplib, dev, g, F, H, up_blocks=u)
    x = _x16(rng, batch, H, H)
    dx, dout = dev.put(x.view(np.int16)), dev.empty(batch * F, np.uint16)
    L.check(hiplib.velox_hip_gemm_q4_0_batch(C.byref(t.m), dx.data_ptr(), batch, H, None, None, 0, dout.data_ptr(), F,
                                             L.GEMV_SWIGLU, None))
    got = dev.get(dout).view(np.float16).reshape(batch, F).astype(np.float64)
    xx = x.astype(np.float64)
    gg = xx @ oracle.q4_0_dequant(g, H).astype(np.float64).T
    uu = xx @ oracle.q4_0_dequant(u, H).astype(np.float64).T
    want = gg / (1.0 + np.exp(-gg)) * uu
    # the output is stored as fp16: half an ulp plus accumulation rounding
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-3)) < 2e-3
    assert rms(got - want) < 5e-4 * rms(want)


def test_gemm_batch_rejects_bad_arguments(hiplib, oracle, dev):
    blocks = _weights(oracle, 64, 576, 9)
    t = TiledQ4(hiplib, dev, blocks, 64, 576)
    dx, dy = dev.empty(33 * 576, np.uint16), dev.empty(33 * 64)
    for batch, ldx in ((0, 576), (33, 576), (4, 500)):
        assert hiplib.velox_hip_gemm_q4_0_batch(C.byref(t.m), dx.data_ptr(), batch, ldx, None, dy.data_ptr(), 64,
                                                None, 0, L.GEMV_STORE, None) == L.EINVAL


# ---- the batched decode step against one oracle replay per sequence -------------------------
from velox_amd.engine import HipBatchEngine, run  # noqa: E402

LOGIT_TOL = 2e-2
SMOLLM = dict(vocab_size=49152, hidden_dim=576, intermediate_dim=1536, num_heads=9, num_kv_heads=3, head_dim=64,
              rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=1)
QWEN_SMALL_VOCAB = dict(vocab_size=4096, hidden_dim=3584, intermediate_dim=18944, num_heads=28, num_kv_heads=4,
                        head_dim=128, rms_norm_eps=1e-6, rope_theta=1000000.0, qkv_bias=1, tied_lm_head=1)
GOLDEN = 0x9E3779B97F4A7C15


def _batch_vs_oracle(oracle, model, cfg, layers, batch, n_steps, max_seq, seed, starts):
    gpu = HipBatchEngine(model, max_batch=batch, seed=seed, norm_sigma=0.1, max_seq_len=max_seq, num_layers=layers)
    V = cfg["vocab_size"]
    prompts = [[int(t) for t in oracle.prompt_tokens(seed + 100 + b, max_seq, V)] for b in range(batch)]
    for b in range(batch):
        gpu.set_prompt_seq(b, prompts[b])
        gpu.set_state_seq(b, starts[b], prompts[b][starts[b]])
    got = [[] for _ in range(batch)]
    for _ in range(n_steps):
        gpu.batch_step(batch)
        gpu.sync()
        for b in range(batch):
            got[b].append(gpu.logits_seq(b))
    ref = oracle.Engine(dict(cfg, num_layers=layers, max_seq_len=max_seq), seed=seed, sigma=0.02, norm_sigma=0.1,
                        q4_0=True, kv_bf16=True, threads=16)
    worst = 0.0
    for b in range(batch):
        ref.reset()  # positions before starts[b] hold zero K/V in both caches
        for t in range(n_steps):
            pos = starts[b] + t
            ref.forward(prompts[b][pos], pos)
            d = float(np.max(np.abs(got[b][t] - ref.logits)))
            worst = max(worst, d)
            assert gpu.ring_seq(b, pos) == oracle.argmax(got[b][t]), (b, pos)
            assert d < LOGIT_TOL, (b, pos, d)
        assert gpu.state_seq(b) == (starts[b] + n_steps, prompts[b][starts[b] + n_steps])
    print(f"[{model} batch {batch}] worst logits maxabs {worst:.3e}", flush=True)
    gpu.close()
    ref.close()


@pytest.mark.parametrize("batch", [3, 17])
def test_batch_decode_smollm_vs_oracle(oracle, batch):
    _batch_vs_oracle(oracle, "smollm_135m", SMOLLM, 4, batch, 5, 16, seed=51, starts=[b % 3 for b in range(batch)])


def test_batch_decode_qwen_bias_32_vs_oracle(oracle):
    _batch_vs_oracle(oracle, QWEN_SMALL_VOCAB, QWEN_SMALL_VOCAB, 1, 32, 2, 8, seed=52, starts=[0] * 32)


def test_batch_run_graph_matches_eager(oracle):
    """velox_hip_run with batch > 1 (hipGraph of the batched step) produces sequence 0's tokens of an
    eager batched decode of the same seeded prompts."""
    seed, B, P, n = 61, 4, 5, 4
    rep, toks = run("smollm_135m", prompt_len=P, warmup=0, steps=n - 1, seed=seed, num_layers=3, batch=B,
                    max_seq_len=16)
    assert rep["status"] == 0 and rep["tok_per_s"] > 0
    gpu = HipBatchEngine("smollm_135m", max_batch=B, seed=seed, max_seq_len=16, num_layers=3)
    for b in range(B):
        pr = [int(t) for t in oracle.prompt_tokens((seed + b * GOLDEN) % (1 << 64), P, 49152)]
        gpu.set_prompt_seq(b, pr)
        gpu.set_state_seq(b, 0, pr[0])
    for _ in range(P + n - 1):
        gpu.batch_step(B)
    gpu.sync()
    assert [gpu.ring_seq(0, p) for p in range(P + n - 1)] == toks[:P + n - 1]
    gpu.close()
