"""Batched decode of independent sequences (src/runners/velox_cuda_runner_k2.cu:553-997 batched
Q4 kernels; benchmark configuration 3): the MFMA GEMM against fp64 with exactly its fp16 activations, and
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


# ---- the batched GEMM over the MFMA-layout copy (the batched decode and prefill steps' GEMM) -------
def _tiled_dwords(blocks: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """GGML Q4_0 blocks [n][k/32][18] -> per block the tiled layout's 4 code dwords (dword w: elements
    8w..8w+7, element e at bits 8 (e % 4) + 4 (e // 4)) and the fp16 scale bits."""
    n = blocks.shape[0] if blocks.ndim == 3 else blocks.size // (k // 32 * 18)
    b = blocks.reshape(n, k // 32, 18)
    d = b[:, :, 0].astype(np.uint16) | (b[:, :, 1].astype(np.uint16) << 8)
    qs = b[:, :, 2:].astype(np.uint32)
    q = np.concatenate([qs & 15, qs >> 4], axis=2)  # element el of the block
    dw = np.zeros((n, k // 32, 4), np.uint32)
    for w in range(4):
        for e in range(8):
            dw[:, :, w] |= q[:, :, 8 * w + e] << (8 * (e % 4) + 4 * (e // 4))
    return dw, d


def _m_order(dw: np.ndarray) -> np.ndarray:
    """Tiled dword nibble order (element e at bit 8 (e % 4) + 4 (e // 4)) -> the M-layout's (bit
    16 (e % 2) + 4 (e // 2))."""
    out = np.zeros_like(dw)
    for e in range(8):
        out |= ((dw >> (8 * (e % 4) + 4 * (e // 4))) & 15) << (16 * (e % 2) + 4 * (e // 2))
    return out


def mlayout_reference(blocks, n, k, up_blocks=None):
    """The M-layout restated: codes [tiles][groups][64][4] uint32, scales [tiles][groups][16][4] uint16."""
    parts = [blocks] if up_blocks is None else [blocks, up_blocks]
    nb = k // 32
    ng = (nb + 3) // 4
    t16 = (n + 15) // 16
    tiles = t16 * len(parts)
    codes = np.zeros((tiles, ng, 64, 4), np.uint32)
    scales = np.zeros((tiles, ng, 16, 4), np.uint16)
    for pi, blk in enumerate(parts):
        dw, d = _tiled_dwords(blk, k)
        dw = _m_order(dw)
        for t in range(t16):
            T = t * len(parts) + pi
            for rho in range(16):
                r = 16 * t + rho
                if r >= n:
                    continue
                for j in range(ng):
                    for bb in range(4):
                        blkid = 4 * j + bb
                        if blkid >= nb:
                            continue
                        scales[T, j, rho, bb] = d[r, blkid]
                        for g in range(4):
                            codes[T, j, rho + 16 * g, bb] = dw[r, blkid, g]
    return codes, scales


class MQ4:
    """The M-layout copy of a TiledQ4 matrix."""

    def __init__(self, hiplib, dev, t: TiledQ4):
        cb, sb = C.c_uint64(), C.c_uint64()
        L.check(hiplib.velox_hip_q4_mlayout_bytes(C.byref(t.m), C.byref(cb), C.byref(sb)))
        self.codes = dev.empty(cb.value, np.uint8)
        self.scales = dev.empty(sb.value, np.uint8)
        L.check(hiplib.velox_hip_q4_mlayout(C.byref(t.m), self.codes.data_ptr(), self.scales.data_ptr(), None))


@pytest.mark.parametrize("n,k,paired", [(100, 576, False), (40, 576, True), (33, 4096, False), (24, 3584, True)])
def test_mlayout_matches_restatement(hiplib, oracle, dev, n, k, paired):
    g = _weights(oracle, n, k, 31)
    u = _weights(oracle, n, k, 32) if paired else None
    t = TiledQ4(hiplib, dev, g, n, k, up_blocks=u)
    mq = MQ4(hiplib, dev, t)
    codes, scales = mlayout_reference(g, n, k, u)
    assert np.array_equal(dev.get(mq.codes).view(np.uint32), codes.ravel())
    assert np.array_equal(dev.get(mq.scales).view(np.uint16), scales.ravel())


def _block_major(x: np.ndarray, k: int) -> np.ndarray:
    """[rows][>= k] fp16 -> [k / 32][rows][32] (ldx 32, xbs 32 * rows)."""
    rows = x.shape[0]
    return np.ascontiguousarray(x[:, :k].reshape(rows, k // 32, 32).transpose(1, 0, 2))


@pytest.mark.parametrize("n,k,batch,ks,bm", [(4608, 3584, 8, 1, 1), (4608, 3584, 32, 4, 1), (960, 576, 5, 1, 0),
                                             (123, 4096, 17, 3, 1), (4096, 14336, 32, 8, 0), (64, 4096, 1, 2, 1),
                                             (200, 1536, 16, 1, 0), (1000, 4096, 40, 2, 1), (6144, 4096, 64, 1, 1),
                                             (96, 576, 64, 5, 0), (6144, 4096, 128, 6, 1), (1000, 4096, 100, 2, 0),
                                             (4096, 14336, 128, 8, 1)])
def test_gemm_m_store_and_residual(hiplib, oracle, dev, n, k, batch, ks, bm):
    """Row-major (bm 0) and block-major (bm 1) activations; 1..8 K splits."""
    rng = np.random.default_rng(n + k + batch + ks)
    blocks = _weights(oracle, n, k, 600 + batch)
    t = TiledQ4(hiplib, dev, blocks, n, k)
    mq = MQ4(hiplib, dev, t)
    deq = oracle.q4_0_dequant(blocks, k).astype(np.float64)
    ldx, ldy = k + 8, n + 3
    x = _x16(rng, batch, k, ldx)
    bias = (0.1 * rng.standard_normal(n)).astype(np.float32)
    if bm:
        dx, ldx, xbs = dev.put(_block_major(x, k).view(np.int16)), 32, 32 * batch
    else:
        dx, xbs = dev.put(x.view(np.int16)), 32
    db = dev.put(bias)
    part = dev.empty(ks * batch * ldy)
    scale = max(1.0, np.sqrt(k / 4096))
    dy = dev.put(np.full((batch, ldy), 7.0, np.float32))
    L.check(hiplib.velox_hip_gemm_q4_0_batch_m(C.byref(t.m), mq.codes.data_ptr(), mq.scales.data_ptr(), dx.data_ptr(),
                                               batch, ldx, xbs, db.data_ptr(), dy.data_ptr(), ldy, None, 0, 0,
                                               L.GEMV_STORE, ks, part.data_ptr(), None))
    got = dev.get(dy).reshape(batch, ldy)
    want = x[:, :k].astype(np.float64) @ deq.T + bias
    assert rms(got[:, :n] - want) < 1e-5 * rms(want) * scale
    assert np.all(got[:, n:] == 7.0)
    y0 = rng.standard_normal((batch, ldy)).astype(np.float32)
    dy = dev.put(y0)
    L.check(hiplib.velox_hip_gemm_q4_0_batch_m(C.byref(t.m), mq.codes.data_ptr(), mq.scales.data_ptr(), dx.data_ptr(),
                                               batch, ldx, xbs, None, dy.data_ptr(), ldy, None, 0, 0, L.GEMV_RESIDUAL,
                                               ks, part.data_ptr(), None))
    got = dev.get(dy).reshape(batch, ldy)
    want = y0[:, :n].astype(np.float64) + x[:, :k].astype(np.float64) @ deq.T
    assert rms(got[:, :n] - want) < 1e-5 * rms(want - y0[:, :n]) * scale
    assert np.array_equal(got[:, n:], y0[:, n:])


@pytest.mark.parametrize("F,H,batch,bm", [(1536, 576, 3, 0), (2048, 3584, 32, 1), (100, 576, 9, 0), (18944, 3584, 20, 1),
                                          (96, 576, 16, 1), (14336, 4096, 64, 1), (160, 576, 47, 0),
                                          (14336, 4096, 128, 1), (160, 576, 77, 0), (18944, 3584, 100, 1)])
def test_gemm_m_swiglu(hiplib, oracle, dev, F, H, batch, bm):
    rng = np.random.default_rng(F + batch + 1)
    g = _weights(oracle, F, H, 41)
    u = _weights(oracle, F, H, 42)
    t = TiledQ4(hiplib, dev, g, F, H, up_blocks=u)
    mq = MQ4(hiplib, dev, t)
    x = _x16(rng, batch, H, H)
    Fp = (F + 31) // 32 * 32  # block-major output rows cover whole blocks
    if bm:
        dx, ldx, xbs = dev.put(_block_major(x, H).view(np.int16)), 32, 32 * batch
        dout, ldo, obs = dev.empty(batch * Fp, np.uint16), 32, 32 * batch
    else:
        dx, ldx, xbs = dev.put(x.view(np.int16)), H, 32
        dout, ldo, obs = dev.empty(batch * F, np.uint16), F, 32
    L.check(hiplib.velox_hip_gemm_q4_0_batch_m(C.byref(t.m), mq.codes.data_ptr(), mq.scales.data_ptr(), dx.data_ptr(),
                                               batch, ldx, xbs, None, None, 0, dout.data_ptr(), ldo, obs,
                                               L.GEMV_SWIGLU, 1, None, None))
    raw = dev.get(dout).view(np.float16)
    if bm:
        raw = raw.reshape(Fp // 32, batch, 32).transpose(1, 0, 2).reshape(batch, Fp)[:, :F]
    got = raw.reshape(batch, F).astype(np.float64)
    xx = x.astype(np.float64)
    gg = xx @ oracle.q4_0_dequant(g, H).astype(np.float64).T
    uu = xx @ oracle.q4_0_dequant(u, H).astype(np.float64).T
    want = gg / (1.0 + np.exp(-gg)) * uu
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 1e-3)) < 2e-3
    assert rms(got - want) < 5e-4 * rms(want)


def test_gemm_m_rejects_bad_arguments(hiplib, oracle, dev):
    blocks = _weights(oracle, 64, 576, 9)
    t = TiledQ4(hiplib, dev, blocks, 64, 576)
    mq = MQ4(hiplib, dev, t)
    dx, dy, part = dev.empty(129 * 576, np.uint16), dev.empty(129 * 64), dev.empty(9 * 129 * 64)
    cases = [(0, 576, 1, part), (129, 576, 1, part), (4, 500, 1, part), (4, 576, 9, part), (4, 576, 2, None),
             (4, 576, 6, part)]  # 576 = 18 blocks = 5 groups: at most 5 splits
    for batch, ldx, ks, p in cases:
        assert hiplib.velox_hip_gemm_q4_0_batch_m(C.byref(t.m), mq.codes.data_ptr(), mq.scales.data_ptr(),
                                                  dx.data_ptr(), batch, ldx, 32, None, dy.data_ptr(), 64, None, 0, 0,
                                                  L.GEMV_STORE, ks, p.data_ptr() if p is not None else None,
                                                  None) == L.EINVAL, (batch, ldx, ks)
    # block-major rows must fit inside a block: xbs >= batch * ldx
    assert hiplib.velox_hip_gemm_q4_0_batch_m(C.byref(t.m), mq.codes.data_ptr(), mq.scales.data_ptr(), dx.data_ptr(),
                                              8, 32, 32 * 7, None, dy.data_ptr(), 64, None, 0, 0, L.GEMV_STORE, 1,
                                              None, None) == L.EINVAL


@pytest.mark.parametrize("n,k,s,batch", [(96, 576, 4, 16), (100, 4096, 8, 16), (64, 4096, 16, 64), (70, 4096, 32, 128),
                                         (40, 4096, 64, 3), (33, 29568, 0, 40)])
def test_gemm_m_weights_enter_exactly(hiplib, oracle, dev, n, k, s, batch):
    """One-hot activation rows: row m selects column k_m, so y[m][n] = d (q - 8) of the weight the
    GEMM applied -- bit for bit the oracle's dequantized value (the block product is exact and the
    scale is applied once in fp32). Pins the M-layout copy and the K order of both GEMM kernels
    (1-16 rows, 17-128 rows) for every lanes-per-row layout of the source matrix."""
    rng = np.random.default_rng(n + k + s)
    blocks = _weights(oracle, n, k, 700 + s)
    t = TiledQ4(hiplib, dev, blocks, n, k, s)
    mq = MQ4(hiplib, dev, t)
    deq = oracle.q4_0_dequant(blocks, k)
    cols = rng.choice(k, size=batch, replace=batch > k)
    edge = [0, 7, 8 * 5 + 3, k - 1]
    cols[:min(4, batch)] = edge[:min(4, batch)]
    x = np.zeros((batch, k), np.float16)
    x[np.arange(batch), cols] = 1.0
    dx = dev.put(x.view(np.int16))
    dy = dev.put(np.zeros((batch, n), np.float32))
    L.check(hiplib.velox_hip_gemm_q4_0_batch_m(C.byref(t.m), mq.codes.data_ptr(), mq.scales.data_ptr(), dx.data_ptr(),
                                               batch, k, 32, None, dy.data_ptr(), n, None, 0, 0, L.GEMV_STORE, 1, None,
                                               None))
    got = dev.get(dy).reshape(batch, n)
    assert np.array_equal(got, deq[:, cols].T)  # (a zero weight of a negative scale: -0 in the oracle)
