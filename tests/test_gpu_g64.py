"""The reference's group-64 weight format (quant_mode 2, its `--quantize q4_0` build) on the GPU.

The reference quantizes fp32 weights at load with velox_cuda_quantize_q4_group64_kernel
(src/codegen.rs:2337-2370) and dequantizes w = fmaf(q, s, m) in its GEMV and embedding
(:2248-2265, :2381-2410). Bars: the device quantizer bit-exact against the oracle's restatement
(packed words and fp16 scale pairs), dequantized tiled weights bit-exact, the GEMV within the
fp32-class bars of the Q4_0 GEMV (and bit for bit where its integer arithmetic is exact), and the
SmolLM-135M decode step within the fp32-accumulation bar (1e-3) against the oracle with the same
dequantized weights on the GPU's bf16 K/V rows.
"""
import ctypes as C
import os
import re
import subprocess

import numpy as np
import pytest

from velox_amd import _lib as L
from velox_amd.engine import HipDecodeEngine, run

from test_gpu_float_rows import SMOLLM, F32_TOL, _shared_kv_step

pytestmark = pytest.mark.gpu

GEMV_RMS, GEMV_MAX = 5e-6, 3e-5  # the Q4_0 GEMV's bars (test_gpu_kernels.py)
HERE = os.path.dirname(os.path.abspath(__file__))


def _edge_groups(rng) -> np.ndarray:
    g = [np.zeros(64), np.full(64, 0.3), np.linspace(-1.0, 1.0, 64), 1.0 + 1e-9 * np.arange(64),
         rng.standard_normal(64) * 1e-6,                  # fp16-subnormal scale
         np.r_[np.full(63, -2.0), 13.0],                  # one value far from the rest
         -3.0 + (np.arange(64) % 16) + 0.5,               # every value on a rounding tie
         rng.standard_normal(64) * 1e3]
    return np.concatenate(g).astype(np.float32)


def test_quantizer_matches_the_reference_codec(hiplib, oracle, dev):
    rng = np.random.default_rng(2337)
    x = np.concatenate([_edge_groups(rng), (rng.standard_normal(64 * 4000) * 0.02).astype(np.float32)])
    ng = x.size // 64
    dx, dp, ds = dev.put(x), dev.empty(ng * 8, np.uint32), dev.empty(ng * 2, np.uint16)
    L.check(hiplib.velox_hip_g64_quantize(dx.data_ptr(), ng, dp.data_ptr(), ds.data_ptr(), None), "g64_quantize")
    packed, sm = oracle.g64_quantize(x)
    assert np.array_equal(dev.get(dp).view(np.uint32).reshape(ng, 8), packed)
    assert np.array_equal(dev.get(ds).view(np.uint16).reshape(ng, 2), sm)


class TiledG64:
    """fp32 rows quantized on the device into a tiled group-64 matrix (velox_hip_g64_pack)."""

    def __init__(self, hiplib, dev, rows, n, k, s=0, up_rows=None):
        paired = up_rows is not None
        self.m = L.Q4Matrix()
        cb, sb = C.c_uint64(), C.c_uint64()
        L.check(hiplib.velox_hip_q4_layout(n, k, s, int(paired), C.byref(self.m), C.byref(cb), C.byref(sb)), "layout")
        self.m.format = L.QUANT_G64
        self.codes = dev.empty(cb.value, np.uint8)  # zeroed: padded slots stay zero
        self.scales = dev.empty(sb.value, np.uint8)
        self.m.codes = self.codes.data_ptr()
        self.m.scales = self.scales.data_ptr()
        self._src = []
        for part, r in enumerate([rows] if not paired else [rows, up_rows]):
            src = dev.put(np.ascontiguousarray(r, np.float32).ravel())
            self._src.append(src)
            L.check(hiplib.velox_hip_g64_pack(src.data_ptr(), n, 0, part, C.byref(self.m), None), "g64_pack")


def _rows(oracle, n, k, tag, sigma=0.02):
    return oracle.fill_normal(n * k, 7, tag, sigma).reshape(n, k)


def _deq(oracle, w):
    return oracle.g64_dequant(*oracle.g64_quantize(w)).reshape(w.shape)


@pytest.mark.parametrize("n,k,s", [(96, 576, 0), (64, 576, 8), (130, 4096, 0), (48, 14336, 0), (64, 1536, 16),
                                   (40, 4096, 4), (24, 4096, 64), (32, 18944, 0)])
def test_pack_dequant_bitexact(hiplib, oracle, dev, n, k, s):
    w = _rows(oracle, n, k, n + k)
    t = TiledG64(hiplib, dev, w, n, k, s)
    out = dev.empty(n * k)
    L.check(hiplib.velox_hip_q4_0_dequant(C.byref(t.m), out.data_ptr(), None))
    assert np.array_equal(dev.get(out).reshape(n, k).view(np.uint32), _deq(oracle, w).view(np.uint32))


def test_paired_pack_dequant_bitexact(hiplib, oracle, dev):
    F, H = 100, 576
    g, u = _rows(oracle, F, H, 1), _rows(oracle, F, H, 2)
    t = TiledG64(hiplib, dev, g, F, H, up_rows=u)
    out = dev.empty(2 * F * H)
    L.check(hiplib.velox_hip_q4_0_dequant(C.byref(t.m), out.data_ptr(), None))
    got = dev.get(out).reshape(2 * F, H)
    assert np.array_equal(got[:F], _deq(oracle, g)) and np.array_equal(got[F:], _deq(oracle, u))


def _gemv(hiplib, dev, t, x, n, mode, gain=None, bias=None, res=None):
    dx, dy = dev.put(x), dev.empty(n)
    dg = dev.put(gain) if gain is not None else None
    db = dev.put(bias) if bias is not None else None
    dr = dev.put(res) if res is not None else None
    ptr = lambda t_: t_.data_ptr() if t_ is not None else None  # noqa: E731
    L.check(hiplib.velox_hip_gemv_q4_0(C.byref(t.m), dx.data_ptr(), ptr(dg), 1e-5, ptr(db), ptr(dr), dy.data_ptr(),
                                       mode, None), "gemv")
    return dev.get(dy)


def _rms(a) -> float:
    return float(np.sqrt(np.mean(np.square(a, dtype=np.float64))))


@pytest.mark.parametrize("n,k,s", [(960, 576, 0), (576, 1536, 0), (1536, 576, 8), (4096, 4096, 0), (123, 4096, 16),
                                   (64, 4096, 4), (64, 4096, 64), (256, 18944, 0)])
def test_gemv_store(hiplib, oracle, dev, n, k, s):
    rng = np.random.default_rng(n + k + s)
    w = _rows(oracle, n, k, 300 + n)
    t = TiledG64(hiplib, dev, w, n, k, s)
    x = rng.standard_normal(k).astype(np.float32)
    got = _gemv(hiplib, dev, t, x, n, L.GEMV_STORE)
    tight = _deq(oracle, w).astype(np.float64) @ x.astype(np.float64)
    assert _rms(got - tight) < GEMV_RMS * _rms(tight)
    assert np.max(np.abs(got - tight)) < GEMV_MAX * np.max(np.abs(tight))


def test_gemv_norm_bias_residual_swiglu(hiplib, oracle, dev):
    rng = np.random.default_rng(11)
    H, F = 576, 1536
    x = rng.standard_normal(H).astype(np.float32)
    gain = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    xn = oracle.rmsnorm(x, gain, 1e-5).astype(np.float64)
    # QKV-shaped store with RMSNorm and bias
    w = _rows(oracle, 960, H, 21)
    b = (rng.standard_normal(960) * 0.1).astype(np.float32)
    got = _gemv(hiplib, dev, TiledG64(hiplib, dev, w, 960, H), x, 960, L.GEMV_STORE, gain=gain, bias=b)
    tight = _deq(oracle, w).astype(np.float64) @ xn + b
    assert np.max(np.abs(got - tight)) < GEMV_MAX * np.max(np.abs(tight))
    # down-shaped residual
    w = _rows(oracle, H, F, 22)
    xf = rng.standard_normal(F).astype(np.float32)
    res = rng.standard_normal(H).astype(np.float32)
    got = _gemv(hiplib, dev, TiledG64(hiplib, dev, w, H, F), xf, H, L.GEMV_RESIDUAL, res=res)
    tight = res + _deq(oracle, w).astype(np.float64) @ xf.astype(np.float64)
    assert np.max(np.abs(got - tight)) < GEMV_MAX * np.max(np.abs(tight))
    # paired gate/up with SwiGLU
    g, u = _rows(oracle, F, H, 23), _rows(oracle, F, H, 24)
    got = _gemv(hiplib, dev, TiledG64(hiplib, dev, g, F, H, up_rows=u), x, F, L.GEMV_SWIGLU, gain=gain)
    g64, u64 = _deq(oracle, g).astype(np.float64) @ xn, _deq(oracle, u).astype(np.float64) @ xn
    tight = g64 / (1.0 + np.exp(-g64)) * u64
    assert np.max(np.abs(got - tight)) < GEMV_MAX * max(1.0, float(np.max(np.abs(tight))))


@pytest.mark.parametrize("n,k,s", [(96, 576, 0), (64, 4096, 0), (40, 1536, 8)])
def test_gemv_integer_weights_bit_exact(hiplib, oracle, dev, n, k, s):
    """Groups holding q - 3 for random q (each with a 0 and a 15, so s = 1 and m = -3 exactly, and
    the (8 s + m) T term is live) against inputs the integer blocks represent exactly: every block
    term, the per-block sums T and the fp32 row sum are exact, so the result must equal the fp64
    product bit for bit. A wrong slot pairing, sign or T term breaks it."""
    rng = np.random.default_rng(k + s)
    q = rng.integers(0, 16, size=(n, k // 64, 64))
    q[:, :, 0], q[:, :, 1] = 0, 15
    w = (q - 3).reshape(n, k).astype(np.float32)
    packed, sm = oracle.g64_quantize(w)
    assert np.all(sm[:, 0].view(np.float16) == 1.0) and np.all(sm[:, 1].view(np.float16) == -3.0)
    t = TiledG64(hiplib, dev, w, n, k, s)
    for p in (-30, 0, 4, 40):
        x = rng.integers(-16, 16, size=k).astype(np.float64) / 8.0
        x[:64] = 0.0
        x[70] = 1.875
        x = (x * 2.0 ** p).astype(np.float32)
        got = _gemv(hiplib, dev, t, x, n, L.GEMV_STORE).astype(np.float64)
        want = w.astype(np.float64) @ x.astype(np.float64)
        assert np.array_equal(got, want), (p, np.max(np.abs(got - want)))


def test_lm_head_argmax(hiplib, oracle, dev):
    """SmolLM's tied head: 49152 x 576 group-64 rows, logits and the greedy token."""
    V, H = 49152, 576
    rng = np.random.default_rng(V)
    w = _rows(oracle, V, H, 13)
    t = TiledG64(hiplib, dev, w, V, H)
    x = rng.standard_normal(H).astype(np.float32)
    gain = np.ones(H, np.float32)
    dx, dg, dl, dt = dev.put(x), dev.put(gain), dev.empty(V), dev.empty(1, np.uint32)
    L.check(hiplib.velox_hip_lm_head_argmax(C.byref(t.m), dx.data_ptr(), dg.data_ptr(), 1e-5, dl.data_ptr(),
                                            dt.data_ptr(), None))
    logits = dev.get(dl)
    assert int(dev.get(dt).view(np.uint32)[0]) == oracle.argmax(logits)
    tight = _deq(oracle, w).astype(np.float64) @ oracle.rmsnorm(x, gain, 1e-5).astype(np.float64)
    assert np.max(np.abs(logits - tight)) < GEMV_MAX * np.max(np.abs(tight))


def test_smollm_group64_matches_the_oracle(oracle):
    """The whole SmolLM-135M step in quant_mode 2 (30 layers, 8 prompt positions): logits within the
    fp32-accumulation bar of the oracle over the same dequantized weights, on the GPU's K/V rows."""
    seed, n = 5, 8
    gpu = HipDecodeEngine(dict(SMOLLM, quant_mode=L.QUANT_G64), seed=seed, norm_sigma=0.1, max_seq_len=16)
    ref = oracle.Engine(dict(SMOLLM, max_seq_len=16), seed=seed, sigma=0.02, norm_sigma=0.1, q4_0=False,
                        kv_bf16=True, w_g64=True, threads=8)
    worst = 0.0
    for pos, tok in enumerate(oracle.prompt_tokens(seed, n, SMOLLM["vocab_size"])):
        tg = gpu.forward_step(int(tok), pos)
        _shared_kv_step(ref, gpu, int(tok), pos, 16)
        d = float(np.max(np.abs(gpu.logits - ref.logits)))
        worst = max(worst, d)
        assert tg == oracle.argmax(gpu.logits) and d < F32_TOL, (pos, d)
    print(f"[smollm group-64] worst logits maxabs vs the oracle on the GPU's K/V rows {worst:.2e}", flush=True)
    gpu.close()
    ref.close()


def test_rows_loader_quantizes_like_synthesis(oracle):
    """velox_hip_load_rows into a group-64 arena: the oracle's fp32 weights, converted on the device,
    decode with logits bit-identical to the device-synthesized group-64 model."""
    seed, layers = 3, 2
    cfg = dict(SMOLLM, num_layers=layers, quant_mode=L.QUANT_G64)
    a = HipDecodeEngine(cfg, seed=seed, norm_sigma=0.1, max_seq_len=8)
    b = HipDecodeEngine(cfg, max_seq_len=8, synthesize=False)
    ref = oracle.Engine(dict(SMOLLM, num_layers=layers, max_seq_len=8), seed=seed, sigma=0.02, norm_sigma=0.1,
                        q4_0=False, kv_bf16=True, threads=8)
    lib = b.lib
    x = ref.tensor(oracle.T_EMBED, 0).view(np.float32)
    L.check(lib.velox_hip_load_rows(C.byref(b.arena), L.T_EMBED, 0, x.ctypes.data, x.nbytes, None), "embed")
    for layer in range(layers):
        for kind in (oracle.T_Q, oracle.T_K, oracle.T_V, oracle.T_O, oracle.T_GATE, oracle.T_UP, oracle.T_DOWN):
            x = ref.tensor(kind, layer).view(np.float32)
            L.check(lib.velox_hip_load_rows(C.byref(b.arena), kind, layer, x.ctypes.data, x.nbytes, None), kind)
        for kind in (oracle.T_ATTN_NORM, oracle.T_MLP_NORM):
            v = ref.tensor(kind, layer).view(np.float32)
            L.check(lib.velox_hip_load_f32(C.byref(b.arena), kind, layer, v.ctypes.data, v.size, None), kind)
    v = ref.tensor(oracle.T_FINAL_NORM, 0).view(np.float32)
    L.check(lib.velox_hip_load_f32(C.byref(b.arena), L.T_FINAL_NORM, 0, v.ctypes.data, v.size, None), "final")
    for pos, tok in enumerate((7, 300, 41000, 9)):
        a.forward_step(tok, pos)
        b.forward_step(tok, pos)
        assert np.array_equal(a.logits, b.logits), pos
    a.close()
    b.close()
    ref.close()


def test_runner_quantize_q4_0_matches_the_engine(oracle):
    """velox_hip_runner --quantize q4_0 (the reference runner's group-64 conversion of its fp32
    model): its tokens equal the engine's own group-64 decode of the same prompt."""
    runner = os.path.join(os.path.dirname(HERE), "velox_amd", "lib", "velox_hip_runner")
    prompt = [int(t) for t in oracle.prompt_tokens(17, 6, SMOLLM["vocab_size"])]
    r = subprocess.run([runner, "--model", "smollm_135m", "--quantize", "q4_0", "--tokens", ",".join(map(str, prompt)),
                        "--steps", "5", "--seed", "17"], capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, r.stderr
    steps = [int(t) for _, t in re.findall(r"^\[Step (\d+)\] Token: (\d+)$", r.stdout, re.M)]
    _, toks = run("smollm_135m", prompt=prompt, warmup=0, steps=4, seed=17, unquantized=3)
    assert len(steps) == 5 and steps == toks[len(prompt) - 1:len(prompt) - 1 + 5]
