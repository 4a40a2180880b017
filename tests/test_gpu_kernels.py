"""Per-kernel parity of the HIP library (through the C ABI) against the CPU oracle.

Bars: bit-exact for the Q4_0 codec, repack/dequant, the synthetic-weight recipe and argmax;
GEMV/attention within stated fp32 tolerances (the GEMV keeps each 32-value block of its input as
integers of 2^-22 of the block's largest magnitude: exact where the input is, pinned bit for bit
below).
"""
import ctypes as C

import numpy as np
import pytest

from velox_amd import _lib as L

pytestmark = pytest.mark.gpu

SEED = 20251201


def _layout(hiplib, n, k, s=0, paired=0):
    m = L.Q4Matrix()
    cb, sb = C.c_uint64(), C.c_uint64()
    L.check(hiplib.velox_hip_q4_layout(n, k, s, paired, C.byref(m), C.byref(cb), C.byref(sb)), "layout")
    return m, cb.value, sb.value


class TiledQ4:
    """A Q4_0 matrix uploaded as GGML blocks and repacked on the device."""

    def __init__(self, hiplib, dev, blocks, n, k, s=0, up_blocks=None):
        paired = up_blocks is not None
        self.m, cb, sb = _layout(hiplib, n, k, s, int(paired))
        self.codes = dev.empty(cb, np.uint8)
        self.scales = dev.empty(sb, np.uint8)
        self.m.codes = self.codes.data_ptr()
        self.m.scales = self.scales.data_ptr()
        self._src = []
        for part, b in enumerate([blocks] if not paired else [blocks, up_blocks]):
            src = dev.put(b)
            self._src.append(src)
            L.check(hiplib.velox_hip_q4_0_repack(src.data_ptr(), n, 0, part, C.byref(self.m), None), "repack")


def _weights(oracle, n, k, tag, sigma=0.02):
    w = oracle.fill_normal(n * k, SEED, tag, sigma).reshape(n, k)
    return oracle.q4_0_quantize(w)


def _fp64_gemv(deq: np.ndarray, x: np.ndarray) -> np.ndarray:
    return deq.astype(np.float64) @ x.astype(np.float64)


def _rms(a) -> float:
    return float(np.sqrt(np.mean(np.square(a, dtype=np.float64))))


# (64, 29568): 32 lanes per row over 924 blocks, 4 zero-padded blocks per row
@pytest.mark.parametrize("n,k,s", [(96, 576, 0), (64, 576, 8), (130, 4096, 0), (48, 14336, 0), (200, 1536, 16),
                                   (64, 29568, 0)])
def test_repack_dequant_bitexact(hiplib, oracle, dev, n, k, s):
    blocks = _weights(oracle, n, k, 100 + n)
    t = TiledQ4(hiplib, dev, blocks, n, k, s)
    out = dev.empty(n * k)
    L.check(hiplib.velox_hip_q4_0_dequant(C.byref(t.m), out.data_ptr(), None))
    got = dev.get(out).reshape(n, k)
    want = oracle.q4_0_dequant(blocks, k)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_paired_repack_dequant_bitexact(hiplib, oracle, dev):
    F, H = 100, 576
    g = _weights(oracle, F, H, 7)
    u = _weights(oracle, F, H, 8)
    t = TiledQ4(hiplib, dev, g, F, H, up_blocks=u)
    out = dev.empty(2 * F * H)
    L.check(hiplib.velox_hip_q4_0_dequant(C.byref(t.m), out.data_ptr(), None))
    got = dev.get(out).reshape(2 * F, H)
    assert np.array_equal(got[:F], oracle.q4_0_dequant(g, H))
    assert np.array_equal(got[F:], oracle.q4_0_dequant(u, H))


@pytest.mark.parametrize("rows,k", [(7, 64), (33, 4096)])
def test_fill_normal_and_quantize_bitexact(hiplib, oracle, dev, rows, k):
    x = dev.empty(rows * k)
    L.check(hiplib.velox_hip_fill_normal(x.data_ptr(), rows * k, SEED, 77, 0.02, 0.0, None))
    xh = dev.get(x)
    want = oracle.fill_normal(rows * k, SEED, 77, 0.02)
    assert np.array_equal(xh.view(np.uint32), want.view(np.uint32))
    blk = dev.empty(rows * (k // 32) * 18, np.uint8)
    L.check(hiplib.velox_hip_q4_0_quantize(x.data_ptr(), rows, k, blk.data_ptr(), None))
    got = dev.get(blk).reshape(rows, -1)
    assert np.array_equal(got, oracle.q4_0_quantize(want.reshape(rows, k)))


def test_quantize_edge_blocks_bitexact(hiplib, oracle, dev):
    """All-zero block, ties at +-8.5 boundaries, a single large value, subnormal scale."""
    k = 32
    rows = [np.zeros(k), np.full(k, -1.0), np.linspace(-1, 1, k), np.r_[np.zeros(31), 3.0],
            np.full(k, 1e-7), np.arange(k) - 15.5, np.r_[np.full(16, 0.5), np.full(16, -0.5)]]
    x = np.array(rows, np.float32)
    d = dev.put(x.ravel())
    blk = dev.empty(len(rows) * 18, np.uint8)
    L.check(hiplib.velox_hip_q4_0_quantize(d.data_ptr(), len(rows), k, blk.data_ptr(), None))
    assert np.array_equal(dev.get(blk).reshape(len(rows), -1), oracle.q4_0_quantize(x))


def _gemv_case(hiplib, oracle, dev, n, k, mode, norm, bias, s=0):
    rng = np.random.default_rng(n * 31 + k)
    blocks = _weights(oracle, n, k, 300 + k)
    t = TiledQ4(hiplib, dev, blocks, n, k, s)
    x = rng.standard_normal(k).astype(np.float32)
    gain = (1.0 + 0.1 * rng.standard_normal(k)).astype(np.float32) if norm else None
    b = rng.standard_normal(n).astype(np.float32) * 0.1 if bias else None
    res = rng.standard_normal(n).astype(np.float32) if mode == L.GEMV_RESIDUAL else None
    dx, dy = dev.put(x), dev.empty(n)
    dg = dev.put(gain) if norm else None
    db = dev.put(b) if bias else None
    dr = dev.put(res) if res is not None else None
    L.check(hiplib.velox_hip_gemv_q4_0(C.byref(t.m), dx.data_ptr(), dg.data_ptr() if norm else None, 1e-5,
                                       db.data_ptr() if bias else None, dr.data_ptr() if res is not None else None,
                                       dy.data_ptr(), mode, None))
    got = dev.get(dy)
    xn = oracle.rmsnorm(x, gain, 1e-5) if norm else x
    want = oracle.matmul_q4_0(xn, blocks, k)
    tight = _fp64_gemv(oracle.q4_0_dequant(blocks, k), xn)
    if bias:
        want = want + b
        tight = tight + b
    if res is not None:
        want = res + want
        tight = res + tight
    return got, want, tight


# fp32-class bars: an fp16 rounding of the input (2^-12 relative) misses them by a factor of about
# 50, a dropped or misplaced digit of the integer activations by far more
GEMV_RMS, GEMV_MAX = 5e-6, 3e-5


# (256, 18944) and (128, 29568): the Qwen down-projection widths, 32 lanes per row with 16 and 4
# zero-padded blocks per row
@pytest.mark.parametrize("n,k,s", [(4096, 4096, 0), (1024, 14336, 0), (960, 576, 0), (1536, 576, 8), (576, 1536, 0),
                                   (123, 4096, 16), (64, 4096, 4), (256, 18944, 0), (128, 29568, 0)])
def test_gemv_store(hiplib, oracle, dev, n, k, s):
    got, want, tight = _gemv_case(hiplib, oracle, dev, n, k, L.GEMV_STORE, False, False, s)
    # against fp64 over the dequantized rows, and against the fp32 oracle (src/runtime.rs
    # matmul_transposed_f32 over dequantized rows)
    for ref in (tight, want):
        assert _rms(got - ref) < GEMV_RMS * _rms(tight)
        assert np.max(np.abs(got - ref)) < GEMV_MAX * np.max(np.abs(tight))


def test_gemv_norm_bias_residual(hiplib, oracle, dev):
    for mode, norm, bias, n in ((L.GEMV_STORE, True, True, 6144), (L.GEMV_RESIDUAL, False, False, 4096)):
        got, want, tight = _gemv_case(hiplib, oracle, dev, n, 4096, mode, norm, bias)
        for ref in (tight, want):
            assert np.max(np.abs(got - ref)) < GEMV_MAX * np.max(np.abs(tight)), (mode, norm, bias)


def _unit_scale_blocks(rng, n, k) -> np.ndarray:
    """GGML Q4_0 blocks with scale 1.0 and random codes: every weight is the integer q - 8."""
    blk = np.zeros((n, k // 32, 18), np.uint8)
    blk[:, :, 0:2] = np.frombuffer(np.float16(1.0).tobytes(), np.uint8)
    blk[:, :, 2:] = rng.integers(0, 256, size=(n, k // 32, 16), dtype=np.uint8)
    return blk.reshape(n, -1)


@pytest.mark.parametrize("n,k,s", [(96, 576, 0), (64, 4096, 0), (40, 1536, 8)])
def test_gemv_integer_activations_bit_exact(hiplib, oracle, dev, n, k, s):
    """Inputs the kernel's integer blocks represent exactly (multiples of 2^(p - 3) below 2^(p + 1),
    p the vector's exponent, every digit value and sign at every position, zero blocks, blocks with
    one non-zero value) against scale-1 weights: each block's dot product and the row's fp32 sum
    are exact, so the result must equal the fp64 product bit for bit. A wrong digit order, sign
    convention or nibble position breaks it."""
    rng = np.random.default_rng(k + s)
    blocks = _unit_scale_blocks(rng, n, k)
    t = TiledQ4(hiplib, dev, blocks, n, k, s)
    deq = oracle.q4_0_dequant(blocks, k).astype(np.float64)
    assert np.array_equal(deq, np.round(deq)) and deq.min() == -8 and deq.max() == 7
    dy = dev.empty(n)
    for p in (-30, -3, 0, 4, 40):
        x = rng.integers(-16, 16, size=k).astype(np.float64) / 8.0  # [-2, 2), eighths
        x[rng.integers(0, k, size=k // 16)] = -2.0
        x[:32] = 0.0                                                  # a zero block
        x[32:64] = 0.0
        x[40] = 1.875                                                 # a block with one value
        x = (x * 2.0 ** p).astype(np.float32)
        dx = dev.put(x)
        L.check(hiplib.velox_hip_gemv_q4_0(C.byref(t.m), dx.data_ptr(), None, 0.0, None, None, dy.data_ptr(),
                                           L.GEMV_STORE, None))
        got = dev.get(dy).astype(np.float64)
        want = deq @ x.astype(np.float64)
        assert np.array_equal(got, want), (p, np.max(np.abs(got - want)))


def test_gemv_nonfinite_inputs(hiplib, oracle, dev):
    """A NaN in the input makes every output NaN, as the fp32 dot products would; an infinity makes
    every output non-finite."""
    n, k = 64, 576
    blocks = _weights(oracle, n, k, 5)
    t = TiledQ4(hiplib, dev, blocks, n, k)
    dy = dev.empty(n)
    for bad in (np.nan, np.inf):
        x = np.ones(k, np.float32)
        x[100] = bad
        dx = dev.put(x)
        L.check(hiplib.velox_hip_gemv_q4_0(C.byref(t.m), dx.data_ptr(), None, 0.0, None, None, dy.data_ptr(),
                                           L.GEMV_STORE, None))
        got = dev.get(dy)
        assert (np.all(np.isnan(got)) if np.isnan(bad) else not np.any(np.isfinite(got))), bad


@pytest.mark.parametrize("F,H", [(14336, 4096), (1536, 576), (100, 576)])
def test_gemv_swiglu(hiplib, oracle, dev, F, H):
    rng = np.random.default_rng(F)
    g = _weights(oracle, F, H, 11)
    u = _weights(oracle, F, H, 12)
    t = TiledQ4(hiplib, dev, g, F, H, up_blocks=u)
    x = rng.standard_normal(H).astype(np.float32)
    gain = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    dx, dg, dy = dev.put(x), dev.put(gain), dev.empty(F)
    L.check(hiplib.velox_hip_gemv_q4_0(C.byref(t.m), dx.data_ptr(), dg.data_ptr(), 1e-5, None, None,
                                       dy.data_ptr(), L.GEMV_SWIGLU, None))
    got = dev.get(dy)
    xn = oracle.rmsnorm(x, gain, 1e-5)
    want = oracle.swiglu(oracle.matmul_q4_0(xn, g, H), oracle.matmul_q4_0(xn, u, H))
    g64 = _fp64_gemv(oracle.q4_0_dequant(g, H), xn)
    u64 = _fp64_gemv(oracle.q4_0_dequant(u, H), xn)
    tight = g64 / (1.0 + np.exp(-g64)) * u64
    # errors of the product silu(g) * u, so relative to its scale
    scale = max(1.0, float(np.max(np.abs(tight))))
    for ref in (tight, want):
        assert np.max(np.abs(got - ref)) < GEMV_MAX * scale


@pytest.mark.parametrize("V,H", [(49152, 576), (128256, 4096)])
def test_lm_head_argmax(hiplib, oracle, dev, V, H):
    rng = np.random.default_rng(V)
    blocks = _weights(oracle, V, H, 13)
    t = TiledQ4(hiplib, dev, blocks, V, H)
    x = rng.standard_normal(H).astype(np.float32)
    gain = np.ones(H, np.float32)
    dx, dg, dl, dt = dev.put(x), dev.put(gain), dev.empty(V), dev.empty(1, np.uint32)
    for _ in range(2):  # second call checks the self-resetting completion counter
        L.check(hiplib.velox_hip_lm_head_argmax(C.byref(t.m), dx.data_ptr(), dg.data_ptr(), 1e-5, dl.data_ptr(),
                                                dt.data_ptr(), None))
        logits = dev.get(dl)
        tok = int(dev.get(dt).view(np.uint32)[0])
        assert tok == oracle.argmax(logits)  # bit-exact on the GPU's own logits
    want = oracle.matmul_q4_0(oracle.rmsnorm(x, gain, 1e-5), blocks, H)
    assert np.max(np.abs(logits - want)) < GEMV_MAX * np.max(np.abs(want))


def test_argmax_ties_and_nan(hiplib, dev):
    x = np.full(100003, -5.0, np.float32)
    x[[77, 5000, 99999]] = 3.0  # ties -> lowest index
    x[10] = np.nan
    d, o = dev.put(x), dev.empty(1, np.uint32)
    L.check(hiplib.velox_hip_argmax_f32(d.data_ptr(), x.size, o.data_ptr(), None))
    assert int(dev.get(o).view(np.uint32)[0]) == 77
    y = np.full(1000, -np.inf, np.float32)
    d2 = dev.put(y)
    L.check(hiplib.velox_hip_argmax_f32(d2.data_ptr(), y.size, o.data_ptr(), None))
    assert int(dev.get(o).view(np.uint32)[0]) == 0  # reference: best_idx starts at 0


def test_rmsnorm(hiplib, oracle, dev):
    rng = np.random.default_rng(5)
    x = rng.standard_normal(4096).astype(np.float32)
    w = rng.standard_normal(4096).astype(np.float32)
    dx, dw, dy = dev.put(x), dev.put(w), dev.empty(4096)
    L.check(hiplib.velox_hip_rmsnorm(dx.data_ptr(), dw.data_ptr(), 4096, 1e-5, dy.data_ptr(), None))
    np.testing.assert_allclose(dev.get(dy), oracle.rmsnorm(x, w, 1e-5), rtol=2e-6, atol=2e-6)
    # reference known answer: [1,2,3,4] -> 1/sqrt(7.50001) (src/runtime.rs:1552-1557)
    x4 = np.array([1, 2, 3, 4], np.float32)
    dx4, dw4, dy4 = dev.put(x4), dev.put(np.ones(4, np.float32)), dev.empty(4)
    L.check(hiplib.velox_hip_rmsnorm(dx4.data_ptr(), dw4.data_ptr(), 4, 1e-5, dy4.data_ptr(), None))
    assert abs(dev.get(dy4)[0] - 1.0 / np.sqrt(np.float32(7.50001))) < 1e-6


def _bf16(a):
    u = np.asarray(a, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r


def _from_bf16(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


def kv_slot(r):
    """Slot of position r (0..31) inside a V block: slot 8j + 4 half + i holds position 16 half + 4j + i."""
    r = np.asarray(r)
    return 8 * ((r % 16) // 4) + 4 * (r // 16) + r % 4


def kv_to_device(cache):
    """[2][hkv][s][D] (K, V) -> the device layer layout: K [hkv][s_cap][D], V [hkv][s_cap/32][D][32]."""
    _, hkv, s, d = cache.shape
    cap = (s + 31) // 32 * 32
    k = np.zeros((hkv, cap, d), cache.dtype)
    k[:, :s] = cache[0]
    v = np.zeros((hkv, cap, d), cache.dtype)
    v[:, :s] = cache[1]
    vb = np.zeros((hkv, cap // 32, d, 32), cache.dtype)
    r = np.arange(32)
    vb[:, :, :, kv_slot(r)] = v.reshape(hkv, cap // 32, 32, d).transpose(0, 1, 3, 2)
    return np.concatenate([k.ravel(), vb.ravel()])


def kv_from_device(flat, hkv, s, d):
    """Inverse of kv_to_device: the device layer layout -> [2][hkv][s][D]."""
    cap = (s + 31) // 32 * 32
    k = flat[:hkv * cap * d].reshape(hkv, cap, d)
    vb = flat[hkv * cap * d:2 * hkv * cap * d].reshape(hkv, cap // 32, d, 32)
    v = vb[:, :, :, kv_slot(np.arange(32))].transpose(0, 1, 3, 2).reshape(hkv, cap, d)
    return np.stack([k[:, :s], v[:, :s]])


def test_kv_layout_roundtrip():
    """The V block slot order is a permutation of 0..31, and the layout helpers invert each other."""
    assert sorted(kv_slot(np.arange(32)).tolist()) == list(range(32))
    c = np.arange(2 * 3 * 40 * 8, dtype=np.uint16).reshape(2, 3, 40, 8)
    assert np.array_equal(kv_from_device(kv_to_device(c), 3, 40, 8), c)


@pytest.mark.parametrize("hq,hkv,D,pos,smax,splits", [
    (32, 8, 128, 0, 64, 4), (32, 8, 128, 383, 512, 13), (9, 3, 64, 37, 64, 2), (28, 4, 128, 1000, 2048, 64),
    (64, 8, 128, 300, 512, 1), (8, 8, 64, 5, 16, 16)])
def test_attention_decode(hiplib, oracle, dev, hq, hkv, D, pos, smax, splits):
    rng = np.random.default_rng(pos + hq)
    theta = 500000.0
    qkv = rng.standard_normal((hq + 2 * hkv) * D).astype(np.float32)
    cache = _bf16(rng.standard_normal((2, hkv, smax, D)).astype(np.float32))
    dq, dkv, dout = dev.put(qkv), dev.put(kv_to_device(cache).view(np.int16)), dev.empty(hq * D)
    L.check(hiplib.velox_hip_attention_decode(dq.data_ptr(), dkv.data_ptr(), hq, hkv, D, smax, pos, theta, splits,
                                              dout.data_ptr(), None))
    got = dev.get(dout)
    new_cache = kv_from_device(dev.get(dkv).view(np.uint16), hkv, smax, D)
    # oracle: rope q and k (src/runtime.rs:745-768), bf16 K/V, two-pass softmax attention
    q = oracle.rope(qkv[:hq * D], hq, D, pos, theta)
    k_new = oracle.rope(qkv[hq * D:(hq + hkv) * D], hkv, D, pos, theta)
    v_new = qkv[(hq + hkv) * D:]
    kc = _from_bf16(cache[0]).copy()
    vc = _from_bf16(cache[1]).copy()
    kc[:, pos, :] = _from_bf16(_bf16(k_new)).reshape(hkv, D)
    vc[:, pos, :] = _from_bf16(_bf16(v_new)).reshape(hkv, D)
    assert np.array_equal(new_cache[0, :, pos, :], _bf16(k_new).reshape(hkv, D))
    assert np.array_equal(new_cache[1, :, pos, :], _bf16(v_new).reshape(hkv, D))
    k_layer = np.ascontiguousarray(kc[:, :pos + 1, :].transpose(1, 0, 2)).reshape(pos + 1, hkv * D)
    v_layer = np.ascontiguousarray(vc[:, :pos + 1, :].transpose(1, 0, 2)).reshape(pos + 1, hkv * D)
    want = oracle.attention(q, k_layer, v_layer, hq, hkv, D, pos)
    assert np.max(np.abs(got - want)) < 2e-5 * max(1.0, np.max(np.abs(want))) * 10


def _arena_matrix(hiplib, dev, eng, kind, layer):
    m = L.Q4Matrix()
    r0 = C.c_uint32()
    L.check(hiplib.velox_hip_arena_matrix(C.byref(eng.arena), kind, layer, C.byref(m), C.byref(r0)), "arena_matrix")
    rows = 2 * m.n if m.paired else m.n
    out = dev.empty(rows * m.k)
    L.check(hiplib.velox_hip_q4_0_dequant(C.byref(m), out.data_ptr(), None), "dequant")
    return dev.get(out).reshape(rows, m.k), r0.value


@pytest.mark.parametrize("name,cfg,layers", [
    ("smollm_135m", dict(vocab_size=49152, hidden_dim=576, intermediate_dim=1536, num_heads=9, num_kv_heads=3,
                         head_dim=64, rms_norm_eps=1e-5, rope_theta=10000.0, qkv_bias=0, tied_lm_head=1), 2),
    ("qwen2_5_7b", dict(vocab_size=152064, hidden_dim=3584, intermediate_dim=18944, num_heads=28, num_kv_heads=4,
                        head_dim=128, rms_norm_eps=1e-6, rope_theta=1000000.0, qkv_bias=1, tied_lm_head=1), 1),
])
def test_synthesized_model_bitexact(hiplib, oracle, dev, name, cfg, layers):
    """Every tensor the device synthesizes (RNG -> GGML Q4_0 quantizer -> tiled layout, norm gains
    N(1, 0.1), biases) equals the oracle's recipe bit for bit, element by element."""
    from velox_amd.engine import HipDecodeEngine

    seed = 11
    ocfg = dict(cfg, num_layers=layers, max_seq_len=8)
    ref = oracle.Engine(ocfg, seed=seed, norm_sigma=0.1, q4_0=True, kv_bf16=True, threads=8)
    gpu = HipDecodeEngine(name, seed=seed, norm_sigma=0.1, max_seq_len=8, num_layers=layers)
    H, F = cfg["hidden_dim"], cfg["intermediate_dim"]
    mats = [(oracle.T_EMBED, 0, H)]
    for layer in range(layers):
        mats += [(k, layer, H) for k in (oracle.T_Q, oracle.T_K, oracle.T_V, oracle.T_GATE, oracle.T_UP)]
        mats += [(oracle.T_O, layer, cfg["num_heads"] * cfg["head_dim"]), (oracle.T_DOWN, layer, F)]
    for kind, layer, k in mats:
        got, r0 = _arena_matrix(hiplib, dev, gpu, kind, layer)
        want = oracle.q4_0_dequant(ref.tensor(kind, layer).reshape(-1, (k // 32) * 18), k)
        sub = got[r0:r0 + want.shape[0]]
        bad = int(np.count_nonzero(sub.view(np.uint32) != want.view(np.uint32)))
        assert bad == 0, (kind, layer, bad)
    vecs = [(oracle.T_FINAL_NORM, 0)] + [(k, layer) for layer in range(layers)
                                         for k in (oracle.T_ATTN_NORM, oracle.T_MLP_NORM)]
    if cfg["qkv_bias"]:
        vecs += [(k, layer) for layer in range(layers) for k in (oracle.T_BQ, oracle.T_BK, oracle.T_BV)]
    for kind, layer in vecs:
        p, n = C.c_void_p(), C.c_uint64()
        L.check(hiplib.velox_hip_arena_vector(C.byref(gpu.arena), kind, layer, C.byref(p), C.byref(n)), "vector")
        got = np.empty(n.value, np.float32)
        L.memcpy_dtoh(got.ctypes.data, p.value, got.nbytes)
        want = ref.tensor(kind, layer).view(np.float32)
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (kind, layer)
    gpu.close()
    ref.close()
