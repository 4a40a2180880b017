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
