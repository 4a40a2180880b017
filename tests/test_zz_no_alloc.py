"""The allocation-free LM head + argmax (velox_hip_lm_head_argmax_noalloc) against the allocating
entry point it varies: identical logits and token, bit for bit (the same kernels), on two calls in
a row, the second on a smaller matrix, so stale candidates of the first call cannot leak into the
second."""
import ctypes as C

import numpy as np
import pytest

from velox_amd import _lib as L

pytestmark = pytest.mark.gpu

SEED = 20251202


def _tiled(hiplib, oracle, dev, n, k, tag):
    m = L.Q4Matrix()
    cb, sb = C.c_uint64(), C.c_uint64()
    L.check(hiplib.velox_hip_q4_layout(n, k, 0, 0, C.byref(m), C.byref(cb), C.byref(sb)), "layout")
    codes, scales = dev.empty(cb.value, np.uint8), dev.empty(sb.value, np.uint8)
    m.codes, m.scales = codes.data_ptr(), scales.data_ptr()
    blocks = oracle.q4_0_quantize(oracle.fill_normal(n * k, SEED, tag, 0.02).reshape(n, k))
    src = dev.put(blocks)
    L.check(hiplib.velox_hip_q4_0_repack(src.data_ptr(), n, 0, 0, C.byref(m), None), "repack")
    return m, (codes, scales, src)


def test_noalloc_lm_head_matches_allocating_entry_point(hiplib, oracle, dev):
    rng = np.random.default_rng(3)
    for V, H in ((128256, 4096), (49152, 576)):  # second call: a smaller head and fewer candidates
        m, keep = _tiled(hiplib, oracle, dev, V, H, 31 + H)
        x = rng.standard_normal(H).astype(np.float32)
        gain = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
        dx, dg = dev.put(x), dev.put(gain)
        l_ref, t_ref = dev.empty(V), dev.empty(1, np.uint32)
        l_new, t_new = dev.empty(V), dev.empty(1, np.uint32)
        L.check(hiplib.velox_hip_lm_head_argmax(C.byref(m), dx.data_ptr(), dg.data_ptr(), 1e-5, l_ref.data_ptr(),
                                                t_ref.data_ptr(), None), "lm_head_argmax")
        L.check(hiplib.velox_hip_lm_head_argmax_noalloc(C.byref(m), dx.data_ptr(), dg.data_ptr(), 1e-5,
                                                        l_new.data_ptr(), t_new.data_ptr(), None), "noalloc")
        ref, new = dev.get(l_ref), dev.get(l_new)
        assert np.array_equal(ref.view(np.uint32), new.view(np.uint32))
        tok = int(dev.get(t_new).view(np.uint32)[0])
        assert tok == int(dev.get(t_ref).view(np.uint32)[0]) == oracle.argmax(new)
        del keep


def test_noalloc_lm_head_rejects_bad_arguments(hiplib, dev):
    m = L.Q4Matrix()
    L.check(hiplib.velox_hip_q4_layout(64, 64, 0, 1, C.byref(m), None, None), "layout")
    buf = dev.empty(64)
    # a paired (gate/up) matrix is not an LM head
    assert hiplib.velox_hip_lm_head_argmax_noalloc(C.byref(m), buf.data_ptr(), None, 1e-5, buf.data_ptr(),
                                                   buf.data_ptr(), None) == L.EINVAL
    assert hiplib.velox_hip_lm_head_argmax_noalloc(None, buf.data_ptr(), None, 1e-5, buf.data_ptr(),
                                                   buf.data_ptr(), None) == L.EINVAL
