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


def test_noalloc_lm_head_replays_from_a_hip_graph(hiplib, oracle, dev):
    """Captured once (after one eager call, which looks the array's address up) into a HIP graph and
    replayed with new activations between replays: every replay equals the allocating entry point's
    eager result for the same input, bit for bit."""
    hip = C.CDLL("libamdhip64.so")
    V, H = 49152, 576
    m, keep = _tiled(hiplib, oracle, dev, V, H, 77)
    rng = np.random.default_rng(11)
    gain = (1.0 + 0.1 * rng.standard_normal(H)).astype(np.float32)
    dx, dg = dev.put(rng.standard_normal(H).astype(np.float32)), dev.put(gain)
    l_new, t_new = dev.empty(V), dev.empty(1, np.uint32)
    l_ref, t_ref = dev.empty(V), dev.empty(1, np.uint32)
    args = (C.byref(m), dx.data_ptr(), dg.data_ptr(), 1e-5, l_new.data_ptr(), t_new.data_ptr())
    L.check(hiplib.velox_hip_lm_head_argmax_noalloc(*args, None), "noalloc eager")
    dev.get(t_new)
    st, graph, exe = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert hip.hipStreamCreate(C.byref(st)) == 0
    try:
        assert hip.hipStreamBeginCapture(st, 1) == 0  # thread-local capture
        rc = hiplib.velox_hip_lm_head_argmax_noalloc(*args, st)
        assert hip.hipStreamEndCapture(st, C.byref(graph)) == 0
        L.check(rc, "noalloc captured")
        assert hip.hipGraphInstantiate(C.byref(exe), graph, None, None, C.c_size_t(0)) == 0
        for rep in range(4):
            x = rng.standard_normal(H).astype(np.float32) * (1.0 + rep)
            dx.copy_(dev.torch.from_numpy(x))  # eager work between the replays
            L.check(hiplib.velox_hip_lm_head_argmax(C.byref(m), dx.data_ptr(), dg.data_ptr(), 1e-5,
                                                    l_ref.data_ptr(), t_ref.data_ptr(), None), "lm_head_argmax")
            ref, tok_ref = dev.get(l_ref), int(dev.get(t_ref).view(np.uint32)[0])
            l_new.zero_()
            t_new.zero_()
            dev.get(t_new)
            assert hip.hipGraphLaunch(exe, st) == 0
            assert hip.hipStreamSynchronize(st) == 0
            new = dev.get(l_new)
            assert np.array_equal(ref.view(np.uint32), new.view(np.uint32)), rep
            assert int(dev.get(t_new).view(np.uint32)[0]) == tok_ref == oracle.argmax(new), rep
    finally:
        if exe.value:
            hip.hipGraphExecDestroy(exe)
        if graph.value:
            hip.hipGraphDestroy(graph)
        hip.hipStreamDestroy(st)
    del keep
