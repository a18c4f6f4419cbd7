"""mdx_sample_topk_noalloc: the device sampler with its scratch in a static
device array of the library (no allocation in the call), against the
allocating entry point it is a variant of, mdx_debug_sample (penalty 1).

Calls in a row on the same device: the full 151936-entry vocabulary at
top-k 40, then a smaller vocabulary and k (the scratch keeps the first
call's contents, which the second must not see), then both radix-select
paths through the static scratch (top-k 300, and a 300001-entry vocabulary
at top-k 12).  A call issued under stream capture and replayed from the
graph three times, with new logits between the replays.  Bar: the same bits
(the two entries run the same kernels on the same logits).  Also: a top_k
beyond the scratch's 1024 candidates is refused before anything runs.
"""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _dev(L, nbytes):
    p = C.c_void_p()
    assert L.mdx_device_malloc(C.byref(p), nbytes) == 0
    return p


def _noalloc(mdx, x, k, T, top_p, u):
    L = mdx.lib()
    V = x.size
    d_logits, d_out = _dev(L, V * 4), _dev(L, 8)
    d_idx, d_val = _dev(L, k * 4), _dev(L, k * 4)
    try:
        assert L.mdx_memcpy_h2d(d_logits, x.ctypes.data, V * 4) == 0
        rc = L.mdx_sample_topk_noalloc(d_logits, V, T, k, top_p, u, d_out, d_idx, d_val, None)
        assert rc == 0
        assert L.mdx_device_synchronize() == 0
        out = np.zeros(2, np.int32)
        idx = np.zeros(k, np.int32)
        val = np.zeros(k, np.float32)
        assert L.mdx_memcpy_d2h(out.ctypes.data, d_out, 8) == 0
        assert L.mdx_memcpy_d2h(idx.ctypes.data, d_idx, k * 4) == 0
        assert L.mdx_memcpy_d2h(val.ctypes.data, d_val, k * 4) == 0
        back = np.empty_like(x)
        assert L.mdx_memcpy_d2h(back.ctypes.data, d_logits, V * 4) == 0
        assert np.array_equal(back.view(np.uint32), x.view(np.uint32))   # logits are read only
    finally:
        for p in (d_logits, d_out, d_idx, d_val):
            L.mdx_device_free(p)
    return int(out[0]), idx, val, int(out[1])


def test_noalloc_sampler_matches_allocating_entry(mdx, gpu):
    rng = np.random.default_rng(2024)
    cases = [(151936, 40, 0.8, 0.9, 0.37),     # then a smaller input, other k and u
             (5003, 7, 1.0, 1.0, 0.91),
             (151936, 300, 0.7, 0.95, 0.5),    # k > 64: the radix-select path
             (300001, 12, 1.1, 1.0, 0.08)]     # V beyond the two-launch path's ranges
    for V, k, T, top_p, u in cases:
        x = (rng.standard_normal(V) * 3).astype(np.float32)
        x[[11, V // 2]] = x.max()                  # ties at the top
        tok, idx, val, kept = _noalloc(mdx, x, k, T, top_p, u)
        rtok, ridx, rval, rkept = mdx.sample(x, top_k=k, temperature=T, top_p=top_p, u=u)
        assert np.array_equal(idx, ridx) and np.array_equal(val.view(np.uint32), rval.view(np.uint32))
        assert (tok, kept) == (rtok, rkept)


def test_noalloc_sampler_rejects_k_beyond_scratch(mdx, gpu, capfd):
    L = mdx.lib()
    V = 4096
    d_logits, d_out = _dev(L, V * 4), _dev(L, 8)
    try:
        rc = L.mdx_sample_topk_noalloc(d_logits, V, 1.0, 1025, 1.0, 0.5, d_out, None, None, None)
        assert rc == -1
        assert "exceeds the scratch capacity" in capfd.readouterr().err
        assert L.mdx_sample_topk_noalloc(d_logits, V, 1.0, 0, 1.0, 0.5, d_out, None, None, None) == -1
    finally:
        L.mdx_device_free(d_logits)
        L.mdx_device_free(d_out)


def _hip():
    """The HIP runtime the library links (already loaded with it)."""
    import os
    for name in ("libamdhip64.so.7", "libamdhip64.so.6", "libamdhip64.so"):
        for d in (os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "lib"), ""):
            try:
                return C.CDLL(os.path.join(d, name) if d else name, mode=C.RTLD_GLOBAL)
            except OSError:
                continue
    pytest.fail("libamdhip64 not found")


def test_noalloc_sampler_under_graph_capture(mdx, gpu):
    """The call recorded by stream capture (after a first call outside the
    capture, which looks up the device's scratch address) and replayed three
    times from the graph, with new logits copied into the same buffer between
    replays and other device work between them; every replay matches the
    allocating entry on those logits bit for bit."""
    L, H = mdx.lib(), _hip()
    V, k, T, top_p, u = 151936, 50, 0.9, 0.9, 0.61
    rng = np.random.default_rng(31)
    x0 = (rng.standard_normal(V) * 3).astype(np.float32)
    _noalloc(mdx, x0, k, T, top_p, u)                     # first call on the device: outside capture
    d_logits, d_out = _dev(L, V * 4), _dev(L, 8)
    d_idx, d_val = _dev(L, k * 4), _dev(L, k * 4)
    stream, graph, exe = C.c_void_p(), C.c_void_p(), C.c_void_p()
    assert H.hipStreamCreate(C.byref(stream)) == 0
    try:
        assert L.mdx_memcpy_h2d(d_logits, x0.ctypes.data, V * 4) == 0
        assert H.hipStreamBeginCapture(stream, 2) == 0           # relaxed capture mode
        rc = L.mdx_sample_topk_noalloc(d_logits, V, T, k, top_p, u, d_out, d_idx, d_val, stream)
        assert H.hipStreamEndCapture(stream, C.byref(graph)) == 0
        assert rc == 0
        assert H.hipGraphInstantiate(C.byref(exe), graph, None, None, C.c_size_t(0)) == 0
        for rep in range(3):
            x = (rng.standard_normal(V) * (2 + rep)).astype(np.float32)
            x[[rep * 1000 + 5, V - 1 - rep]] = x.max()
            assert L.mdx_memcpy_h2d(d_logits, x.ctypes.data, V * 4) == 0
            assert L.mdx_device_synchronize() == 0
            assert H.hipGraphLaunch(exe, stream) == 0
            assert H.hipStreamSynchronize(stream) == 0
            out = np.zeros(2, np.int32)
            idx = np.zeros(k, np.int32)
            val = np.zeros(k, np.float32)
            assert L.mdx_memcpy_d2h(out.ctypes.data, d_out, 8) == 0
            assert L.mdx_memcpy_d2h(idx.ctypes.data, d_idx, k * 4) == 0
            assert L.mdx_memcpy_d2h(val.ctypes.data, d_val, k * 4) == 0
            rtok, ridx, rval, rkept = mdx.sample(x, top_k=k, temperature=T, top_p=top_p, u=u)
            assert np.array_equal(idx, ridx), rep
            assert np.array_equal(val.view(np.uint32), rval.view(np.uint32)), rep
            assert (int(out[0]), int(out[1])) == (rtok, rkept), rep
            _noalloc(mdx, x, 7, 1.0, 1.0, 0.5)                   # other eager work on the scratch
    finally:
        if exe.value:
            H.hipGraphExecDestroy(exe)
        if graph.value:
            H.hipGraphDestroy(graph)
        H.hipStreamDestroy(stream)
        for p in (d_logits, d_out, d_idx, d_val):
            L.mdx_device_free(p)
