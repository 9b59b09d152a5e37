"""hx_swiglu_ffn_noalloc through the C ABI: the FFN block with its
intermediates in the library's fixed per-GPU scratch.  Its output must equal
hx_swiglu_ffn's bit for bit (the same kernels and configurations run), on two
calls in a row, the second with fewer tokens; it must allocate no device
memory; it can be captured into a HIP graph and replayed; and a shape whose
intermediates exceed the scratch is refused before anything runs."""
import ctypes

import numpy as np
import pytest

from conftest import rng, to_dev, to_np

pytestmark = pytest.mark.gpu

H, I = 4096, 11008


def _weights(hx, dev, seed):
    r = rng(seed)
    wg = r.integers(-127, 128, (H, I), dtype=np.int8)
    wu = r.integers(-127, 128, (H, I), dtype=np.int8)
    wd = r.integers(-127, 128, (I, H), dtype=np.int8)
    sg = (r.uniform(0.5, 1.5, I) / (127 * np.sqrt(H / 3))).astype(np.float16)
    su = (r.uniform(0.5, 1.5, I) / (127 * np.sqrt(H / 3))).astype(np.float16)
    sd = (r.uniform(0.5, 1.5, H) / (127 * np.sqrt(I / 3))).astype(np.float16)
    return (hx.ResidentWeight(to_dev(wg, dev), to_dev(sg, dev)), hx.ResidentWeight(to_dev(wu, dev), to_dev(su, dev)),
            hx.ResidentWeight(to_dev(wd, dev), to_dev(sd, dev)))


def _noalloc(hx, x, gamma, eps, Wg, Wu, Wd, y, stream):
    from hexagon_mlir_amd import ops
    fn = hx._abi.load().hx_swiglu_ffn_noalloc
    mx, mg, my = ops.memref2d(x, "x"), ops.memref1d(gamma, "gamma"), ops.memref2d(y, "y")
    return fn(ctypes.byref(mx), ctypes.byref(mg), eps, Wg.handle, Wu.handle, Wd.handle, ctypes.byref(my),
              ctypes.c_void_p(stream.cuda_stream))


def test_noalloc_matches_and_allocates_nothing(hx, dev):
    """No-allocation calls in a row (256 tokens: the fused gate/up GEMM and
    the K-split down projection; 64 and 40: the decode GEMVs' four row
    blocks, the down projection's split over workgroups; then 24 tokens:
    the decode GEMVs, the down
    projection's two row blocks split over workgroups; then 16: the down
    projection's decode GEMV split over workgroups; the splits' partials and
    counters in the scratch) leave the device's free memory unchanged and
    equal hx_swiglu_ffn bit for bit.  A
    warm-up pass first lets the HIP runtime load the kernels' code objects
    and set up the stream (its own lazy allocations, not the call's)."""
    import torch
    Wg, Wu, Wd = _weights(hx, dev, 500)
    stream = torch.cuda.Stream()  # a stream the workspace path has never seen
    # set-up: hx_init resolves this device's scratch (and loads the code
    # object that holds it)
    assert hx._abi.load().hx_init() == 0, hx._abi.last_error()
    try:
        gamma = to_dev(rng(501).normal(1, 0.1, H).astype(np.float16), dev)
        shapes = (256, 64, 40, 24, 16)
        xs = {T: to_dev(rng(502 + T).normal(0, 1, (T, H)).astype(np.float16), dev) for T in shapes}
        ys = {T: torch.full((T, H), 7.0, dtype=torch.float16, device=dev) for T in shapes}
        refs = {T: torch.full((T, H), 3.0, dtype=torch.float16, device=dev) for T in shapes}
        for T in shapes:  # warm-up
            with torch.cuda.stream(stream):
                assert _noalloc(hx, xs[T], gamma, 1e-6, Wg, Wu, Wd, ys[T], stream) == 0, hx._abi.last_error()
            stream.synchronize()
            ys[T].fill_(7.0)
        torch.cuda.synchronize()
        free_before = torch.cuda.mem_get_info()[0]
        for T in shapes:  # the measured calls, in that order
            with torch.cuda.stream(stream):
                rc = _noalloc(hx, xs[T], gamma, 1e-6, Wg, Wu, Wd, ys[T], stream)
            assert rc == 0, hx._abi.last_error()
            stream.synchronize()
        assert torch.cuda.mem_get_info()[0] == free_before, "the no-allocation calls allocated"
        for T in shapes:
            with torch.cuda.stream(stream):
                hx.swiglu_ffn(xs[T], gamma, 1e-6, Wg, Wu, Wd, out=refs[T])
            stream.synchronize()
            a, b = to_np(refs[T]), to_np(ys[T])
            assert np.isfinite(a.astype(np.float32)).all()
            assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"T={T}"
    finally:
        Wg.release(); Wu.release(); Wd.release()


def test_noalloc_fused_gate_up_with_split_down_gemv(hx, dev):
    """At H = 4096, I = 8192 and 40 tokens the gate and up products take the
    fused GEMM (512 column tiles) while the down projection takes the
    decode GEMV's four row blocks split over workgroups: its partials and
    counters come from the scratch, and the no-allocation call equals
    hx_swiglu_ffn bit for bit."""
    import torch
    Hs, Is, T = 4096, 8192, 40
    r = rng(520)
    ws = []
    for shape, n in (((Hs, Is), Is), ((Hs, Is), Is), ((Is, Hs), Hs)):
        w = to_dev(r.integers(-127, 128, shape, dtype=np.int8), dev)
        sc = to_dev((r.uniform(0.5, 1.5, n) / (127 * np.sqrt(shape[0] / 3))).astype(np.float16), dev)
        ws.append(hx.ResidentWeight(w, sc))
    Wg, Wu, Wd = ws
    stream = torch.cuda.Stream()
    try:
        x = to_dev(rng(521).normal(0, 1, (T, Hs)).astype(np.float16), dev)
        gamma = to_dev(rng(522).normal(1, 0.1, Hs).astype(np.float16), dev)
        y = torch.full((T, Hs), 7.0, dtype=torch.float16, device=dev)
        ref = torch.full((T, Hs), 3.0, dtype=torch.float16, device=dev)
        with torch.cuda.stream(stream):
            assert _noalloc(hx, x, gamma, 1e-6, Wg, Wu, Wd, y, stream) == 0, hx._abi.last_error()
            hx.swiglu_ffn(x, gamma, 1e-6, Wg, Wu, Wd, out=ref)
        stream.synchronize()
        a, b = to_np(ref), to_np(y)
        assert np.isfinite(a.astype(np.float32)).all()
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    finally:
        Wg.release(); Wu.release(); Wd.release()


@pytest.mark.parametrize("T", [256, 24, 16])
def test_noalloc_in_a_hip_graph(hx, dev, T):
    """The call captured into a HIP graph (256 tokens: the GEMM path; 24: the
    decode GEMVs; 16: with the K-split decode GEMV, whose counters every
    replay returns to zero), then three replays, each after eager work that rewrites
    the activations and a synchronization, each equal bit for bit to the
    eager hx_swiglu_ffn on the same activations."""
    import torch
    Wg, Wu, Wd = _weights(hx, dev, 520)
    assert hx._abi.load().hx_init() == 0, hx._abi.last_error()
    try:
        gamma = to_dev(rng(521).normal(1, 0.1, H).astype(np.float16), dev)
        x = to_dev(rng(522).normal(0, 1, (T, H)).astype(np.float16), dev)
        y = torch.zeros((T, H), dtype=torch.float16, device=dev)
        ref = torch.zeros((T, H), dtype=torch.float16, device=dev)
        side = torch.cuda.Stream()
        with torch.cuda.stream(side):  # warm-up outside the capture
            assert _noalloc(hx, x, gamma, 1e-6, Wg, Wu, Wd, y, side) == 0, hx._abi.last_error()
        side.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g, stream=side):
            rc = _noalloc(hx, x, gamma, 1e-6, Wg, Wu, Wd, y, torch.cuda.current_stream())
        assert rc == 0, hx._abi.last_error()
        for i in range(3):
            x.copy_(to_dev(rng(530 + i).normal(0, 1, (T, H)).astype(np.float16), dev))
            y.fill_(9.0)
            torch.cuda.synchronize()
            g.replay()
            torch.cuda.synchronize()
            hx.swiglu_ffn(x, gamma, 1e-6, Wg, Wu, Wd, out=ref)
            a, b = to_np(ref), to_np(y)
            assert np.isfinite(a.astype(np.float32)).all()
            assert np.array_equal(a.view(np.uint16), b.view(np.uint16)), f"T={T} replay {i}"
        del g
    finally:
        Wg.release(); Wu.release(); Wd.release()


def test_noalloc_refuses_what_does_not_fit(hx, dev):
    import torch
    Wg, Wu, Wd = _weights(hx, dev, 510)
    try:
        T = 2048  # 16.8 MB + 45 MB of intermediates alone
        x = torch.zeros((T, H), dtype=torch.float16, device=dev)
        gamma = torch.ones(H, dtype=torch.float16, device=dev)
        y = torch.full((T, H), 5.0, dtype=torch.float16, device=dev)
        stream = torch.cuda.current_stream()
        rc = _noalloc(hx, x, gamma, 1e-6, Wg, Wu, Wd, y, stream)
        assert rc == -7, rc  # HX_ERR_UNSUPPORTED
        assert "scratch" in hx._abi.last_error()
        torch.cuda.synchronize()
        assert bool((y == 5.0).all()), "a refused call must launch nothing"
    finally:
        Wg.release(); Wu.release(); Wd.release()
