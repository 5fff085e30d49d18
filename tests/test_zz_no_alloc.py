"""qmm_gemm_noalloc (the allocation-free qmm_gemm) against qmm_gemm, through the C ABI.

Both run the same kernels and launch plans, so results must be bit-identical.  The cases use
the static scratch for both of its contents: the f16 copy of fp32 activations and the split-K
partial tiles (a narrow N splits K over workgroups).  Two calls in a row, the second smaller,
check that the shared array carries nothing from one call into the next; a plan larger than the
array is refused before any launch (QMM_ERR_UNSUPPORTED).  With the per-stream workspaces released
first, a call on a new stream leaves the device's free memory unchanged, and a call captured into a
HIP graph (where a hipMalloc or a stream synchronisation would break the capture) replays bit for
bit like qmm_gemm, on new inputs too.
"""

import numpy as np
import pytest

import gguf_oracle as O

pytestmark = pytest.mark.gpu


def _call(fn, t, X, W, C, M, N, K, a_dt, c_dt):
    import qmm
    qmm.check(fn(t, X.data_ptr(), a_dt, W.data_ptr(), C.data_ptr(), c_dt, M, N, K, qmm._stream_handle()))


@pytest.mark.parametrize("a32", [True, False])
def test_noalloc_matches_gemm_twice(cuda, a32):
    import torch
    import qmm
    lib = qmm.lib()
    rng = np.random.default_rng(4242 + a32)
    # each call smaller than the one before; the second runs the 256 x 256 tile (128 tiles, no K
    # split, its output tile through LDS), the last the 32-row tile with K split 8 ways
    cases = [(O.GGML_Q6_K, 512, 4096, 14336), (O.GGML_Q4_K, 256, 32768, 256), (O.GGML_Q4_K, 64, 1024, 4096),
             (O.GGML_Q4_K, 24, 512, 8192)]
    for t, M, N, K in cases:
        print(f"noalloc case type={t} M={M} N={N} K={K} fp32_in={a32}", flush=True)
        raw = O.synth_weights(t, N, K, rng)
        W = torch.from_numpy(raw).to(cuda)
        x = rng.standard_normal((M, K)).astype(np.float32)
        X = torch.from_numpy(x if a32 else x.astype(np.float16)).to(cuda)
        a_dt = qmm.DTYPE_F32 if a32 else qmm.DTYPE_F16
        ref = torch.empty((M, N), device=cuda, dtype=torch.float32)
        got = torch.full((M, N), float("nan"), device=cuda, dtype=torch.float32)
        _call(lib.qmm_gemm, t, X, W, ref, M, N, K, a_dt, qmm.DTYPE_F32)
        _call(lib.qmm_gemm_noalloc, t, X, W, got, M, N, K, a_dt, qmm.DTYPE_F32)
        torch.cuda.synchronize()
        r, g = ref.cpu().numpy(), got.cpu().numpy()
        np.testing.assert_array_equal(g, r)
        rows = np.sort(rng.choice(N, size=8, replace=False))
        rb = O.weight_bytes(t, 1, K)
        sub = np.concatenate([raw[i * rb:(i + 1) * rb] for i in rows])
        xin = X.float().cpu().numpy()
        assert O.max_rel_err(g[:, rows].astype(np.float64), O.matmul_f64(t, xin, sub, rows.size, K)) <= 1e-2


def test_noalloc_gemv_and_limit(cuda):
    import torch
    import qmm
    lib = qmm.lib()
    rng = np.random.default_rng(7)
    t, N, K = O.GGML_Q4_K, 512, 4096
    raw = O.synth_weights(t, N, K, rng)
    W = torch.from_numpy(raw).to(cuda)
    X = torch.from_numpy(rng.standard_normal((3, K)).astype(np.float16)).to(cuda)
    ref = torch.empty((3, N), device=cuda)
    got = torch.empty((3, N), device=cuda)
    _call(lib.qmm_gemm, t, X, W, ref, 3, N, K, qmm.DTYPE_F16, qmm.DTYPE_F32)
    _call(lib.qmm_gemm_noalloc, t, X, W, got, 3, N, K, qmm.DTYPE_F16, qmm.DTYPE_F32)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())
    # fp32 activations at M = 4096, K = 16384: their f16 copy alone (128 MiB) exceeds the array;
    # the plan is refused before anything runs (the tensors are never read)
    assert lib.qmm_noalloc_scratch_bytes() == 64 << 20
    M, K2, N2 = 4096, 16384, 256
    Xb = torch.empty((M, K2), device=cuda, dtype=torch.float32)
    Wb = torch.empty(qmm.weight_bytes(t, N2, K2), device=cuda, dtype=torch.uint8)
    Cb = torch.empty((M, N2), device=cuda, dtype=torch.float32)
    rc = lib.qmm_gemm_noalloc(t, Xb.data_ptr(), qmm.DTYPE_F32, Wb.data_ptr(), Cb.data_ptr(), qmm.DTYPE_F32, M, N2, K2,
                              qmm._stream_handle())
    assert rc == qmm.QMM_ERR_UNSUPPORTED, rc
    assert "scratch" in qmm.last_error()


# fp32 activations, the 32-row tile with K split over workgroups: both scratch contents in use
COLD = (O.GGML_Q4_K, 24, 512, 8192)


def _cold_case(cuda, seed):
    import torch
    t, M, N, K = COLD
    rng = np.random.default_rng(seed)
    W = torch.from_numpy(O.synth_weights(t, N, K, rng)).to(cuda)
    xs = [torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(cuda) for _ in range(2)]
    return W, xs


def test_noalloc_new_stream_allocates_nothing(cuda):
    """Per-stream workspaces released, a call on a stream that never ran a GEMM leaves the free
    device memory unchanged (qmm_gemm would allocate that stream's workspace there), and matches
    qmm_gemm bit for bit; the call orders itself after the previous one on another stream."""
    import torch
    import qmm
    lib = qmm.lib()
    t, M, N, K = COLD
    W, (X, _) = _cold_case(cuda, 91)
    ref = torch.empty((M, N), device=cuda)
    got = torch.full((M, N), float("nan"), device=cuda)
    _call(lib.qmm_gemm, t, X, W, ref, M, N, K, qmm.DTYPE_F32, qmm.DTYPE_F32)
    _call(lib.qmm_gemm_noalloc, t, X, W, got, M, N, K, qmm.DTYPE_F32, qmm.DTYPE_F32)  # kernels loaded
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        got.fill_(float("nan"))  # the stream's first launch sets up its hardware queue
    torch.cuda.synchronize()
    qmm.check(lib.qmm_release_workspace())
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    with torch.cuda.stream(side):
        _call(lib.qmm_gemm_noalloc, t, X, W, got, M, N, K, qmm.DTYPE_F32, qmm.DTYPE_F32)
    torch.cuda.synchronize()
    free1 = torch.cuda.mem_get_info()[0]
    assert free1 == free0, (free0, free1)
    np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy())


def test_noalloc_captured_in_graph_replays_bit_exact(cuda):
    """qmm_gemm_noalloc captured into a HIP graph with every workspace released: the capture
    succeeds and each replay (eager work and synchronisation between them, the inputs changed
    in place between them) equals qmm_gemm run outside the capture, bit for bit."""
    import torch
    import qmm
    lib = qmm.lib()
    t, M, N, K = COLD
    W, (X0, X1) = _cold_case(cuda, 92)
    X = X0.clone()
    refs = []
    for src in (X0, X1):
        r = torch.empty((M, N), device=cuda)
        _call(lib.qmm_gemm, t, src, W, r, M, N, K, qmm.DTYPE_F32, qmm.DTYPE_F32)
        refs.append(r)
    got = torch.full((M, N), float("nan"), device=cuda)
    torch.cuda.synchronize()
    qmm.check(lib.qmm_release_workspace())
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        rc = lib.qmm_gemm_noalloc(t, X.data_ptr(), qmm.DTYPE_F32, W.data_ptr(), got.data_ptr(), qmm.DTYPE_F32,
                                  M, N, K, qmm._stream_handle())
    assert rc == qmm.QMM_OK, qmm.last_error()
    for rep, (src, ref) in enumerate([(X0, refs[0]), (X1, refs[1]), (X0, refs[0])]):
        print(f"graph replay {rep}", flush=True)
        X.copy_(src)
        got.fill_(float("nan"))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got.cpu().numpy(), ref.cpu().numpy(), err_msg=f"replay {rep}")
    del g
