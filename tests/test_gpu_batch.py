"""GPU tests of qmm_gemm_batch (C ABI), including the fused launch of consecutive descriptors
that share their activations (the q/k/v and gate/up projections of a layer).

Bars (written into each check):
* GEMV sizes: a batch computes exactly what the same descriptors launched one by one compute:
  outputs are bit-identical to single qmm_gemm calls, fused or not;
* every GEMV output is within max_i|y_i - y64_i| / max_i|y64_i| <= 1e-3 of fp64 on the exact
  weights;
* prefill sizes: fused outputs are within 1e-5 (same measure) of single calls and of the fp64
  product of the kernel's f16 operands (only the fp32 summation order may differ), and within
  1e-2 of fp64 on the exact weights;
* descriptors whose outputs overlap each other or the shared input keep sequential semantics.
"""

import numpy as np
import pytest

import gguf_oracle as O

pytestmark = pytest.mark.gpu

TYPES = [O.GGML_Q4_0, O.GGML_Q8_0, O.GGML_Q4_K, O.GGML_Q6_K]
GEMV_TOL = 1e-3


@pytest.fixture(scope="module")
def dev(cuda):
    import qmm  # noqa: F401  (fails loudly if the library is not built)
    return cuda


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def descs_of(items):
    """items: (t, A, W, C, N, K) with device tensors -> ctypes array of GemmDesc."""
    import qmm
    arr = (qmm.GemmDesc * len(items))()
    for d, (t, A, W, C, N, K) in zip(arr, items):
        d.ggml_type, d.A, d.a_dtype, d.W, d.C, d.c_dtype = (t, A.data_ptr(), qmm._dtype_code(A.dtype), W.data_ptr(),
                                                            C.data_ptr(), qmm._dtype_code(C.dtype))
        d.M, d.N, d.K = A.shape[0], N, K
        d.ev_before = d.ev_after = None
    return arr


def single(t, A, W, N, K, out_dtype):
    import torch
    import qmm
    C = qmm.gemm(t, A, W, N, K, out_dtype=out_dtype)
    torch.cuda.synchronize()
    return C.cpu()


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("M", [1, 2, 4, 7])
def test_batch_shared_input_matches_single_launches(dev, t, M):
    # q, k, v-like projections (8:1:1 rows) sharing x, then a second pair sharing another input.
    import torch
    import qmm
    rng = np.random.default_rng(900 + 10 * t + M)
    K = 2048
    x = rng.standard_normal((M, K)).astype(np.float32)
    x2 = rng.standard_normal((M, K)).astype(np.float32)
    A, A2 = to_dev(x, dev), to_dev(x2, dev)
    shapes = [(1024, A, x), (128, A, x), (128, A, x), (768, A2, x2), (256, A2, x2)]
    raws = [O.synth_weights(t, n, K, rng) for n, _, _ in shapes]
    Ws = [to_dev(r, dev) for r in raws]
    Cs = [torch.full((M, n), float("nan"), device=dev) for n, _, _ in shapes]
    qmm.gemm_batch(descs_of([(t, a, w, c, n, K) for (n, a, _), w, c in zip(shapes, Ws, Cs)]))
    torch.cuda.synchronize()
    for (n, a, xx), w, c, raw in zip(shapes, Ws, Cs, raws):
        ref = single(t, a, w, n, K, torch.float32)
        assert torch.equal(c.cpu(), ref), (O.TYPE_NAMES[t], M, n)
        assert O.max_rel_err(c.cpu().numpy().astype(np.float64), O.matmul_f64(t, xx, raw, n, K)) <= GEMV_TOL


@pytest.mark.parametrize("K", [4096, 8192])
def test_batch_gate_up_large_rows_match_single_launches(dev, K):
    """Fused Q4_K gate + up at M = 1 with 16384 rows or more: two rows per wave item (and, with
    one 4096-k window, 4-wave workgroups), odd row counts in both matrices.  Each output matches
    its matrix's single launch (one row per item) bit for bit, and fp64 on sampled rows."""
    import torch
    import qmm
    t = O.GGML_Q4_K
    rng = np.random.default_rng(950 + K)
    x = rng.standard_normal((1, K)).astype(np.float16)
    A = to_dev(x, dev)
    ns = [14337, 8191]
    raws = [O.synth_weights(t, n, K, rng) for n in ns]
    Ws = [to_dev(r, dev) for r in raws]
    Cs = [torch.full((1, n), float("nan"), device=dev, dtype=torch.float16) for n in ns]
    qmm.gemm_batch(descs_of([(t, A, w, c, n, K) for n, w, c in zip(ns, Ws, Cs)]))
    torch.cuda.synchronize()
    rb = O.weight_bytes(t, 1, K)
    for n, w, c, raw in zip(ns, Ws, Cs, raws):
        assert torch.equal(c.cpu(), single(t, A, w, n, K, torch.float16)), n
        rows = np.concatenate([np.sort(rng.choice(n, size=30, replace=False)), [n - 1]])
        sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
        yo = O.matmul_f64(t, x.astype(np.float32), sub, rows.size, K)
        assert O.max_rel_err(c.cpu().numpy().astype(np.float64)[:, rows], yo) <= GEMV_TOL, n


@pytest.mark.parametrize("t", [O.GGML_Q4_K, O.GGML_Q6_K])
def test_batch_more_descriptors_than_one_launch_takes(dev, t):
    # Seven descriptors on one input: served by more than one fused launch.
    import torch
    import qmm
    rng = np.random.default_rng(950 + t)
    M, K = 1, 4096
    x = rng.standard_normal((M, K)).astype(np.float32)
    A = to_dev(x, dev)
    ns = [64, 320, 1024, 96, 512, 32, 256]
    raws = [O.synth_weights(t, n, K, rng) for n in ns]
    Ws = [to_dev(r, dev) for r in raws]
    Cs = [torch.empty((M, n), device=dev, dtype=torch.float16) for n in ns]
    qmm.gemm_batch(descs_of([(t, A, w, c, n, K) for n, w, c in zip(ns, Ws, Cs)]))
    torch.cuda.synchronize()
    for n, w, c, raw in zip(ns, Ws, Cs, raws):
        assert torch.equal(c.cpu(), single(t, A, w, n, K, torch.float16)), n


def test_batch_overlapping_outputs_keep_sequential_order(dev):
    # Both descriptors write the same buffer: the second one's result must be what remains.
    import torch
    import qmm
    t = O.GGML_Q4_K
    rng = np.random.default_rng(970)
    M, N, K = 2, 256, 1024
    A = to_dev(rng.standard_normal((M, K)).astype(np.float32), dev)
    W1, W2 = (to_dev(O.synth_weights(t, N, K, rng), dev) for _ in range(2))
    C = torch.empty((M, N), device=dev)
    qmm.gemm_batch(descs_of([(t, A, W1, C, N, K), (t, A, W2, C, N, K)]))
    torch.cuda.synchronize()
    assert torch.equal(C.cpu(), single(t, A, W2, N, K, torch.float32))


def test_batch_output_feeding_the_next_descriptor(dev):
    # The first descriptor's output is the second one's activations: run in order, the second sees
    # the first one's result.  An output over the descriptor's own input is rejected (every
    # workgroup reads all of A while others write C).
    import torch
    import qmm
    t = O.GGML_Q8_0
    rng = np.random.default_rng(971)
    K = 512
    x = rng.standard_normal((1, K)).astype(np.float32)
    raw1, raw2 = O.synth_weights(t, K, K, rng), O.synth_weights(t, 64, K, rng)
    W1, W2 = to_dev(raw1, dev), to_dev(raw2, dev)
    A = to_dev(x, dev)
    B = torch.empty((1, K), device=dev)
    C2 = torch.empty((1, 64), device=dev)
    qmm.gemm_batch(descs_of([(t, A, W1, B, K, K), (t, B, W2, C2, 64, K)]))
    torch.cuda.synchronize()
    y1 = single(t, to_dev(x, dev), W1, K, K, torch.float32)
    assert torch.equal(B.cpu(), y1)
    assert torch.equal(C2.cpu(), single(t, y1.to(dev), W2, 64, K, torch.float32))
    with pytest.raises(ValueError, match="must not overlap A"):
        qmm.gemm_batch(descs_of([(t, A, W1, A, K, K)]))


def test_batch_events_between_descriptors(dev):
    # An event recorded between two descriptors splits the launch; results are unchanged and
    # the event completes.
    import torch
    import qmm
    t = O.GGML_Q4_K
    rng = np.random.default_rng(972)
    M, K = 1, 2048
    A = to_dev(rng.standard_normal((M, K)).astype(np.float32), dev)
    Ws = [to_dev(O.synth_weights(t, n, K, rng), dev) for n in (512, 128)]
    Cs = [torch.empty((M, n), device=dev) for n in (512, 128)]
    ev = torch.cuda.Event()
    ev.record()  # torch creates the underlying hipEvent_t lazily, on first record
    torch.cuda.synchronize()
    assert ev.cuda_event
    arr = descs_of([(t, A, Ws[0], Cs[0], 512, K), (t, A, Ws[1], Cs[1], 128, K)])
    arr[0].ev_after = ev.cuda_event
    qmm.gemm_batch(arr)
    torch.cuda.synchronize()
    assert ev.query()
    for w, c, n in zip(Ws, Cs, (512, 128)):
        assert torch.equal(c.cpu(), single(t, A, w, n, K, torch.float32))


def test_batch_mixed_types_and_unaligned_weights(dev):
    # Same input, different formats (not fusable across types), and a Q4_K weight at a 2-byte
    # offset inside a run (the byte-load fallback serves it).
    import torch
    import qmm
    rng = np.random.default_rng(973)
    M, K = 3, 2048
    x = rng.standard_normal((M, K)).astype(np.float32)
    A = to_dev(x, dev)
    t4, t6 = O.GGML_Q4_K, O.GGML_Q6_K
    raw_a, raw_b, raw_c = O.synth_weights(t4, 256, K, rng), O.synth_weights(t4, 128, K, rng), O.synth_weights(t6, 192, K, rng)
    buf = torch.zeros(raw_b.size + 16, dtype=torch.uint8, device=dev)
    buf[2:2 + raw_b.size] = to_dev(raw_b, dev)
    Wa, Wb, Wc = to_dev(raw_a, dev), buf[2:2 + raw_b.size], to_dev(raw_c, dev)
    Ca, Cb, Cc = (torch.empty((M, n), device=dev) for n in (256, 128, 192))
    qmm.gemm_batch(descs_of([(t4, A, Wa, Ca, 256, K), (t4, A, Wb, Cb, 128, K), (t6, A, Wc, Cc, 192, K)]))
    torch.cuda.synchronize()
    for t, raw, c, n in ((t4, raw_a, Ca, 256), (t4, raw_b, Cb, 128), (t6, raw_c, Cc, 192)):
        assert O.max_rel_err(c.cpu().numpy().astype(np.float64), O.matmul_f64(t, x, raw, n, K)) <= GEMV_TOL
    assert torch.equal(Ca.cpu(), single(t4, A, Wa, 256, K, torch.float32))
    assert torch.equal(Cc.cpu(), single(t6, A, Wc, 192, K, torch.float32))


PF_TOL_F16 = 1e-5
PF_TOL_F64 = 1e-2


def single_any(t, A, W, N, K, out_dtype):
    return single(t, A, W, N, K, out_dtype).float().numpy().astype(np.float64)


@pytest.mark.parametrize("t", TYPES)
def test_batch_prefill_shared_input_fused(dev, t):
    # q/k/v-like (8:2:2 rows) on one input, then a gate/up-like pair on another, M = 96.
    import torch
    import qmm
    rng = np.random.default_rng(990 + t)
    M, K = 96, 1024
    x = rng.standard_normal((M, K)).astype(np.float32)
    x2 = rng.standard_normal((M, K)).astype(np.float32)
    A, A2 = to_dev(x, dev), to_dev(x2, dev)
    shapes = [(512, A, x), (128, A, x), (128, A, x), (768, A2, x2), (768, A2, x2)]
    raws = [O.synth_weights(t, n, K, rng) for n, _, _ in shapes]
    Ws = [to_dev(r, dev) for r in raws]
    Cs = [torch.full((M, n), float("nan"), device=dev) for n, _, _ in shapes]
    qmm.gemm_batch(descs_of([(t, a, w, c, n, K) for (n, a, _), w, c in zip(shapes, Ws, Cs)]))
    torch.cuda.synchronize()
    for (n, a, xx), w, c, raw in zip(shapes, Ws, Cs, raws):
        y = c.cpu().numpy().astype(np.float64)
        assert O.max_rel_err(y, single_any(t, a, w, n, K, torch.float32)) <= PF_TOL_F16, (O.TYPE_NAMES[t], n)
        assert O.max_rel_err(y, O.matmul_f16_operands(t, xx, raw, n, K)) <= PF_TOL_F16, (O.TYPE_NAMES[t], n)
        assert O.max_rel_err(y, O.matmul_f64(t, xx, raw, n, K)) <= PF_TOL_F64, (O.TYPE_NAMES[t], n)


@pytest.mark.parametrize("t", [O.GGML_Q4_K, O.GGML_Q6_K, O.GGML_Q8_0])
def test_batch_prefill_gate_up_fused_wide_grid(dev, t):
    # Two 16384-row matrices at M = 256: alone each fills 64 tiles of 256 x 256, fused 128, so
    # the fused launch takes the wide tile while single calls do not.  Sampled columns are
    # checked against the oracle and against single calls; fp16 activations and outputs.
    import torch
    import qmm
    rng = np.random.default_rng(995 + t)
    M, N, K = 256, 16384, 1024
    x = rng.standard_normal((M, K)).astype(np.float32)
    A = to_dev(x.astype(np.float16), dev)
    xa = x.astype(np.float16).astype(np.float32)
    raws = [O.synth_weights(t, N, K, rng) for _ in range(2)]
    Ws = [to_dev(r, dev) for r in raws]
    Cs = [torch.empty((M, N), device=dev, dtype=torch.float16) for _ in range(2)]
    qmm.gemm_batch(descs_of([(t, A, w, c, N, K) for w, c in zip(Ws, Cs)]))
    torch.cuda.synchronize()
    cols = np.array(sorted(set(rng.choice(N, size=40, replace=False).tolist()) | {0, N - 1}))
    rb = O.weight_bytes(t, 1, K)
    for w, c, raw in zip(Ws, Cs, raws):
        y = c.float().cpu().numpy().astype(np.float64)
        assert np.all(np.isfinite(y))
        assert O.max_rel_err(y, single_any(t, A, w, N, K, torch.float16)) <= 1e-3  # fp16 outputs
        sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in cols])
        ys = y[:, cols]
        assert O.max_rel_err(ys, O.matmul_f16_operands(t, xa, sub, cols.size, K)) <= 1e-3
        assert O.max_rel_err(ys, O.matmul_f64(t, xa, sub, cols.size, K)) <= PF_TOL_F64


def test_batch_prefill_overlapping_outputs_keep_sequential_order(dev):
    import torch
    import qmm
    t = O.GGML_Q4_K
    rng = np.random.default_rng(998)
    M, N, K = 64, 256, 1024
    A = to_dev(rng.standard_normal((M, K)).astype(np.float32), dev)
    W1, W2 = (to_dev(O.synth_weights(t, N, K, rng), dev) for _ in range(2))
    C = torch.empty((M, N), device=dev)
    qmm.gemm_batch(descs_of([(t, A, W1, C, N, K), (t, A, W2, C, N, K)]))
    torch.cuda.synchronize()
    assert torch.equal(C.cpu(), single(t, A, W2, N, K, torch.float32))
