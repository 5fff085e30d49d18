"""The benchmark's own launches against the oracle (GPU, through the C ABI).

bench.py times these exact calls; here each one runs on synthetic weights of the same shape and
type and is checked against the oracle:
* the 70B Q4_K_M layer's fused GEMV launches through qmm_gemm_batch, fp16 activations and
  outputs, at M = 1, 4 and 16: q/k/v (8192 + 1024 + 1024 rows x 8192) and gate/up
  (2 x 28672 rows x 8192).  Sampled rows of every matrix (the first, the last, random ones)
  within max_i|y_i - y64_i| / max_i|y64_i| <= 1e-3 of the fp64 product on the exact weights
  (the bar includes the fp16 rounding of the outputs, at most 2^-11 relative), and every
  output bit-identical to the matrix's single qmm_gemm call;
* the 8B prefill's fused gate/up (2 x 14336 x 4096 Q4_K, M = 512, 224 tiles of 256 x 256), with
  fp16 activations and outputs and with fp32 activations and outputs: sampled output columns
  within 1e-3 of the fp64 product of the kernel's f16 operands (oracle.matmul_f16_operands;
  the bar is the fp16 rounding of the outputs or of the fp32 activations plus fp32
  accumulation) and within 1e-2 of fp64 on the exact weights.
"""

import numpy as np
import pytest

import gguf_oracle as O

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-3


@pytest.fixture(scope="module")
def dev(cuda):
    import qmm  # noqa: F401  (fails loudly if the library is not built)
    return cuda


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def batch(items):
    """items: (t, A, W, C, N, K) device tensors -> one qmm_gemm_batch call on the current stream."""
    import torch
    import qmm
    arr = (qmm.GemmDesc * len(items))()
    for d, (t, A, W, C, N, K) in zip(arr, items):
        d.ggml_type, d.A, d.a_dtype, d.W, d.C, d.c_dtype = (t, A.data_ptr(), qmm._dtype_code(A.dtype), W.data_ptr(),
                                                            C.data_ptr(), qmm._dtype_code(C.dtype))
        d.M, d.N, d.K = A.shape[0], N, K
        d.ev_before = d.ev_after = None
    qmm.gemm_batch(arr)
    torch.cuda.synchronize()


def sampled(raw, t, N, K, rows):
    rb = O.weight_bytes(t, 1, K)
    return np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])


FUSED_70B = {
    "qkv": [8192, 1024, 1024],
    "gate_up": [28672, 28672],
}


@pytest.mark.parametrize("name", sorted(FUSED_70B))
@pytest.mark.parametrize("M", [1, 4, 16])
def test_70b_fused_gemv_launch(dev, name, M):
    import torch
    import qmm
    t, K = O.GGML_Q4_K, 8192
    ns = FUSED_70B[name]
    rng = np.random.default_rng(1300 + 10 * M + len(ns))
    print(f"70B fused {name} M={M}", flush=True)
    x = rng.standard_normal((M, K)).astype(np.float16)
    A = to_dev(x, dev)
    raws = [O.synth_weights(t, n, K, rng) for n in ns]
    Ws = [to_dev(r, dev) for r in raws]
    Cs = [torch.full((M, n), float("nan"), device=dev, dtype=torch.float16) for n in ns]
    batch([(t, A, w, c, n, K) for n, w, c in zip(ns, Ws, Cs)])
    for n, w, c, raw in zip(ns, Ws, Cs, raws):
        y = c.cpu()
        ref = qmm.gemm(t, A, w, n, K, out_dtype=torch.float16)
        torch.cuda.synchronize()
        assert torch.equal(y, ref.cpu()), (name, M, n)
        rows = np.unique(np.concatenate([[0, n - 1], rng.choice(n, size=30, replace=False)]))
        y64 = O.matmul_f64(t, x.astype(np.float32), sampled(raw, t, n, K, rows), rows.size, K)
        assert O.max_rel_err(y.float().numpy().astype(np.float64)[:, rows], y64) <= GEMV_TOL, (name, M, n)


@pytest.mark.parametrize("adt", ["f16", "f32"])
def test_8b_prefill_fused_gate_up_launch(dev, adt):
    import torch
    t, M, N, K = O.GGML_Q4_K, 512, 14336, 4096
    rng = np.random.default_rng(1400)
    print(f"8B prefill fused gate+up a{adt}", flush=True)
    x = rng.standard_normal((M, K)).astype(np.float16 if adt == "f16" else np.float32)
    A = to_dev(x, dev)
    raws = [O.synth_weights(t, N, K, rng) for _ in range(2)]
    Ws = [to_dev(r, dev) for r in raws]
    Cs = [torch.empty((M, N), device=dev, dtype=A.dtype) for _ in range(2)]
    batch([(t, A, w, c, N, K) for w, c in zip(Ws, Cs)])
    cols = np.unique(np.concatenate([[0, N - 1, 255, 256], rng.choice(N, size=36, replace=False)]))
    xa = x.astype(np.float32)
    for c, raw in zip(Cs, raws):
        y = c.float().cpu().numpy().astype(np.float64)
        assert np.all(np.isfinite(y))
        sub = sampled(raw, t, N, K, cols)
        assert O.max_rel_err(y[:, cols], O.matmul_f16_operands(t, xa, sub, cols.size, K)) <= 1e-3
        assert O.max_rel_err(y[:, cols], O.matmul_f64(t, xa, sub, cols.size, K)) <= 1e-2
