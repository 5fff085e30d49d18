"""fp32 activations outside the f16 range (GPU, through the C ABI of libqmm_gfx950.so).

The reference multiplies fp32 activations in fp32 (tests/test_gguf_and_q4.py:127-128), so a value
above 65504 or below f16's normal range is an ordinary input there.  The GEMV kernels stage
activations as f16: a 4096-k window of one row whose largest magnitude lies outside [2^-14, 65504)
is staged as x * 2^-e and its products are multiplied by 2^e (both exact); the prefill GEMM does
the same per row.  Bars:
* per activation row m: max_n |y[m, n] - y64[m, n]| / max_n |y64[m, n]| <= 1e-3 (GEMV) or 1e-2
  (prefill) against the fp64 product on the exact weights, with rows scaled by 1e6, 3e4 and 1e-7
  next to ordinary rows;
* GEMV rows bit-identical for every M (M = 3 and 4 against M = 1 calls), including the two
  2-row blocks of resident activations that M = 3, 4 take at K = 28672 (four staged rows do not
  fit the LDS) against the one-row kernel of M = 1.
"""

import numpy as np
import pytest

import gguf_oracle as O

pytestmark = pytest.mark.gpu

TYPES = [O.GGML_Q4_0, O.GGML_Q8_0, O.GGML_Q4_K, O.GGML_Q6_K, O.GGML_F16]


@pytest.fixture(scope="module")
def dev(cuda):
    import qmm  # noqa: F401  (fails loudly if the library is not built)
    return cuda


def weights(t, N, K, rng):
    """Packed weights (uint8) and their exact fp64 values [N, K]."""
    if t == O.GGML_F16:
        w = (rng.standard_normal((N, K)) / 64).astype(np.float16)
        return w, w.astype(np.float64)
    raw = O.synth_weights(t, N, K, rng)
    return raw, O.dequantize_f64(t, raw, N * K).reshape(N, K)


def activations(M, K, rng):
    """Row 0: its second 4096-k window times 1e6; row 1: times 1e-7 everywhere; row 2: its
    first window times 3e4 (|x| beyond 65504); row 3: ordinary N(0, 1)."""
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0, 4096:8192] *= 1e6
    if M > 1:
        x[1] *= 1e-7
    if M > 2:
        x[2, :4096] *= 3e4
    return x


def run(t, x, w, N, K, dev):
    import torch
    import qmm
    A = torch.from_numpy(np.ascontiguousarray(x)).to(dev)
    W = torch.from_numpy(np.ascontiguousarray(w)).to(dev)
    C = qmm.gemm(t, A, W, N, K, out_dtype=torch.float32)
    torch.cuda.synchronize()
    return C.cpu().numpy().astype(np.float64)


def row_errors(y, y64):
    return [float(np.max(np.abs(y[m] - y64[m])) / np.max(np.abs(y64[m]))) for m in range(y.shape[0])]


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("K", [8192, 28672])
def test_gemv_fp32_beyond_f16_range(dev, t, K):
    rng = np.random.default_rng(100 + t + K)
    N = 64
    w, w64 = weights(t, N, K, rng)
    x = activations(4, K, rng)
    y4 = run(t, x, w, N, K, dev)
    y64 = x.astype(np.float64) @ w64.T
    assert np.all(np.isfinite(y4)), f"{O.TYPE_NAMES.get(t, t)} K={K}: non-finite outputs"
    errs = row_errors(y4, y64)
    assert max(errs) <= 1e-3, f"{O.TYPE_NAMES.get(t, t)} K={K}: per-row rel err {errs} > 1e-3"
    # every row equals its own M = 1 call bit for bit
    for m in range(4):
        y1 = run(t, x[m:m + 1], w, N, K, dev)
        assert np.array_equal(y1[0], y4[m]), f"{O.TYPE_NAMES.get(t, t)} K={K}: row {m} differs from M=1"
    y3 = run(t, x[:3], w, N, K, dev)
    assert np.array_equal(y3, y4[:3]), f"{O.TYPE_NAMES.get(t, t)} K={K}: M=3 rows differ from M=4"


@pytest.mark.parametrize("t", [O.GGML_Q4_K, O.GGML_Q6_K, O.GGML_Q8_0])
@pytest.mark.parametrize("M", [48, 20])  # 128-row and 32-row tiles
def test_prefill_fp32_beyond_f16_range(dev, t, M):
    rng = np.random.default_rng(7 + t + M)
    N, K = 256, 4096
    w, w64 = weights(t, N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0] *= 1e6
    x[5, :100] *= 3e5
    x[9] *= 1e-7
    x[17] *= 1e-11
    y = run(t, x, w, N, K, dev)
    y64 = x.astype(np.float64) @ w64.T
    assert np.all(np.isfinite(y))
    errs = row_errors(y, y64)
    assert max(errs) <= 1e-2, f"{O.TYPE_NAMES[t]} prefill: worst per-row rel err {max(errs):.3e} > 1e-2"


def test_ordinary_rows_unchanged_by_a_rescaled_neighbour(dev):
    """A rescaled row does not change the other rows of the launch (the factor is per row)."""
    rng = np.random.default_rng(3)
    N, K = 128, 8192
    w, _ = weights(O.GGML_Q4_K, N, K, rng)
    x = rng.standard_normal((4, K)).astype(np.float32)
    base = run(O.GGML_Q4_K, x, w, N, K, dev)
    x2 = x.copy()
    x2[1] *= 1e6
    y2 = run(O.GGML_Q4_K, x2, w, N, K, dev)
    for m in (0, 2, 3):
        assert np.array_equal(base[m], y2[m])
