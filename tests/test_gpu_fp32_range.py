"""fp32 activations outside the f16 range (GPU, through the C ABI of libqmm_gfx950.so).

The reference multiplies fp32 activations in fp32 (tests/test_gguf_and_q4.py:127-128), so a value
above 65504 or below f16's normal range is an ordinary input there.  The GEMV kernels stage
activations as f16: a 4096-k window of one row whose largest magnitude lies outside [2^-14, 65504)
(down to 2^-126, the smallest normal fp32 number) is staged as x * 2^-e and its products are
multiplied by 2^e (both exact while the scaled values are normal); the prefill GEMM does the same
per row.  Bars:
* per activation row m: max_n |y[m, n] - y64[m, n]| / max_n |y64[m, n]| <= 1e-3 (GEMV) or 1e-2
  (prefill) against the fp64 product on the exact weights, with rows scaled by 1e6, 3e4, 1e-7,
  1e-25 and about 1e35 (outputs near 1e37) next to ordinary rows, for every GEMV kernel family (M = 1 calls and M = 6);
* GEMV rows bit-identical for every M in row-identity mode (M = 3 and 6 against M = 1 calls),
  including the two 2-row blocks of resident activations that M = 3, 4 take at K = 28672 (four
  staged rows do not fit the LDS) against the one-row kernel of M = 1.
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


def activations(M, K, rng, w64=None):
    """Row 0: its second 4096-k window times 1e6; row 1: times 1e-7 everywhere; row 2: its
    first window times 3e4 (|x| beyond 65504); row 3: ordinary N(0, 1); row 4: times 1e-25
    everywhere (below 2^-60); row 5: its last window times a power of two that brings the row's
    largest output (fp64, on the weights w64) to [2^122, 2^123), about 1e37, near the top of the
    fp32 range."""
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0, 4096:8192] *= 1e6
    if M > 1:
        x[1] *= 1e-7
    if M > 2:
        x[2, :4096] *= 3e4
    if M > 4:
        x[4] *= 1e-25
    if M > 5:
        x[5, :K - 4096] = 0.0  # the outputs then scale with the window
        top = np.abs(x[5].astype(np.float64) @ w64.T).max()
        x[5, K - 4096:] *= np.float32(2.0 ** (122 - int(np.floor(np.log2(top)))))
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
    import qmm
    rng = np.random.default_rng(100 + t + K)
    N = 64
    w, w64 = weights(t, N, K, rng)
    name = O.TYPE_NAMES.get(t, t)
    x = activations(6, K, rng, w64)
    y64 = x.astype(np.float64) @ w64.T
    y6 = run(t, x, w, N, K, dev)
    y1 = np.concatenate([run(t, x[m:m + 1], w, N, K, dev) for m in range(6)])
    for label, y in (("M=6", y6), ("M=1", y1)):
        assert np.all(np.isfinite(y)), f"{name} K={K} {label}: non-finite outputs"
        errs = row_errors(y, y64)
        assert max(errs) <= 1e-3, f"{name} K={K} {label}: per-row rel err {errs} > 1e-3"
    # row-identity mode: every row equals its own M = 1 call bit for bit
    with qmm.row_identity_mode():
        y6i = run(t, x, w, N, K, dev)
        for m in range(6):
            y1 = run(t, x[m:m + 1], w, N, K, dev)
            assert np.array_equal(y1[0], y6i[m]), f"{name} K={K}: row {m} differs from M=1"
        y3 = run(t, x[:3], w, N, K, dev)
        assert np.array_equal(y3, y6i[:3]), f"{name} K={K}: M=3 rows differ from M=6"


@pytest.mark.parametrize("t", [O.GGML_Q4_K, O.GGML_Q6_K, O.GGML_Q8_0])
@pytest.mark.parametrize("M", [256, 48, 20])  # 256-row (wide, 128 tiles), 128-row and 32-row tiles
def test_prefill_fp32_beyond_f16_range(dev, t, M):
    rng = np.random.default_rng(7 + t + M)
    N, K = (32768, 256) if M >= 256 else (256, 4096)
    w, w64 = weights(t, N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[0] *= 1e6
    x[5, :100] *= 3e5
    x[9] *= 1e-7
    x[17] *= 1e-11
    x[3] *= np.float32(2.0 ** (122 - int(np.floor(np.log2(np.abs(x[3].astype(np.float64) @ w64.T).max())))))
    x[M - 1] *= 1e-25
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
