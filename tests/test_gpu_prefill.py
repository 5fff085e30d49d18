"""GPU parity of the f16-MFMA prefill GEMM (M >= qmm_gemv_max_m) through the C ABI.

Bars (written into each check):
* max_i|y_i - y64_i| / max_i|y64_i| <= 1e-2 against fp64 on the exact weights;
* max_i|y_i - yo_i| / max_i|yo_i| <= 1e-5 against the fp64 product of the kernel's f16 operands
  (activations rounded to f16, weights from gguf_oracle.dequantize_f16_operands; only the fp32
  accumulation differs), which pins dequantization, scale rounding and the k ordering;
* edge shapes: M, N not multiples of the 128 x 256 tile (M < 256) or of the 256 x 256 wide tile
  (M >= 256), K tails of 32 for Q4_0 / Q8_0, split K, fp16 and fp32 activations and outputs; the
  Llama-3-8B prefill shapes (M = 512) on sampled rows.
"""

import zlib

import numpy as np
import pytest

import gguf_oracle as O

pytestmark = pytest.mark.gpu

TYPES = [O.GGML_Q4_0, O.GGML_Q8_0, O.GGML_Q4_K, O.GGML_Q6_K]
TOL_F64 = 1e-2
TOL_F16 = 1e-5


@pytest.fixture(scope="module")
def dev(cuda):
    import qmm  # noqa: F401
    return cuda


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def run(t, x, raw, N, K, dev, a16=False, c16=False):
    import torch
    import qmm
    A = to_dev(x.astype(np.float16 if a16 else np.float32), dev)
    C = qmm.gemm(t, A, to_dev(raw, dev), N, K, out_dtype=torch.float16 if c16 else torch.float32)
    torch.cuda.synchronize()
    return C.float().cpu().numpy().astype(np.float64)


def shapes(t):
    if t in (O.GGML_Q4_K, O.GGML_Q6_K):
        return [(32, 256, 512), (128, 512, 2048), (200, 300, 1024), (129, 257, 256)]
    return [(32, 256, 512), (128, 512, 2048), (200, 300, 544), (129, 257, 96), (40, 64, 32)]


def wide_shapes(t):
    # The 256 x 256 tile serves M >= 256 when its tiles cover at least half the CUs (>= 128 tiles):
    # exact tiles, ragged M / N with a K tail, and a K long enough to split over workgroups.
    if t in (O.GGML_Q4_K, O.GGML_Q6_K):
        return [(256, 32768, 256), (400, 16428, 1280), (256, 32768, 4096)]
    return [(256, 32768, 128), (448, 16420, 544), (256, 32768, 4096)]


def sampled_cols(rng, N):
    # output columns (weight rows) checked against the oracle: random ones plus the first and
    # the last tile's
    cols = set(rng.choice(N, size=40, replace=False).tolist()) | {0, 1, N - 2, N - 1, (N // 256) * 256}
    return np.array(sorted(c for c in cols if c < N))


def test_prefill_threshold(dev):
    import qmm
    assert qmm.gemv_max_m() == 32


@pytest.mark.parametrize("t", TYPES)
def test_prefill_vs_fp64_and_f16_operands(dev, t):
    rng = np.random.default_rng(4000 + t)
    for M, N, K in shapes(t):
        raw = O.synth_weights(t, N, K, rng)
        x = rng.standard_normal((M, K)).astype(np.float32)
        y = run(t, x, raw, N, K, dev)
        assert O.max_rel_err(y, O.matmul_f64(t, x, raw, N, K)) <= TOL_F64, (O.TYPE_NAMES[t], M, N, K)
        assert O.max_rel_err(y, O.matmul_f16_operands(t, x, raw, N, K)) <= TOL_F16, (O.TYPE_NAMES[t], M, N, K)


@pytest.mark.parametrize("t", TYPES)
def test_prefill_wide_tile_vs_fp64_and_f16_operands(dev, t):
    rng = np.random.default_rng(4100 + t)
    for i, (M, N, K) in enumerate(wide_shapes(t)):
        raw = O.synth_weights(t, N, K, rng)
        x = rng.standard_normal((M, K)).astype(np.float32)
        y = run(t, x, raw, N, K, dev, a16=i == 1, c16=i == 2)
        assert np.all(np.isfinite(y))
        if i == 1:
            x = x.astype(np.float16).astype(np.float32)  # the activations the kernel was given
        cols = sampled_cols(rng, N)
        rb = O.weight_bytes(t, 1, K)
        sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in cols])
        ys = y[:, cols]
        assert O.max_rel_err(ys, O.matmul_f64(t, x, sub, cols.size, K)) <= TOL_F64, (O.TYPE_NAMES[t], M, N, K)
        tol = 1e-3 if i == 2 else TOL_F16  # fp16 output: one more rounding of each result
        assert O.max_rel_err(ys, O.matmul_f16_operands(t, x, sub, cols.size, K)) <= tol, (O.TYPE_NAMES[t], M, N, K)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("a16,c16", [(True, True), (True, False), (False, True)])
def test_prefill_dtypes(dev, t, a16, c16):
    rng = np.random.default_rng(4100 + t)
    M, N, K = 96, 320, 1024
    raw = O.synth_weights(t, N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    xa = x.astype(np.float16).astype(np.float32) if a16 else x
    y = run(t, x, raw, N, K, dev, a16=a16, c16=c16)
    tol_b = 1e-3 if c16 else TOL_F16  # fp16 output rounding: 2^-11 relative
    assert O.max_rel_err(y, O.matmul_f64(t, xa, raw, N, K)) <= TOL_F64
    assert O.max_rel_err(y, O.matmul_f16_operands(t, xa, raw, N, K)) <= tol_b


@pytest.mark.parametrize("t", TYPES)
def test_prefill_reference_quantizer_inputs(dev, t):
    # Inputs built like the reference's own tests (quantize_*_cpu of N(0,1)-scaled weights),
    # at a prefill-sized M.
    rng = np.random.default_rng(4200 + t)
    M, N, K = 64, 256, 1024
    A = (rng.standard_normal((M, K), dtype=np.float32) * 0.2).astype(np.float16)
    B = O.QUANTIZE[t](rng.standard_normal((N, K), dtype=np.float32) * 0.2)
    y = run(t, A.astype(np.float32), B, N, K, dev, a16=True, c16=True)
    assert O.max_rel_err(y, O.matmul_f64(t, A.astype(np.float32), B, N, K)) <= TOL_F64


PREFILL_FULL = [
    ("8b_q4_k_gate", O.GGML_Q4_K, 14336, 4096),
    ("8b_q6_k_down", O.GGML_Q6_K, 4096, 14336),
    ("8b_q8_0_up", O.GGML_Q8_0, 14336, 4096),
]


@pytest.mark.parametrize("name,t,N,K", PREFILL_FULL)
def test_prefill_full_size_m512(dev, name, t, N, K):
    import torch
    import qmm
    rng = np.random.default_rng(zlib.crc32(name.encode()))
    M = 512
    raw = O.synth_weights(t, N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    y = qmm.gemm(t, to_dev(x, dev), to_dev(raw, dev), N, K)
    torch.cuda.synchronize()
    y = y.cpu().numpy().astype(np.float64)
    assert np.all(np.isfinite(y))
    rows = np.sort(rng.choice(N, size=32, replace=False))
    rb = O.weight_bytes(t, 1, K)
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
    assert O.max_rel_err(y[:, rows], O.matmul_f64(t, x, sub, rows.size, K)) <= TOL_F64
    assert O.max_rel_err(y[:, rows], O.matmul_f16_operands(t, x, sub, rows.size, K)) <= TOL_F16


def test_prefill_workspace_release_and_regrow(dev):
    # fp32 activations and a narrow N use the prefill workspace (f16 copy, split-K partials);
    # qmm_release_workspace frees it and the next call re-grows it with identical results.
    import torch
    import qmm
    t = O.GGML_Q6_K
    rng = np.random.default_rng(4300)
    M, N, K = 64, 256, 4096
    raw = O.synth_weights(t, N, K, rng)
    A = to_dev(rng.standard_normal((M, K)).astype(np.float32), dev)
    W = to_dev(raw, dev)
    y1 = qmm.gemm(t, A, W, N, K)
    torch.cuda.synchronize()
    qmm.check(qmm.lib().qmm_release_workspace())
    y2 = qmm.gemm(t, A, W, N, K)
    torch.cuda.synchronize()
    assert torch.equal(y1, y2)
    assert O.max_rel_err(y2.cpu().numpy().astype(np.float64), O.matmul_f64(t, A.cpu().numpy(), raw, N, K)) <= TOL_F64
