"""GPU parity of the f16-MFMA prefill GEMM (M >= qmm_gemv_max_m) through the C ABI.

Bars (written into each check):
* max_i|y_i - y64_i| / max_i|y64_i| <= 1e-2 against fp64 on the exact weights;
* max_i|y_i - yo_i| / max_i|yo_i| <= 1e-5 against the fp64 product of the kernel's f16 operands
  (activations rounded to f16, weights from gguf_oracle.dequantize_f16_operands; only the fp32
  accumulation differs), which pins dequantization, scale rounding and the k ordering;
* edge shapes: M, N not multiples of the 128 x 256 tile (M < 256) or of the 256 x 256 wide tile
  (M >= 256), K tails of 32 for Q4_0 / Q8_0, split K, fp16 and fp32 activations and outputs; the
  Llama-3-8B prefill shapes (M = 512) on sampled rows;
* a wide grid whose last round is split over K in a second launch (single matrices and fused
  pairs with the split inside either matrix): fp16 outputs within 1e-3 of the f16-operand
  product (one more rounding of each result) and of single calls.
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
    # exact tiles, ragged M / N with a K tail, a K long enough to split over workgroups, and
    # fp32 outputs with N % 4 == 2 (rows whose 16-byte column groups straddle the row end or
    # start 8 bytes off a 16-byte boundary, stored element by element).
    if t in (O.GGML_Q4_K, O.GGML_Q6_K):
        return [(256, 32768, 256), (400, 16428, 1280), (256, 32768, 4096), (450, 32770, 256)]
    return [(256, 32768, 128), (448, 16420, 544), (256, 32768, 4096), (450, 32770, 96)]


def sampled_cols(rng, N):
    # output columns (weight rows) checked against the oracle: random ones plus the first and
    # the last tile's
    cols = set(rng.choice(N, size=40, replace=False).tolist()) | {0, 1, N - 2, N - 1, (N // 256) * 256}
    return np.array(sorted(c for c in cols if c < N))


def test_prefill_threshold(dev):
    import qmm
    # M <= 16 stays in the GEMV family: the reference asserts M = 4, 7, 16 bit-identical to M = 1
    assert qmm.gemv_max_m() == 17


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
def test_prefill_small_tile_vs_fp64_and_f16_operands(dev, t):
    """M = 17..32 run the 32-row tile: the threshold row count, ragged M, N and K tails, fp16
    activations and outputs, and a long K over few tiles (split over workgroups, then summed)."""
    rng = np.random.default_rng(4200 + t)
    kq = t in (O.GGML_Q4_K, O.GGML_Q6_K)
    cases = [(17, 256, 512, False), (24, 300, 1024 if kq else 544, True), (31, 257, 256 if kq else 96, False),
             (32, 512, 8192, True), (20, 64, 4096, False)]
    for M, N, K, half in cases:
        raw = O.synth_weights(t, N, K, rng)
        x = rng.standard_normal((M, K)).astype(np.float32)
        if half:
            x = x.astype(np.float16).astype(np.float32)
        y = run(t, x, raw, N, K, dev, a16=half, c16=half)
        tol16 = 1e-3 if half else TOL_F16  # fp16 outputs round to 2^-11 relative
        assert O.max_rel_err(y, O.matmul_f64(t, x, raw, N, K)) <= TOL_F64, (O.TYPE_NAMES[t], M, N, K)
        assert O.max_rel_err(y, O.matmul_f16_operands(t, x, raw, N, K)) <= tol16, (O.TYPE_NAMES[t], M, N, K)


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


@pytest.mark.parametrize("K", [16384, 16640])
def test_prefill_fp32_activations_long_rows(dev, K):
    """fp32 activations are converted to f16 row by row before the MFMA tiles: rows of up to
    16384 values (after padding to the step) are read once and held in registers, longer ones
    take the two-pass conversion.  Both sides of that bound, against fp64 and the f16-operand
    product, with one row scaled past f16's range (its rescaling path)."""
    t = O.GGML_Q4_K
    rng = np.random.default_rng(4500 + K)
    M, N = 40, 64
    raw = O.synth_weights(t, N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[3] *= 1e6
    y = run(t, x, raw, N, K, dev)
    assert np.all(np.isfinite(y))
    assert O.max_rel_err(y, O.matmul_f64(t, x, raw, N, K)) <= TOL_F64
    keep = np.arange(M) != 3  # the rescaled row: fp64 bar only (its operands differ from a plain f16 cast)
    assert O.max_rel_err(y[keep], O.matmul_f16_operands(t, x[keep], raw, N, K)) <= TOL_F16


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


def tail_cols(rng, N, split):
    # sampled columns plus those around the n-tile where the tail launch starts
    cols = set(sampled_cols(rng, N).tolist()) | {split - 2, split - 1, split, split + 1, split + 255, split + 256}
    return np.array(sorted(c for c in cols if 0 <= c < N))


def check_cols(t, x, raw, y, cols, K, tol_b, what):
    rb = O.weight_bytes(t, 1, K)
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in cols])
    ys = y[:, cols]
    assert np.all(np.isfinite(y)), what
    assert O.max_rel_err(ys, O.matmul_f64(t, x, sub, cols.size, K)) <= TOL_F64, what
    assert O.max_rel_err(ys, O.matmul_f16_operands(t, x, sub, cols.size, K)) <= tol_b, what


@pytest.mark.parametrize("t", [O.GGML_Q4_K, O.GGML_Q6_K, O.GGML_Q8_0])
def test_prefill_wide_tail_split(dev, t):
    # cus + 40 wide tiles (M = 256, a ragged last tile, K = 4096: 32 steps of 128) fill the CUs
    # once and leave a last round of 40 tiles.  Those n-tiles run as a second launch with K split
    # over the CUs; its partial tiles are summed into that column range of C.  Checked on
    # columns of the first, the split-adjacent and the last tiles, with fp16 in and out (f16
    # activations read in place) and fp32 in and out (an f16 copy in the same workspace as the
    # partial tiles).
    import torch
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rng = np.random.default_rng(4400 + t)
    M, K = 256, 4096
    N = (cus + 40) * 256 - 100
    raw = O.synth_weights(t, N, K, rng)
    x = rng.standard_normal((M, K)).astype(np.float32)
    for a16, c16 in ((True, True), (False, False)):
        y = run(t, x, raw, N, K, dev, a16=a16, c16=c16)
        xa = x.astype(np.float16).astype(np.float32) if a16 else x
        check_cols(t, xa, raw, y, tail_cols(rng, N, cus * 256), K, 1e-3 if c16 else TOL_F16,
                   (O.TYPE_NAMES[t], a16, c16))


@pytest.mark.parametrize("tiles", ["tail_inside_first", "tail_inside_second"])
def test_prefill_wide_tail_split_fused_segments(dev, tiles):
    # Two matrices on one input through qmm_gemm_batch (one fused launch of cus + 40 wide
    # tiles): the tail starts inside the first matrix (its last 14 n-tiles and all of the
    # second are split), or inside the second (whose first tiles run unsplit).  The first
    # matrix of the second case ends in a ragged tile.  fp16 outputs match single calls (which
    # plan their own splits, so the fp32 sums may round differently) and the f16-operand product
    # on sampled columns within 1e-3: one more rounding of each result.
    import torch
    import qmm
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    t = O.GGML_Q4_K
    rng = np.random.default_rng(4500 + len(tiles))
    M, K = 256, 4096
    if tiles == "tail_inside_first":
        ns = [(cus + 14) * 256, 26 * 256 - 50]
    else:
        ns = [150 * 256 - 10, (cus + 40 - 150) * 256]
    split = cus * 256  # first column (in the concatenated rows) of the tail launch
    x = rng.standard_normal((M, K)).astype(np.float16)
    A = to_dev(x, dev)
    raws = [O.synth_weights(t, n, K, rng) for n in ns]
    Ws = [to_dev(r, dev) for r in raws]
    Cs = [torch.empty((M, n), device=dev, dtype=torch.float16) for n in ns]
    arr = (qmm.GemmDesc * 2)()
    for d, w, c, n in zip(arr, Ws, Cs, ns):
        d.ggml_type, d.A, d.a_dtype, d.W, d.C, d.c_dtype = t, A.data_ptr(), qmm.DTYPE_F16, w.data_ptr(), \
            c.data_ptr(), qmm.DTYPE_F16
        d.M, d.N, d.K = M, n, K
        d.ev_before = d.ev_after = None
    qmm.gemm_batch(arr)
    torch.cuda.synchronize()
    off = 0
    for raw, w, c, n in zip(raws, Ws, Cs, ns):
        y = c.float().cpu().numpy().astype(np.float64)
        ref = qmm.gemm(t, A, w, n, K, out_dtype=torch.float16)
        torch.cuda.synchronize()
        assert O.max_rel_err(y, ref.float().cpu().numpy().astype(np.float64)) <= 1e-3, (tiles, n)
        local = split - off  # the tail's first column inside this matrix (may lie outside it)
        check_cols(t, x.astype(np.float32), raw, y, tail_cols(rng, n, min(max(local, 2), n - 2)), K, 1e-3,
                   (tiles, n))
        off += n


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


@pytest.mark.parametrize("t", TYPES)
def test_prefill_unaligned_weights_bit_identical(dev, t):
    """Weights 2 bytes past a 4-byte boundary, and rows whose byte length is 2 mod 4
    (Q6_K with an odd number of super-blocks per row): the prefill loads such rows' blocks as
    they lie, 4-aligned rows through the aligned-load-and-shift path (Q6_K blocks at odd indices
    start 2 bytes off a 4-byte boundary).  Every case matches the call on a 256-aligned copy of
    the same bytes bit for bit, on the 32-row, 128-row and 256-row (wide) tiles; Q4_K weights that
    are not 16-byte aligned run the GEMV family instead (checked against fp64)."""
    import torch
    import qmm
    rng = np.random.default_rng(4400 + t)
    kq = t in (O.GGML_Q4_K, O.GGML_Q6_K)
    cases = [(24, 300, 2048 if kq else 544), (96, 512, 1280 if kq else 1024), (256, 32768, 512)]
    for M, N, K in cases:
        raw = O.synth_weights(t, N, K, rng)
        A = to_dev(rng.standard_normal((M, K)).astype(np.float16), dev)
        W = to_dev(raw, dev)
        ref = qmm.gemm(t, A, W, N, K, out_dtype=torch.float32)
        buf = torch.zeros(raw.size + 16, dtype=torch.uint8, device=dev)
        buf[2:2 + raw.size] = W
        y = qmm.gemm(t, A, buf[2:2 + raw.size], N, K, out_dtype=torch.float32)
        torch.cuda.synchronize()
        if t == O.GGML_Q4_K:
            # the prefill reads Q4_K headers with 16-byte loads: such weights take the GEMV family
            sub = raw[:min(N, 64) * O.weight_bytes(t, 1, K)]
            yo = O.matmul_f64(t, A.cpu().numpy().astype(np.float32), sub, min(N, 64), K)
            assert O.max_rel_err(y[:, :min(N, 64)].cpu().numpy().astype(np.float64), yo) <= TOL_F64
        else:
            assert torch.equal(y, ref), (O.TYPE_NAMES[t], M, N, K)
        yo = O.matmul_f16_operands(t, A.cpu().numpy().astype(np.float32), raw, N, K) if N <= 512 else None
        if yo is not None:
            assert O.max_rel_err(ref.cpu().numpy().astype(np.float64), yo) <= TOL_F16, (O.TYPE_NAMES[t], M, N, K)
