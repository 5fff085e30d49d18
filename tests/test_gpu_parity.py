"""GPU parity of the HIP path against the oracle (run on an MI355X; every call goes through the
C ABI of libqmm_gfx950.so).

Bars (tolerances are written into each check):
* dequantize: bit-exact against the oracle in fp16, bf16 and fp32;
* GEMV (M < qmm_gemv_max_m): max_i|y_i - y64_i| / max_i|y64_i| <= 1e-3 against fp64 on the
  exact weights, and the reference tests' own absolute tolerances against the reference
  formula (fp16-rounded weights, fp32 matmul);
* row results bit-identical for every M in the GEMV range in row-identity mode (the
  reference's invariant, tests/test_phase5_scale.py:274-310, 371-379), and within each kernel
  family in the default mode (Q4_K from M = 2 and Q6_K from M = 3 run the matrix-core GEMV, smaller
  M the v_dot2 GEMV; the families agree within the GEMV bar);
* full 8B / 70B shapes: sampled rows against fp64, linearity in x.
"""

import os
import zlib

import numpy as np
import pytest

import gguf_oracle as O

pytestmark = pytest.mark.gpu

TYPES = [O.GGML_Q4_0, O.GGML_Q8_0, O.GGML_Q4_K, O.GGML_Q6_K]
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kat_blocks.npz")
GEMV_TOL = 1e-3


@pytest.fixture(scope="module")
def dev(cuda):
    import qmm  # noqa: F401  (fails loudly if the library is not built)
    return cuda


def to_dev(a, dev):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def gemm(t, A_np, raw_np, N, K, dev, a_dtype="f32", c_dtype="f32"):
    import torch
    import qmm
    A = to_dev(A_np.astype(np.float32 if a_dtype == "f32" else np.float16), dev)
    W = to_dev(raw_np, dev)
    C = qmm.gemm(t, A, W, N, K, out_dtype=torch.float32 if c_dtype == "f32" else torch.float16)
    torch.cuda.synchronize()
    return C.float().cpu().numpy().astype(np.float64)


# ------------------------------------------------------------------------------ dequantize

@pytest.mark.parametrize("t", TYPES)
def test_dequant_kat_bit_exact(dev, t):
    import torch
    import qmm
    kat = np.load(GOLDEN, allow_pickle=False)
    name = O.TYPE_NAMES[t]
    raw, n = kat[f"{name}_raw"], kat[f"{name}_w64"].size
    W = to_dev(raw, dev)
    f16 = qmm.dequantize(t, W, n, out_dtype=torch.float16).cpu().numpy()
    f32 = qmm.dequantize(t, W, n, out_dtype=torch.float32).cpu().numpy()
    np.testing.assert_array_equal(f16.view(np.uint16), kat[f"{name}_f16"].view(np.uint16))
    np.testing.assert_array_equal(f32.view(np.uint32), kat[f"{name}_f32"].view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("out", ["f16", "bf16", "f32"])
def test_dequant_synthetic_bit_exact(dev, t, out):
    import torch
    import qmm
    rng = np.random.default_rng(100 + t)
    qk, bb = O.BLOCK_INFO[t]
    n = 96 * 4096
    raw = O.synth_weights(t, 96, 4096, rng)
    dt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[out]
    got = qmm.dequantize(t, to_dev(raw, dev), n, out_dtype=dt)
    torch.cuda.synchronize()
    f32 = O.DEQUANT_F32[t](raw, n)
    if out == "f16":
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint16), f32.astype(np.float16).view(np.uint16))
    elif out == "bf16":
        np.testing.assert_array_equal(got.view(torch.int16).cpu().numpy().view(np.uint16), O.f32_to_bf16_bits(f32))
    else:
        np.testing.assert_array_equal(got.cpu().numpy().view(np.uint32), f32.view(np.uint32))


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("blocks", [1, 3, 9, 13, 257])
def test_dequant_ragged_sizes_leave_tail_untouched(dev, t, blocks):
    """Sizes that are not whole multiples of 256 weights (Q4_0 / Q8_0), of eight super-blocks or of
    the 16-super-block batches the K-quant kernels stage through LDS (257 blocks: 16 batches, then
    one block read straight from memory), written into a larger buffer: values bit-exact, the
    sentinel past num_elements untouched."""
    import torch
    import qmm
    rng = np.random.default_rng(31 * blocks + t)
    qk, bb = O.BLOCK_INFO[t]
    n = blocks * qk
    raw = O.synth_weights(t, 1, n, rng)
    for dt, view in ((torch.float16, torch.int16), (torch.float32, torch.int32)):
        out = torch.full((n + 512,), -7.0, dtype=dt, device=dev)
        qmm.dequantize(t, to_dev(raw, dev), n, out=out)
        torch.cuda.synchronize()
        got = out.cpu()
        want = O.DEQUANT_F32[t](raw, n)
        if dt == torch.float16:
            np.testing.assert_array_equal(got[:n].numpy().view(np.uint16), want.astype(np.float16).view(np.uint16))
        else:
            np.testing.assert_array_equal(got[:n].numpy().view(np.uint32), want.view(np.uint32))
        assert torch.all(got[n:] == -7.0), f"{O.TYPE_NAMES[t]} n={n}: write past num_elements"


@pytest.mark.parametrize("t", TYPES)
def test_dequant_weights_2_bytes_off_bit_exact(dev, t):
    """Packed weights starting 2 bytes past a 4-byte boundary (and at one), odd and even block
    counts: the Q6_K dequantizers read blocks that sit 2 bytes off a 4-byte boundary with aligned
    reads and shift them back, never below the first block; 16-byte aligned K-quant weights go
    through the LDS-staged kernels, the others straight from memory.  Values bit-exact."""
    import torch
    import qmm
    rng = np.random.default_rng(77 + t)
    qk, bb = O.BLOCK_INFO[t]
    for blocks in (1, 2, 13, 258):
        n = blocks * qk
        raw = O.synth_weights(t, 1, n, rng)
        want = O.DEQUANT_F32[t](raw, n).astype(np.float16).view(np.uint16)
        for off in (0, 2):
            buf = torch.zeros(raw.size + 16, dtype=torch.uint8, device=dev)
            buf[off:off + raw.size] = to_dev(raw, dev)
            out = torch.empty((n,), dtype=torch.float16, device=dev)
            qmm.dequantize(t, buf[off:off + raw.size], n, out=out)
            torch.cuda.synchronize()
            np.testing.assert_array_equal(out.cpu().numpy().view(np.uint16), want,
                                          err_msg=f"{O.TYPE_NAMES[t]} blocks={blocks} off={off}")


@pytest.mark.parametrize("t", TYPES)
def test_dequant_random_bytes_nan_aware(dev, t):
    import torch
    import qmm
    rng = np.random.default_rng(7 + t)
    qk, bb = O.BLOCK_INFO[t]
    raw = rng.integers(0, 256, size=512 * bb, dtype=np.uint8)
    got = qmm.dequantize(t, to_dev(raw, dev), 512 * qk, out_dtype=torch.float32).cpu().numpy()
    ref = O.DEQUANT_F32[t](raw, 512 * qk)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    ok = ~np.isnan(ref)
    np.testing.assert_array_equal(got[ok].view(np.uint32), ref[ok].view(np.uint32))


REF_VECTORS = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_vectors.npz")


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("which", ["deq", "quant"])
def test_dequant_matches_reference_cpu_output(dev, t, which):
    # fp16 output of the reference's own dequantize_*_cpu (tests/golden/make_ref_vectors.py)
    import torch
    import qmm
    ref = np.load(REF_VECTORS, allow_pickle=False)
    name = O.TYPE_NAMES[t]
    raw = ref[f"{name}_deq_in"] if which == "deq" else ref[f"{name}_quant_out"]
    want = ref[f"{name}_deq_out"] if which == "deq" else ref[f"{name}_quant_deq"]
    got = qmm.dequantize(t, to_dev(raw, dev), want.size, out_dtype=torch.float16).cpu().numpy()
    np.testing.assert_array_equal(got.view(np.uint16), want.view(np.uint16))


def test_dequantize_q4_0_reference_case(dev):
    # tests/test_gguf_and_q4.py:94-112: 1M elements, seed 42, x ~ N(0,1) * 0.1; documented exact.
    import matmul_module
    rng = np.random.default_rng(42)
    n = 1024 * 1024
    q4 = O.quantize_q4_0(rng.standard_normal(n, dtype=np.float32) * 0.1)
    out = np.zeros(n, dtype=np.float16)
    matmul_module.dequantize_q4_0(q4, out, n)
    np.testing.assert_array_equal(out.view(np.uint16), O.dequantize_f16(O.GGML_Q4_0, q4, n).view(np.uint16))


@pytest.mark.parametrize("t,seed", [(O.GGML_Q8_0, 501), (O.GGML_Q4_K, 502), (O.GGML_Q6_K, 611)])
def test_dequantize_host_api_reference_cases(dev, t, seed):
    # tests/test_phase5_scale.py:42-102, 347-356: GPU dequant vs CPU reference (ours: exact).
    import matmul_module
    rng = np.random.default_rng(seed)
    n = {O.GGML_Q8_0: 4096 * 32, O.GGML_Q4_K: 256 * 256, O.GGML_Q6_K: 512 * 256}[t]
    q = O.QUANTIZE[t](rng.standard_normal(n, dtype=np.float32) * 0.4)
    out = np.empty(n, dtype=np.float16)
    getattr(matmul_module, f"dequantize_{O.TYPE_NAMES[t]}")(q, out, n)
    np.testing.assert_array_equal(out.view(np.uint16), O.dequantize_f16(t, q, n).view(np.uint16))


# ------------------------------------------------------------------------------ GEMV

GEMV_SHAPES = {
    # full windows, tail window, tiny, and several windows ending in a half window (K = 14336,
    # the 8B down projection's K: the streamed Q8_0 window's partial last load instruction)
    O.GGML_Q4_0: [(512, 4096), (300, 2304), (64, 256), (257, 14336)],
    O.GGML_Q8_0: [(512, 4096), (300, 2304), (64, 256), (257, 14336)],
    O.GGML_Q4_K: [(512, 4096), (300, 2304), (96, 256)],
    O.GGML_Q6_K: [(512, 4096), (257, 6144), (96, 512)],
}


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("M", [1, 2, 3, 4, 8])
def test_gemv_vs_fp64(dev, t, M):
    rng = np.random.default_rng(1000 * t + M)
    for N, K in GEMV_SHAPES[t]:
        raw = O.synth_weights(t, N, K, rng)
        x = rng.standard_normal((M, K)).astype(np.float32)
        y64 = O.matmul_f64(t, x, raw, N, K)
        y = gemm(t, x, raw, N, K, dev)
        err = O.max_rel_err(y, y64)
        assert err <= GEMV_TOL, (O.TYPE_NAMES[t], M, N, K, err)


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("a_dtype,c_dtype", [("f16", "f16"), ("f16", "f32"), ("f32", "f16")])
def test_gemv_dtypes(dev, t, a_dtype, c_dtype):
    rng = np.random.default_rng(77 + t)
    N, K = GEMV_SHAPES[t][0]
    raw = O.synth_weights(t, N, K, rng)
    x = rng.standard_normal((2, K)).astype(np.float32)
    xa = x.astype(np.float16).astype(np.float32) if a_dtype == "f16" else x
    y64 = O.matmul_f64(t, xa, raw, N, K)
    y = gemm(t, x, raw, N, K, dev, a_dtype=a_dtype, c_dtype=c_dtype)
    assert O.max_rel_err(y, y64) <= GEMV_TOL


@pytest.mark.parametrize("M", [3, 4, 16])
def test_q6k_extreme_subscales_within_bound(dev, M):
    """Q6_K blocks whose sub-scales are all -128 or 127 and whose 6-bit codes are 0, 15, 48 or 63
    (ql and qh bytes all 0x00 or 0xFF), so most products s (u - 32) lie above 2048 in magnitude,
    where the matrix-core GEMV's f16 operand s (u - 32) is rounded (M >= 3, K a multiple of 2048):
    the result stays within the GEMV bar against fp64 on the exact weights, with fp16 activations
    (the decode dtype) and with fp32 activations."""
    rng = np.random.default_rng(4242 + M)
    N, K = 64, 4096
    blk = O.synth_weights(O.GGML_Q6_K, N, K, rng).reshape(-1, 210)
    nb = blk.shape[0]
    blk[:, 0:192] = np.where(rng.integers(0, 2, size=(nb, 192)) == 1, 0xFF, 0x00).astype(np.uint8)
    blk[:, 192:208] = np.where(rng.integers(0, 2, size=(nb, 16)) == 1, 0x80, 0x7F).astype(np.uint8)
    raw = blk.reshape(-1)
    x = rng.standard_normal((M, K)).astype(np.float32)
    for a_dtype in ("f16", "f32"):
        xa = x.astype(np.float16).astype(np.float32) if a_dtype == "f16" else x
        y64 = O.matmul_f64(O.GGML_Q6_K, xa, raw, N, K)
        y = gemm(O.GGML_Q6_K, x, raw, N, K, dev, a_dtype=a_dtype)
        err = O.max_rel_err(y, y64)
        assert err <= GEMV_TOL, (M, a_dtype, err)


@pytest.mark.parametrize("t", TYPES)
def test_gemv_rows_bit_identical_across_m(dev, t):
    import qmm
    rng = np.random.default_rng(601 + t)
    with qmm.row_identity_mode():
        for N, K in GEMV_SHAPES[t][:2] + GEMV_SHAPES[t][-1:]:
            raw = O.synth_weights(t, N, K, rng)
            Mmax = min(qmm.gemv_max_m() - 1, 31)
            x = rng.standard_normal((Mmax, K)).astype(np.float32)
            single = np.stack([gemm(t, x[m:m + 1], raw, N, K, dev)[0] for m in range(Mmax)])
            # 4-row blocks (M % 8 in 1..4) and 8-row blocks (M % 8 == 0 or >= 5) of the v_dot2
            # kernels; one 16-row pass of the matrix-core GEMV
            for M in sorted({2, 3, 4, 5, 7, 8, 9, 12, 13, 16, Mmax}):
                y = gemm(t, x[:M], raw, N, K, dev)
                np.testing.assert_array_equal(y, single[:M], err_msg=f"{O.TYPE_NAMES[t]} M={M} N={N} K={K}")


def mfma_min_m(t, K):
    """Smallest M that runs the matrix-core GEMV in the default mode (99: none)."""
    if t == O.GGML_Q4_K:
        return 2
    if t == O.GGML_Q6_K and K % 2048 == 0:
        return 3
    return 99


@pytest.mark.parametrize("t", TYPES)
def test_default_mode_rows_bit_identical_within_each_family(dev, t):
    """Default mode: every M from the format's matrix-core threshold on (Q4_K 2, Q6_K 3) gives each
    row bit for bit the same result, and so does every M below it (the v_dot2 GEMV); the two families
    agree within the GEMV bar.  Formats without the matrix-core path run one family for every M."""
    import qmm
    assert not qmm.row_identity()
    rng = np.random.default_rng(651 + t)
    for N, K in GEMV_SHAPES[t]:
        raw = O.synth_weights(t, N, K, rng)
        x = rng.standard_normal((16, K)).astype(np.float32)
        thr = mfma_min_m(t, K)
        y16 = gemm(t, x, raw, N, K, dev)
        y1 = np.stack([gemm(t, x[m:m + 1], raw, N, K, dev)[0] for m in range(16)])
        for M in (2, 3, 5, 8, 13):
            want = y16 if M >= thr else y1
            np.testing.assert_array_equal(gemm(t, x[:M], raw, N, K, dev), want[:M],
                                          err_msg=f"{O.TYPE_NAMES[t]} M={M} N={N} K={K}")
        y64 = O.matmul_f64(t, x, raw, N, K)
        assert O.max_rel_err(y1, y64) <= GEMV_TOL and O.max_rel_err(y16, y64) <= GEMV_TOL
        if thr > 16:
            np.testing.assert_array_equal(y1, y16, err_msg=f"{O.TYPE_NAMES[t]} N={N} K={K}")


def test_row_identity_and_thread_threshold_are_per_thread(dev):
    """qmm_set_row_identity and qmm_set_thread_gemv_max_m change the calling thread only."""
    import threading
    import qmm
    base = qmm.gemv_max_m()
    seen = {}

    def other():
        seen["identity"], seen["gmax"] = qmm.row_identity(), qmm.gemv_max_m()
    with qmm.row_identity_mode():
        qmm.set_thread_gemv_max_m(200)
        try:
            assert qmm.row_identity() and qmm.gemv_max_m() == 200
            th = threading.Thread(target=other)
            th.start()
            th.join()
        finally:
            qmm.set_thread_gemv_max_m(0)
    assert seen == {"identity": False, "gmax": base}
    assert not qmm.row_identity() and qmm.gemv_max_m() == base


@pytest.mark.parametrize("t", TYPES)
def test_raised_threshold_keeps_every_m_bit_identical(dev, t):
    """With the GEMV / prefill threshold raised (qmm_set_gemv_max_m), M = 40 and 100 run the GEMV
    family and every row equals its M = 1 call bit for bit, as the reference's TILE_M = 4 kernels
    give at any M; at the default threshold the same rows come from the MFMA tiles and agree with
    them within the prefill bar."""
    import qmm
    rng = np.random.default_rng(811 + t)
    N, K = 96, 4096
    raw = O.synth_weights(t, N, K, rng)
    x = rng.standard_normal((100, K)).astype(np.float32)
    before = qmm.gemv_max_m()
    try:
        qmm.set_gemv_max_m(4096)
        with qmm.row_identity_mode():
            single = np.stack([gemm(t, x[m:m + 1], raw, N, K, dev)[0] for m in range(100)])
            for M in (40, 100):
                np.testing.assert_array_equal(gemm(t, x[:M], raw, N, K, dev), single[:M],
                                              err_msg=f"{O.TYPE_NAMES[t]} M={M}")
    finally:
        qmm.set_gemv_max_m(before)
    # the same through the calling thread's own threshold, the process value untouched
    qmm.set_thread_gemv_max_m(4096)
    try:
        with qmm.row_identity_mode():
            np.testing.assert_array_equal(gemm(t, x[:40], raw, N, K, dev), single[:40])
    finally:
        qmm.set_thread_gemv_max_m(0)
    assert qmm.gemv_max_m() == before
    y = gemm(t, x[:40], raw, N, K, dev)
    assert O.max_rel_err(y, single[:40]) <= 1e-2


@pytest.mark.parametrize("t", TYPES)
def test_gemv_rows_bit_identical_across_m_windowed_f16_io(dev, t):
    """fp16 activations and outputs at K = 16384 (four windows: the 8-row blocks take the windowed
    kernel, the M = 1 call the resident one): every row equals its M = 1 call bit for bit."""
    import torch
    import qmm
    rng = np.random.default_rng(701 + t)
    N, K = 80, 16384
    raw = O.synth_weights(t, N, K, rng)
    x = rng.standard_normal((16, K)).astype(np.float16)
    W = torch.from_numpy(raw).to(dev)

    def run(a):
        C = qmm.gemm(t, torch.from_numpy(np.ascontiguousarray(a)).to(dev), W, N, K, out_dtype=torch.float16)
        torch.cuda.synchronize()
        return C.cpu().numpy()
    with qmm.row_identity_mode():
        single = np.concatenate([run(x[m:m + 1]) for m in range(16)])
        for M in (5, 8, 13, 16):
            np.testing.assert_array_equal(run(x[:M]).view(np.uint16), single[:M].view(np.uint16),
                                          err_msg=f"{O.TYPE_NAMES[t]} M={M}")


@pytest.mark.parametrize("t", TYPES)
def test_gemv_rows_bit_identical_across_m_long_k(dev, t):
    """K = 28672 (seven windows, the 70B down): M = 3, 4 run two 2-row blocks of resident
    activations (four staged rows do not fit the LDS), M = 2 one, M = 5, 8 the windowed 8-row
    kernel; fp32 and fp16 activations.  Every row equals its M = 1 call bit for bit."""
    import torch
    import qmm
    rng = np.random.default_rng(741 + t)
    N, K = 48, 28672
    raw = O.synth_weights(t, N, K, rng)
    W = torch.from_numpy(raw).to(dev)
    for dt in (np.float32, np.float16):
        x = rng.standard_normal((8, K)).astype(dt)

        def run(a):
            C = qmm.gemm(t, torch.from_numpy(np.ascontiguousarray(a)).to(dev), W, N, K, out_dtype=torch.float32)
            torch.cuda.synchronize()
            return C.cpu().numpy()
        with qmm.row_identity_mode():
            single = np.concatenate([run(x[m:m + 1]) for m in range(8)])
            for M in (2, 3, 4, 5, 8):
                np.testing.assert_array_equal(run(x[:M]), single[:M],
                                              err_msg=f"{O.TYPE_NAMES[t]} M={M} {dt.__name__}")


@pytest.mark.parametrize("t", TYPES)
def test_golden_gemv(dev, t):
    kat = np.load(GOLDEN, allow_pickle=False)
    name = O.TYPE_NAMES[t]
    n_rows, k = (int(v) for v in kat[f"{name}_gemv_n"])
    y = gemm(t, kat[f"{name}_gemv_x"], kat[f"{name}_raw"], n_rows, k, dev)
    assert O.max_rel_err(y, kat[f"{name}_gemv_y64"]) <= GEMV_TOL


@pytest.mark.parametrize("t", TYPES)
def test_gemv_unaligned_weights_fallback(dev, t):
    import torch
    import qmm
    rng = np.random.default_rng(31 + t)
    N, K = 64, 2048
    raw = O.synth_weights(t, N, K, rng)
    buf = torch.zeros(raw.size + 16, dtype=torch.uint8, device=dev)
    buf[2:2 + raw.size] = to_dev(raw, dev)
    W = buf[2:2 + raw.size]  # 2-byte aligned: the byte-load fallback must serve it
    x = rng.standard_normal((3, K)).astype(np.float32)
    y = qmm.gemm(t, to_dev(x, dev), W, N, K).cpu().numpy().astype(np.float64)
    assert O.max_rel_err(y, O.matmul_f64(t, x, raw, N, K)) <= GEMV_TOL


# --------------------------------------------------- the reference's own test cases (host API)

def _ref_matmul_case(dev, t, seed, shapes, scale, tol, quant=True):
    import matmul_module
    fn = getattr(matmul_module, f"matmul_{O.TYPE_NAMES[t]}")
    rng = np.random.default_rng(seed)
    for M, N, K in shapes:
        s = scale if scale is not None else 1.0 / np.sqrt(K)
        A = (rng.standard_normal((M, K), dtype=np.float32) * s).astype(np.float16)
        B = O.QUANTIZE[t](rng.standard_normal((N, K), dtype=np.float32) * s)
        C = np.zeros((M, N), dtype=np.float16)
        fn(A, B, C, M, N, K)
        C_ref = O.matmul_reference(t, A, B, N, K).astype(np.float16)
        err = float(np.max(np.abs(C.astype(np.float32) - C_ref.astype(np.float32))))
        assert err < tol, (O.TYPE_NAMES[t], M, N, K, err)
        assert O.max_rel_err(C.astype(np.float64), O.matmul_f64(t, A.astype(np.float32), B, N, K)) <= GEMV_TOL


def test_fused_matmul_q4_0_reference_case(dev):
    # tests/test_gguf_and_q4.py:115-148 (seed 99, abs < 1e-3).
    _ref_matmul_case(dev, O.GGML_Q4_0, 99, [(1, 4096, 4096), (16, 2048, 2048)], None, 1e-3)


def test_matmul_q8_0_reference_case(dev):
    # tests/test_phase5_scale.py:42-69 (seed 501, x 0.2, abs < 1e-2).
    _ref_matmul_case(dev, O.GGML_Q8_0, 501, [(1, 512, 1024), (8, 256, 512)], 0.2, 1e-2)


def test_matmul_q4_k_reference_case(dev):
    # tests/test_phase5_scale.py:72-102 (seed 502, x 0.1, abs < 2e-2, incl. K = 8192).
    _ref_matmul_case(dev, O.GGML_Q4_K, 502, [(1, 256, 512), (8, 256, 512), (1, 1024, 8192)], 0.1, 2e-2)


def test_matmul_q6_k_reference_case(dev):
    # tests/test_phase5_scale.py:358-369 (seed 611, N=64, K=512, M in {1,4,7}, abs < 5e-2).
    _ref_matmul_case(dev, O.GGML_Q6_K, 611, [(1, 64, 512), (4, 64, 512), (7, 64, 512)], 0.2, 5e-2)


@pytest.mark.parametrize("t", TYPES)
def test_prefill_tile_equals_m1_reference_case(dev, t):
    # tests/test_phase5_scale.py:274-310 / 371-379: M in {4, 7, 16} bit-identical to M = 1 calls.
    import matmul_module
    fn = getattr(matmul_module, f"matmul_{O.TYPE_NAMES[t]}")
    rng = np.random.default_rng(601)
    N, K = (128, 256) if t != O.GGML_Q6_K else (64, 512)
    w = O.QUANTIZE[t](rng.standard_normal((N, K), dtype=np.float32) * 0.2)
    for M in (4, 7, 16):
        A = (rng.standard_normal((M, K), dtype=np.float32) * 0.2).astype(np.float16)
        c_all = np.empty((M, N), dtype=np.float16)
        fn(A, w, c_all, M, N, K)
        c_one = np.empty((M, N), dtype=np.float16)
        for m in range(M):
            row = np.empty((1, N), dtype=np.float16)
            fn(np.ascontiguousarray(A[m:m + 1]), w, row, 1, N, K)
            c_one[m] = row[0]
        np.testing.assert_array_equal(c_all.view(np.uint16), c_one.view(np.uint16))


@pytest.mark.parametrize("t", TYPES)
def test_device_launchers_fp16(dev, t):
    import torch
    import qmm
    rng = np.random.default_rng(5 + t)
    N, K = 256, 4096
    raw = O.synth_weights(t, N, K, rng)
    A = rng.standard_normal((3, K)).astype(np.float16)
    C = torch.empty((3, N), dtype=torch.float16, device=dev)
    getattr(qmm, f"matmul_{O.TYPE_NAMES[t]}_device")(to_dev(A, dev), to_dev(raw, dev), C, 3, N, K)
    torch.cuda.synchronize()
    y = C.float().cpu().numpy().astype(np.float64)
    assert O.max_rel_err(y, O.matmul_f64(t, A.astype(np.float32), raw, N, K)) <= GEMV_TOL


def test_empty_and_invalid_on_device(dev):
    import torch
    import qmm
    A = torch.zeros((0, 256), device=dev)
    W = torch.zeros(144 * 4, dtype=torch.uint8, device=dev)
    C = qmm.gemm(O.GGML_Q4_K, A, W, 4, 256)
    assert C.shape == (0, 4)
    with pytest.raises(ValueError):
        qmm.gemm(O.GGML_Q4_K, torch.zeros((1, 200), device=dev), W, 4, 200)


# ------------------------------------------------------------------ full-size shapes

FULL_SHAPES = [
    # the 8B Q8_0 layer's seven GEMVs (q/o, k/v, gate/up, down), fp32 activations
    ("8b_q8_0_gate", O.GGML_Q8_0, 14336, 4096),
    ("8b_q8_0_q", O.GGML_Q8_0, 4096, 4096),
    ("8b_q8_0_kv", O.GGML_Q8_0, 1024, 4096),
    ("8b_q8_0_down", O.GGML_Q8_0, 4096, 14336),
    ("8b_q4_0_down", O.GGML_Q4_0, 4096, 14336),
    ("8b_q4_k_q", O.GGML_Q4_K, 4096, 4096),
    ("8b_q6_k_down", O.GGML_Q6_K, 4096, 14336),
    ("8b_q6_k_lm_head", O.GGML_Q6_K, 128256, 4096),
    ("8b_q4_k_gate_up_rows", O.GGML_Q4_K, 28672, 4096),
    ("70b_q4_k_gate", O.GGML_Q4_K, 28672, 8192),
    ("70b_q4_k_q_o", O.GGML_Q4_K, 8192, 8192),
    ("70b_q4_k_kv", O.GGML_Q4_K, 1024, 8192),
    ("70b_q6_k_down", O.GGML_Q6_K, 8192, 28672),
    ("4k_q4_0", O.GGML_Q4_0, 4096, 4096),
]


@pytest.mark.parametrize("name,t,N,K", FULL_SHAPES)
@pytest.mark.parametrize("M", [1, 4, 16])
def test_full_size_sampled_rows_and_linearity(dev, name, t, N, K, M):
    import torch
    import qmm
    rng = np.random.default_rng(zlib.crc32(name.encode()) + M)
    raw = O.synth_weights(t, N, K, rng)
    W = to_dev(raw, dev)
    # fp16-exact activations on disjoint supports (x1 on even k, x2 on odd k): x1 + x2 and
    # 4 * x1 are exact in every activation format the kernels stage, so the checks below
    # measure the kernel's own arithmetic, not input rounding.
    x1 = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    x2 = rng.standard_normal((M, K)).astype(np.float16).astype(np.float32)
    x1[:, 1::2] = 0.0
    x2[:, 0::2] = 0.0
    y1 = qmm.gemm(t, to_dev(x1, dev), W, N, K)
    y2 = qmm.gemm(t, to_dev(x2, dev), W, N, K)
    y3 = qmm.gemm(t, to_dev(x1 + x2, dev), W, N, K)
    y4 = qmm.gemm(t, to_dev(4.0 * x1, dev), W, N, K)
    torch.cuda.synchronize()
    y1, y2, y3, y4 = (v.cpu().numpy().astype(np.float64) for v in (y1, y2, y3, y4))
    # sampled rows against the fp64 oracle (row bytes are contiguous in the packed matrix)
    rows = np.sort(rng.choice(N, size=48, replace=False))
    rb = O.weight_bytes(t, 1, K)
    sub = np.concatenate([raw[r * rb:(r + 1) * rb] for r in rows])
    for x, y in ((x1, y1), (x1 + x2, y3)):
        assert O.max_rel_err(y[:, rows], O.matmul_f64(t, x, sub, rows.size, K)) <= GEMV_TOL
    # additivity to fp32 accumulation accuracy; scaling by a power of two is exact
    assert np.max(np.abs(y3 - (y1 + y2))) <= 1e-4 * np.max(np.abs(y3))
    np.testing.assert_array_equal(y4, 4.0 * y1)
    assert np.all(np.isfinite(y1))
