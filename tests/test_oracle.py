"""CPU tests that pin the oracle (oracle/gguf_oracle.py) before the GPU tests compare against it.

What pins what:
* layouts + dequant formulas  -> known-answer blocks packed byte-by-byte from the GGML layout
  (tests/golden/make_golden.py), expected values from exact fp64 field arithmetic;
* route 1 (restated reference dequantizers) vs route 2 (fields decomposition) -> bit-exact
  agreement on random blocks of every format;
* fp16 / bf16 output rounding -> NumPy's own fp16 cast and torch's bf16 cast (independent
  implementations of round-to-nearest-even);
* GEMV references -> closed forms (constant codes, zero codes) and brute force on tiny inputs;
* the restated test-input quantizers -> the reference's own round-trip bounds
  (tests/test_cpu_only.py:208-228);
* mutation checks plant a mistake in the oracle (never on the GPU) and confirm a KAT fails.
"""

import os

import numpy as np
import pytest

import gguf_oracle as O

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "kat_blocks.npz")
TYPES = [O.GGML_Q4_0, O.GGML_Q8_0, O.GGML_Q4_K, O.GGML_Q6_K]


@pytest.fixture(scope="module")
def kat():
    return np.load(GOLDEN, allow_pickle=False)


@pytest.mark.parametrize("t", TYPES)
def test_kat_dequant_matches_first_principles(kat, t):
    name = O.TYPE_NAMES[t]
    raw = kat[f"{name}_raw"]
    n = kat[f"{name}_w64"].size
    assert raw.size == n // O.BLOCK_INFO[t][0] * O.BLOCK_INFO[t][1]
    np.testing.assert_array_equal(O.dequantize_f64(t, raw, n), kat[f"{name}_w64"])
    f32 = O.DEQUANT_F32[t](raw, n)
    assert f32.dtype == np.float32
    np.testing.assert_array_equal(f32.view(np.uint32), kat[f"{name}_f32"].view(np.uint32))
    f16 = O.dequantize_f16(t, raw, n)
    np.testing.assert_array_equal(f16.view(np.uint16), kat[f"{name}_f16"].view(np.uint16))


def test_kat_q4_0_spec_values(kat):
    # Block 0: d = 1, low nibble j, high nibble 15 - j  ->  w[j] = j - 8, w[16 + j] = 7 - j.
    w = kat["q4_0_w64"][:32]
    np.testing.assert_array_equal(w[:16], np.arange(16) - 8)
    np.testing.assert_array_equal(w[16:], 7 - np.arange(16))
    f16 = O.dequantize_f16(O.GGML_Q4_0, kat["q4_0_raw"], 128)
    # Block 2 has a subnormal fp16 scale (2^-20): products must stay subnormal, not flush.
    sub = f16[64:96].astype(np.float64)
    assert np.all(np.abs(sub[sub != 0]) < 2.0 ** -14)
    assert np.count_nonzero(sub) > 0


@pytest.mark.parametrize("t", TYPES)
@pytest.mark.parametrize("seed", [0, 1])
def test_routes_agree_bitwise(t, seed):
    rng = np.random.default_rng(seed)
    qk, bb = O.BLOCK_INFO[t]
    n = 64 * qk
    raw = O.synth_weights(t, 1, n, rng)
    r1 = O.DEQUANT_F32[t](raw, n)
    r2 = O.dequantize_fields_f32(t, raw, n)
    np.testing.assert_array_equal(r1.view(np.uint32), r2.view(np.uint32))
    # fp32 route equals the exact value rounded once to fp32
    np.testing.assert_array_equal(r1, O.dequantize_f64(t, raw, n).astype(np.float32))


def test_random_byte_blocks_all_formats():
    # Arbitrary bytes (not only the benchmark distributions), including NaN/Inf scales.
    rng = np.random.default_rng(7)
    for t in TYPES:
        qk, bb = O.BLOCK_INFO[t]
        raw = rng.integers(0, 256, size=16 * bb, dtype=np.uint8)
        a = O.DEQUANT_F32[t](raw, 16 * qk)
        b = O.dequantize_fields_f32(t, raw, 16 * qk)
        np.testing.assert_array_equal(np.isnan(a), np.isnan(b))
        ok = ~np.isnan(a)
        np.testing.assert_array_equal(a[ok].view(np.uint32), b[ok].view(np.uint32))


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 100000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1e-45, 3.4e38, 1.0 + 2.0 ** -8,
                                  1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -9], dtype=np.float32)]).astype(np.float32)
    mine = O.f32_to_bf16_bits(x)
    ref = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(mine, ref)
    np.testing.assert_array_equal(O.bf16_bits_to_f32(mine), torch.from_numpy(mine.view(np.int16)).view(torch.bfloat16).float().numpy())


@pytest.mark.parametrize("t", TYPES)
def test_golden_gemv_brute_force(kat, t):
    name = O.TYPE_NAMES[t]
    n_rows, k = (int(v) for v in kat[f"{name}_gemv_n"])
    x = kat[f"{name}_gemv_x"]
    y64 = O.matmul_f64(t, x, kat[f"{name}_raw"], n_rows, k)
    np.testing.assert_allclose(y64, kat[f"{name}_gemv_y64"], rtol=0, atol=1e-12 * np.abs(y64).max())
    # brute force: explicit triple loop over the exact weights
    W = kat[f"{name}_w64"].reshape(n_rows, k)
    brute = np.array([[sum(float(x[m, i]) * float(W[r, i]) for i in range(k)) for r in range(n_rows)]
                      for m in range(x.shape[0])])
    np.testing.assert_allclose(y64, brute, rtol=1e-12, atol=1e-12)


def test_closed_form_constant_codes_q4_k():
    rng = np.random.default_rng(11)
    nsb, c = 4, 9
    d16 = (np.abs(rng.standard_normal(nsb)) * 0.01).astype(np.float16)
    dmin16 = (np.abs(rng.standard_normal(nsb)) * 0.01).astype(np.float16)
    sc = rng.integers(0, 64, (nsb, 8))
    m = rng.integers(0, 64, (nsb, 8))
    raw = O.pack_q4_k(d16, dmin16, sc, m, np.full((nsb, 256), c))
    x = rng.standard_normal(nsb * 256)
    y = O.matmul_f64(O.GGML_Q4_K, x[None, :], raw, 1, nsb * 256)[0, 0]
    xs = x.reshape(nsb, 8, 32).sum(axis=2)
    closed = np.sum((d16.astype(np.float64)[:, None] * sc * c - dmin16.astype(np.float64)[:, None] * m) * xs)
    assert abs(y - closed) <= 1e-12 * max(1.0, abs(closed))


def test_closed_form_constant_codes_q6_k():
    rng = np.random.default_rng(12)
    nsb, u = 3, 50
    d16 = (np.abs(rng.standard_normal(nsb)) * 0.01).astype(np.float16)
    sc = rng.integers(-128, 128, (nsb, 16)).astype(np.int8)
    raw = O.pack_q6_k(d16, sc, np.full((nsb, 256), u))
    x = rng.standard_normal(nsb * 256)
    y = O.matmul_f64(O.GGML_Q6_K, x[None, :], raw, 1, nsb * 256)[0, 0]
    closed = np.sum(d16.astype(np.float64)[:, None] * sc * (u - 32) * x.reshape(nsb, 16, 16).sum(axis=2))
    assert abs(y - closed) <= 1e-12 * max(1.0, abs(closed))


def test_zero_code_cases():
    rng = np.random.default_rng(13)
    # Q4_0 with every code = 8 is the zero matrix.
    q = O.quantize_q4_0(np.zeros(32 * 8, dtype=np.float32))
    raw = q.reshape(8, 18).copy()
    raw[:, 0:2] = np.array([0.75], dtype=np.float16).view(np.uint8)
    raw[:, 2:] = 0x88
    assert np.all(O.dequantize_f64(O.GGML_Q4_0, raw.reshape(-1), 256) == 0)
    # Q4_K with sc = 0 and m > 0 gives y = -dmin * m * sum(x) per sub-block.
    d16 = np.array([0.5], dtype=np.float16)
    dmin16 = np.array([0.25], dtype=np.float16)
    m = rng.integers(1, 64, (1, 8))
    raw = O.pack_q4_k(d16, dmin16, np.zeros((1, 8), int), m, rng.integers(0, 16, (1, 256)))
    x = rng.standard_normal(256)
    y = O.matmul_f64(O.GGML_Q4_K, x[None], raw, 1, 256)[0, 0]
    assert abs(y + 0.25 * np.sum(m[0] * x.reshape(8, 32).sum(axis=1))) < 1e-12


@pytest.mark.parametrize("t,bound", [(O.GGML_Q4_0, 0.08), (O.GGML_Q8_0, 0.01), (O.GGML_Q4_K, 0.06),
                                     (O.GGML_Q6_K, 0.02)])
def test_quantizer_roundtrip_bounds(t, bound):
    # Reference bounds: tests/test_cpu_only.py:208-228 (seed 42, 512 elements x 0.2).
    rng = np.random.default_rng(42)
    x = (rng.standard_normal(512, dtype=np.float32) * 0.2).astype(np.float32)
    q = O.QUANTIZE[t](x)
    assert q.nbytes == 512 // O.BLOCK_INFO[t][0] * O.BLOCK_INFO[t][1]
    d = O.dequantize_f16(t, q, 512).astype(np.float32)
    assert float(np.max(np.abs(x - d))) < bound


@pytest.mark.parametrize("t", TYPES)
def test_synth_distributions(t):
    rng = np.random.default_rng(5)
    qk, bb = O.BLOCK_INFO[t]
    raw = O.synth_weights(t, 8, 4 * qk, rng).reshape(-1, bb)
    off = 208 if t == O.GGML_Q6_K else 0
    d = raw[:, off:off + 2].copy().view(np.float16).astype(np.float32)
    assert np.all(np.isfinite(d)) and np.all(d >= 0)
    assert 0.001 < float(np.median(d)) < 0.05


def test_weight_bytes_shapes():
    # Llama-3-70B Q4_K_M layer: q,o 8192^2; k,v 1024x8192; gate,up 28672x8192 (Q4_K); down Q6_K.
    wb = O.weight_bytes
    q4k = 2 * wb(O.GGML_Q4_K, 8192, 8192) + 2 * wb(O.GGML_Q4_K, 1024, 8192) + 2 * wb(O.GGML_Q4_K, 28672, 8192)
    assert q4k + wb(O.GGML_Q6_K, 8192, 28672) == 541_851_648
    with pytest.raises(ValueError):
        wb(O.GGML_Q4_K, 1, 100)


# ---- mutation checks: a planted mistake in the oracle must be caught by the KATs ----------

def _kat_fails(kat, t):
    name = O.TYPE_NAMES[t]
    n = kat[f"{name}_w64"].size
    try:
        f32 = O.DEQUANT_F32[t](kat[f"{name}_raw"], n)
        f64 = O.dequantize_f64(t, kat[f"{name}_raw"], n)
    except Exception:
        return True
    return (not np.array_equal(f32, kat[f"{name}_f32"])) or (not np.array_equal(f64, kat[f"{name}_w64"]))


def test_mutation_swapped_high_scale_bits_detected(kat, monkeypatch):
    orig = O.get_scale_min_k4

    def swapped(j, q):
        sc, m = orig(j, q)
        return (m, sc) if j >= 4 else (sc, m)

    monkeypatch.setattr(O, "get_scale_min_k4", swapped)
    name = "q4_k"
    n = kat[f"{name}_w64"].size
    assert not np.array_equal(O.dequantize_f64(O.GGML_Q4_K, kat[f"{name}_raw"], n), kat[f"{name}_w64"])


def test_mutation_q6_k_wrong_qh_shift_detected(kat, monkeypatch):
    orig = O.dequantize_q6_k_f32

    def wrong(raw, n):
        b = O._blocks(raw, O.GGML_Q6_K, n).copy()
        b[:, 128:192] = ((b[:, 128:192] >> 2) | (b[:, 128:192] << 6)).astype(np.uint8)  # rotate qh lanes
        return orig(b.reshape(-1), n)

    monkeypatch.setitem(O.DEQUANT_F32, O.GGML_Q6_K, wrong)
    assert _kat_fails(kat, O.GGML_Q6_K)


def test_mutation_q4_0_swapped_nibbles_detected(kat, monkeypatch):
    orig = O.dequantize_q4_0_f32

    def wrong(raw, n):
        b = O._blocks(raw, O.GGML_Q4_0, n).copy()
        b[:, 2:] = ((b[:, 2:] >> 4) | (b[:, 2:] << 4)).astype(np.uint8)
        return orig(b.reshape(-1), n)

    monkeypatch.setitem(O.DEQUANT_F32, O.GGML_Q4_0, wrong)
    assert _kat_fails(kat, O.GGML_Q4_0)


@pytest.mark.parametrize("t", TYPES)
def test_matmul_reference_and_f16_operands_brute_force(t):
    # matmul_reference: the reference tests' formula (fp16-rounded dequantized weights, fp32
    # accumulate); matmul_f16_operands: f16 activations times the prefill's f16 weight operands,
    # fp64 accumulate.  Each is checked against an explicit triple loop on a tiny case, so a
    # transposed operand, a dropped activation rounding or a wrong row stride fails here.
    rng = np.random.default_rng(314 + t)
    qk, _ = O.BLOCK_INFO[t]
    M, N, K = 3, 5, 2 * max(qk, 64)
    raw = O.synth_weights(t, N, K, rng)
    A = rng.standard_normal((M, K)).astype(np.float32)
    w16 = O.dequantize_f16(t, raw, N * K).astype(np.float64).reshape(N, K)
    wo = O.dequantize_f16_operands(t, raw, N * K).astype(np.float64).reshape(N, K)
    ref = np.zeros((M, N))
    refo = np.zeros((M, N))
    for m in range(M):
        for n in range(N):
            s = 0.0
            so = 0.0
            for k in range(K):
                s += float(A[m, k]) * w16[n, k]
                so += float(np.float16(A[m, k])) * wo[n, k]
            ref[m, n] = s
            refo[m, n] = so
    got = O.matmul_reference(t, A, raw, N, K).astype(np.float64)
    assert np.max(np.abs(got - ref)) <= 1e-5 * np.max(np.abs(ref))
    np.testing.assert_allclose(O.matmul_f16_operands(t, A, raw, N, K), refo, rtol=1e-12, atol=1e-12 * np.max(np.abs(refo)))


@pytest.mark.parametrize("t", [O.GGML_Q4_0, O.GGML_Q8_0])
def test_f16_operands_equal_reference_dequant_for_block_scales(t):
    # Q4_0 / Q8_0: the scale is the block's fp16 d, so code*d rounded once to f16 is exactly the
    # reference CPU dequantizer's fp16 output (fp32 code*d is exact, then one cast).
    rng = np.random.default_rng(77 + t)
    raw = O.synth_weights(t, 64, 1024, rng)
    np.testing.assert_array_equal(O.dequantize_f16_operands(t, raw, 64 * 1024),
                                  O.dequantize_f16(t, raw, 64 * 1024).astype(np.float32))


@pytest.mark.parametrize("t", [O.GGML_Q4_K, O.GGML_Q6_K])
def test_f16_operands_error_bound_and_exact_cases(t):
    # K-quants round the sub-block scale a (and the min b) to f16 before the code multiply, so
    # |w16 - w| <= |code| * ulp(a16)/2 + ulp(b16)/2 + ulp(w16)/2 against the exact weight; the
    # result equals the reference's fp32-then-fp16 weight whenever a and b are themselves f16
    # values (power-of-two d, dmin).
    rng = np.random.default_rng(91 + t)
    raw = O.synth_weights(t, 64, 1024, rng)
    n = 64 * 1024
    a, code, b = O.fields(t, raw, n)
    w = O.dequantize_f16_operands(t, raw, n).astype(np.float64)
    half_ulp = lambda x: np.spacing(np.abs(x).astype(np.float16)).astype(np.float64) / 2
    bound = np.abs(code) * half_ulp(a) + np.where(b != 0, half_ulp(b), 0.0) + half_ulp(w)
    assert np.all(np.abs(w - (a * code - b)) <= bound)
    assert np.any(w != O.dequantize_f16(t, raw, n))  # the two routes do differ on random scales
    blk = raw.reshape(-1, O.BLOCK_INFO[t][1]).copy()
    one = np.array([0.0078125], np.float16).view(np.uint8)  # 2^-7: every d*sc, dmin*m is an f16 value
    if t == O.GGML_Q4_K:
        blk[:, 0:2] = one
        blk[:, 2:4] = one
    else:
        blk[:, 208:210] = one
    raw2 = blk.reshape(-1)
    np.testing.assert_array_equal(O.dequantize_f16_operands(t, raw2, n), O.dequantize_f16(t, raw2, n).astype(np.float32))


def test_f16_operands_known_answers():
    # Hand-worked f16 values (f16 has 10 fraction bits; ulp is 2^-9 on [2, 4), 2^-5 on [32, 64),
    # 2^-4 on [64, 128)).  d = 1 + 2^-10 is an f16 value.
    d = np.float16(1.0 + 2.0 ** -10)
    # Q4_K sub-block 0: sc = 3, codes 15, no min.  d*sc = 3.0029296875 = 3 + 1.5 ulp, a tie that
    # rounds to the even neighbour 3 + 2 ulp = 3.00390625; 15 * 3.00390625 = 45.05859375 =
    # 1441.875 ulp -> 45.0625.  (The reference route rounds the exact 45.0439453125 -> 45.03125.)
    # Sub-block 1: sc = 1 (d = 1 there via a second block), dmin*m = (1 + 2^-10)*3 -> 3.00390625
    # as above; codes 5: 5 - 3.00390625 = 1.99609375 exactly.  (Reference: 5 - 3.0029296875 =
    # 1.9970703125, also an f16 value.)
    sc = np.zeros((2, 8), np.uint8)
    m = np.zeros((2, 8), np.uint8)
    q = np.zeros((2, 256), np.uint8)
    sc[0, 0] = 3
    q[0, 0:32] = 15
    sc[1, 1] = 1
    m[1, 1] = 3
    q[1, 32:64] = 5
    raw = O.pack_q4_k(np.array([d, 1.0], np.float16), np.array([0.0, d], np.float16), sc, m, q)
    w = O.dequantize_f16_operands(O.GGML_Q4_K, raw, 512)
    r = O.dequantize_f16(O.GGML_Q4_K, raw, 512)
    assert np.all(w[0:32] == 45.0625) and np.all(r[0:32] == 45.03125)
    assert np.all(w[256 + 32:256 + 64] == 1.99609375) and np.all(r[256 + 32:256 + 64] == 1.9970703125)
    # Q6_K group 0 (sub-scale 0 covers weights 0..15): sc = 3, unsigned code 63 (q = 31):
    # 31 * 3.00390625 = 93.12109375 = 1489.9375 ulp -> 93.125; sc = -3 gives -93.125.
    # (Reference: 31 * 3.0029296875 = 93.0908203125 -> 93.0625.)
    sc6 = np.zeros((1, 16), np.int8)
    sc6[0, 0] = 3
    sc6[0, 1] = -3
    u = np.full((1, 256), 32, np.uint8)
    u[0, 0:32] = 63
    raw6 = O.pack_q6_k(np.array([d], np.float16), sc6, u)
    w6 = O.dequantize_f16_operands(O.GGML_Q6_K, raw6, 256)
    r6 = O.dequantize_f16(O.GGML_Q6_K, raw6, 256)
    assert np.all(w6[0:16] == 93.125) and np.all(w6[16:32] == -93.125)
    assert np.all(r6[0:16] == 93.0625)
