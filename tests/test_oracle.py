"""Pins the CPU oracle against the reference's known answers, independent
implementations and closed forms (no GPU)."""
import json
import os

import numpy as np
import pytest

import oracle as O

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def _fills():
    with open(os.path.join(GOLD, "fills.json")) as f:
        return json.load(f)


def test_f16_to_f32_all_patterns_match_numpy():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ours = O.f16_bits_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rounding_matches_numpy():
    rng = np.random.default_rng(7)
    xs = np.concatenate([
        rng.uniform(-1, 1, 20000).astype(np.float32),
        (rng.standard_normal(20000) * 1e4).astype(np.float32),
        (rng.uniform(-1, 1, 20000) * 2.0 ** -14).astype(np.float32),   # subnormal range
        (rng.uniform(-1, 1, 5000) * 2.0 ** -25).astype(np.float32),    # flush / tie region
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e6, -1e6, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 2.0 ** -14 * (1 - 2.0 ** -12)], dtype=np.float32),
    ])
    # Exact halfway cases between neighbouring halves, where ties-to-even decides.
    h = np.arange(0x0001, 0x7BFF, 37, dtype=np.uint16)
    lo = h.view(np.float16).astype(np.float64)
    hi = (h + 1).view(np.float16).astype(np.float64)
    xs = np.concatenate([xs, ((lo + hi) / 2).astype(np.float32)])
    ours = np.array([O.f32_to_f16(float(x)) for x in xs], dtype=np.uint16)
    ref = xs.astype(np.float16).view(np.uint16)
    assert np.array_equal(ours, ref)


def test_lcg_fill_hand_arithmetic():
    # seed 0x1234 + 256 = 4916: s1 = 4916 * 1664525 + 1013904223 = 9196709123,
    # minus 2 * 2^32 = 606774531; (s1 >> 16) & 0x7fff = 9258;
    # 9258 / 32767 - 0.5 = -0.21744... -> nearest half -0.2174 (0xB2F5).
    bits = O.lcg_fill_f16(1, 4916)
    assert float(np.float16(bits.view(np.float16)[0])) == pytest.approx(9258 / 32767 - 0.5, abs=2.0 ** -12)
    assert bits[0] == np.array([np.float32(9258) / np.float32(32767) - np.float32(0.5)],
                               dtype=np.float32).astype(np.float16).view(np.uint16)[0]


def test_lcg_fill_matches_golden():
    for seed, d in _fills()["lcg"].items():
        got = O.lcg_fill_f16(16, int(seed))
        assert got.tolist() == d["half_bits"], seed


def test_lcg_fill_range_and_mean():
    v = O.lcg_fill_f16(1 << 16, 0x9ABC).view(np.float16).astype(np.float64)
    assert v.min() >= -0.5 and v.max() <= 0.5
    assert abs(v.mean()) < 0.01


def test_splitmix64_published_vector():
    # Vigna's splitmix64.c seeded with 1234567: the first five outputs.
    want = [6457827717110365317, 3203168211198807973, 9817491932198370423,
            4593380528125082431, 16408922859458223821]
    assert [O.splitmix64_at(1234567, i) for i in range(5)] == want
    assert [int(x) for x in _fills()["splitmix64"]["1234567"]] == want


def test_uniform_fill_matches_golden_and_range():
    for seed, bits in _fills()["uniform"].items():
        assert O.uniform_fill_f16(16, int(seed)).tolist() == bits
    v = O.uniform_fill_f16(1 << 16, 3).view(np.float16).astype(np.float64)
    assert v.min() >= -1.0 and v.max() <= 1.0
    assert abs(v.mean()) < 0.02 and v.std() == pytest.approx(1 / np.sqrt(3), rel=0.02)


def _halves(a):
    return np.asarray(a, dtype=np.float16).view(np.uint16)


def test_gemm_identity_returns_b_exactly():
    n, N = 64, 48
    eye = _halves(np.eye(n))
    B = O.uniform_fill_f16(n * N, 11)
    C = O.gemm_f64(eye, B, n, N, n)
    assert np.array_equal(C, B.view(np.float16).astype(np.float64).reshape(n, N))


def test_gemm_one_hot_selects_single_product():
    M, N, K = 8, 8, 32
    A = np.zeros((M, K), np.float16)
    B = np.zeros((K, N), np.float16)
    A[3, 17] = 1.5
    B[17, 5] = -0.25
    C = O.gemm_f64(_halves(A), _halves(B), M, N, K)
    want = np.zeros((M, N))
    want[3, 5] = -0.375
    assert np.array_equal(C, want)


def test_gemm_small_integers_exact_and_naive_equals_parallel():
    rng = np.random.default_rng(3)
    M, N, K = 37, 29, 130
    A = rng.integers(-8, 9, (M, K))
    B = rng.integers(-8, 9, (K, N))
    Ab, Bb = _halves(A), _halves(B)
    C1 = O.gemm_f64(Ab, Bb, M, N, K, naive=True)
    C2 = O.gemm_f64(Ab, Bb, M, N, K, threads=4)
    assert np.array_equal(C1, (A @ B).astype(np.float64))
    assert np.array_equal(C1, C2)


def test_gemm_random_halves_against_numpy_float64():
    M, N, K = 96, 80, 256
    Ab = O.lcg_fill_f16(M * K, 0x1234 + M)
    Bb = O.lcg_fill_f16(K * N, 0x9ABC + N)
    C = O.gemm_f64(Ab, Bb, M, N, K, naive=True)
    ref = Ab.view(np.float16).astype(np.float64).reshape(M, K) @ Bb.view(np.float16).astype(np.float64).reshape(K, N)
    assert np.allclose(C, ref, rtol=0, atol=1e-12)
    # A transposed operand (a plausible indexing slip) is far outside tolerance.
    wrong = Ab.view(np.float16).astype(np.float64).reshape(M, K)[:, ::-1] @ \
        Bb.view(np.float16).astype(np.float64).reshape(K, N)
    assert not O.passes(wrong.astype(np.float32), C, 0.5, 0.5, K)[0]


def test_error_stats_reference_selftest_vectors():
    # bench/check-gemm.cu:203-259: an exact copy passes, and three corruptions
    # shaped like real kernel bugs must each be rejected by at least one criterion.
    ref = O.selftest_ref(4096)
    assert ref[0] == pytest.approx(((1013904223 + 0xC0FFEE * 1664525) % 2 ** 32 >> 16 & 0x7FFF) / 32767 - 0.5)

    def rejected(bad):
        frob, mx = O.error_stats(bad.astype(np.float32), ref)
        return frob > O.REL_FROB_TOL or mx > O.MAX_ELEM_TOL

    assert not rejected(ref.copy())
    assert rejected(ref * 1.05)
    tail = ref.copy()
    tail[int(4096 * 0.97):] *= 0.5
    assert rejected(tail)
    one = ref.copy()
    one[4096 // 3] += 1.0
    assert rejected(one)


def test_error_stats_closed_forms():
    ref = np.linspace(-3, 5, 1001)
    for e in (0.0, 1e-3, 0.25):
        frob, mx = O.error_stats((ref * (1 + e)).astype(np.float64).astype(np.float32), ref)
        assert frob == pytest.approx(e, abs=1e-7)
        assert mx == pytest.approx(e, abs=1e-7)
    # zero reference conventions (check-gemm.cu:131-132)
    z = np.zeros(10)
    assert O.error_stats(z.astype(np.float32), z) == (0.0, 0.0)
    assert O.error_stats(np.ones(10, np.float32), z) == (1.0, 1.0)


def test_normalized_max_err():
    ref = np.array([0.0, 1.0, -2.0])
    got = np.array([0.0, 1.5, -2.0], np.float32)
    assert O.normalized_max_err(got, ref, 1.0, 0.5, 100) == pytest.approx(0.5 / 50.0)


def _fp16_accumulated(A, B):
    """C = A B with every partial sum rounded to FP16 (an FP16 accumulator),
    products formed in FP32: the mistake the FP16-output gate must catch."""
    acc = np.zeros((A.shape[0], B.shape[1]), dtype=np.float16)
    for k in range(A.shape[1]):
        acc = (acc.astype(np.float32) + np.outer(A[:, k], B[k, :]).astype(np.float32)).astype(np.float16)
    return acc.astype(np.float32)


@pytest.mark.parametrize("K", [128, 256])
def test_fp16_output_gate_rejects_fp16_accumulation_the_reference_gate_accepts(K):
    """U[-1,1) operands: an FP32-accumulated, once-rounded FP16 C meets the
    FP16-output gate; a C accumulated in FP16 fails it, although the reference's
    three gates (1e-2 Frobenius, 5e-2 max element, 1e-3 normalised) accept it."""
    M, N = 96, 80
    Ab = O.uniform_fill_f16(M * K, 21).reshape(M, K)
    Bb = O.uniform_fill_f16(K * N, 22).reshape(K, N)
    A = O.f16_bits_to_f32(Ab).reshape(M, K)
    B = O.f16_bits_to_f32(Bb).reshape(K, N)
    ref = O.gemm_f64(Ab, Bb, M, N, K)
    absprod = O.gemm_f64(O.abs_bits(Ab), O.abs_bits(Bb), M, N, K)
    good = (A.astype(np.float32) @ B.astype(np.float32)).astype(np.float16).astype(np.float32)
    ok, frob, worst = O.passes_fp16(good, ref, absprod, K)
    assert ok and frob < 4e-4 and worst < 1.0
    bad = _fp16_accumulated(A, B)
    assert O.passes(bad, ref, 1.0, 1.0, K)[0]          # the reference's gates accept it
    ok, frob, worst = O.passes_fp16(bad, ref, absprod, K)
    assert not ok and frob > 1e-3 and worst > 1.0       # the FP16-output gate does not


def test_fp16_output_bound_closed_forms():
    """The bound is 2^-11 |ref| + (1 + 2^-11) gamma + 2^-25 with gamma =
    1.001 K 2^-24 |A||B|; a result off by one FP16 half-ulp of ref passes, one
    off by two full ulps of a normal ref fails."""
    ref = np.array([[1.0, -3.0, 1000.0]])
    absprod = np.zeros_like(ref)
    b = O.fp16_output_bound(ref, absprod, 1)
    assert np.allclose(b, 2.0 ** -11 * np.abs(ref) + 2.0 ** -25)
    half_ulp = np.array([[2.0 ** -11, 2.0 ** -10, 0.25]])  # half an FP16 ulp at 1, 3 and 1000
    assert O.passes_fp16(ref + half_ulp, ref, absprod, 1)[2] <= 1.0
    two_ulp = np.array([[2.0 ** -9, 0.0, 0.0]])
    assert O.passes_fp16(ref + two_ulp, ref, absprod, 1)[2] > 1.0
    g = O.fp16_output_bound(np.zeros((1, 1)), np.array([[4.0]]), 1024)
    assert g[0, 0] == pytest.approx((1 + 2.0 ** -11) * 1.001 * 1024 * 2.0 ** -24 * 4.0 + 2.0 ** -25)
