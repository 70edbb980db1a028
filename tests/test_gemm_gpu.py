"""GPU parity: every registered variant against the CPU f64 oracle, through the
C ABI, on the reference's correctness shapes (bench/check-gemm.cu:83-94) and the
BASELINE configs; bit-exact checks where the arithmetic is exact."""
import os

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

import oracle as O  # noqa: E402
from ridge_amd import gemm as G  # noqa: E402

DEV = "cuda:0"

# bench/check-gemm.cu:87-94.
REFERENCE_SHAPES = [(256, 256, 64), (256, 512, 128), (512, 256, 192), (1024, 1024, 64),
                    (1024, 512, 1024), (2048, 2048, 2048)]


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    G.lib()
    yield
    torch.cuda.synchronize()


def _to_dev(bits, shape):
    return torch.from_numpy(bits.view(np.int16).reshape(shape).copy()).to(DEV).view(torch.float16)


def _bits(t):
    return t.cpu().view(torch.int16).numpy().view(np.uint16).ravel()


def _run(i, A, B, M, N, K):
    C = torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV)
    rc = G.launch(i, A, B, C, M, N, K)
    assert rc == 0, "variant %d launch returned %d" % (i, rc)
    torch.cuda.synchronize()
    return C


def test_device_fills_match_oracle_bit_exact():
    n = (1 << 20) + 37
    t = torch.empty(n, dtype=torch.float16, device=DEV)
    for seed in (0x1234 + 256, 0x55AA, 0xFFFFFFFF):
        G.fill_lcg(t, seed)
        assert np.array_equal(_bits(t), O.lcg_fill_f16(n, seed)), seed
    for seed in (1, 2, 0xDEADBEEFCAFEF00D):
        G.fill_uniform(t, seed)
        assert np.array_equal(_bits(t), O.uniform_fill_f16(n, seed)), seed


@pytest.mark.parametrize("M,N,K", REFERENCE_SHAPES)
def test_reference_shapes_all_dividing_variants(M, N, K):
    print("shape %dx%dx%d" % (M, N, K), flush=True)
    Ab = O.lcg_fill_f16(M * K, 0x1234 + M)
    Bb = O.lcg_fill_f16(K * N, 0x9ABC + N)
    A, B = _to_dev(Ab, (M, K)), _to_dev(Bb, (K, N))
    # f64 where the reference affords it (M*N*K <= 2^32, check-gemm.cu:279); for
    # larger shapes an f64 reference on a sample of 128 rows.
    rows = np.arange(M) if M * N * K <= (1 << 32) else np.linspace(0, M - 1, 128).astype(int)
    ref = O.gemm_f64(Ab.reshape(M, K)[rows].ravel(), Bb, len(rows), N, K)
    tested = 0
    for v in G.variants():
        if not v.divides(M, N, K):
            continue
        print("  variant %d %s" % (v.index, v.label()), flush=True)
        C = _run(v.index, A, B, M, N, K)
        got = O.f16_bits_to_f32(_bits(C)).reshape(M, N)[rows]
        ok, frob, mx, ne = O.passes(got, ref, _max_abs(Ab), _max_abs(Bb), K)
        assert ok, "%s on %dx%dx%d: frob %.3e maxRel %.3e norm %.3e" % (v.label(), M, N, K, frob, mx, ne)
        tested += 1
    assert tested > 0


def _exact_case(M, N, K, lo, hi, seed):
    """Integer-valued halves whose products and partial sums are exact in FP32:
    the kernel's FP32 result is exact, so its FP16 output must equal the exact
    integer rounded once to FP16 (nearest even)."""
    rng = np.random.default_rng(seed)
    A = rng.integers(lo, hi + 1, (M, K)).astype(np.float16)
    B = rng.integers(lo, hi + 1, (K, N)).astype(np.float16)
    # Integer sums below 2^53 are exact in float64, so BLAS gives the exact value.
    exact = A.astype(np.float64) @ B.astype(np.float64)
    assert np.abs(exact).max() < 2 ** 24
    want = exact.astype(np.float16).view(np.uint16).ravel()
    return A.view(np.uint16), B.view(np.uint16), want


@pytest.mark.parametrize("M,N,K", [(256, 256, 64), (512, 256, 192), (1024, 1024, 1024)])
def test_small_integer_inputs_bit_exact_every_variant(M, N, K):
    Ab, Bb, want = _exact_case(M, N, K, -3, 3, M + N + K)
    A, B = _to_dev(Ab.ravel(), (M, K)), _to_dev(Bb.ravel(), (K, N))
    for v in G.variants():
        if not v.divides(M, N, K):
            continue
        got = _bits(_run(v.index, A, B, M, N, K))
        bad = int(np.count_nonzero(got != want))
        assert bad == 0, "%s: %d of %d outputs differ" % (v.label(), bad, M * N)


@pytest.mark.parametrize("subnormal", ["A", "B", "C"])
def test_fp16_subnormal_operands_are_not_flushed(subnormal):
    """A or B holds FP16 subnormals (integers times 2^-24) and the other operand
    integers times 2^10; or ("C") both hold integers times 2^-12, so that most
    outputs are FP16 subnormals. Every product and sum is exact in FP32 and in
    FP16, so each variant must return the exact product. A matrix unit that
    flushed subnormal inputs, or an epilogue that flushed subnormal outputs, would
    return zeros where the reference keeps the values."""
    M, N, K = 256, 256, 128
    rng = np.random.default_rng(314)
    ai = rng.integers(-3, 4, (M, K))
    bi = rng.integers(-3, 4, (K, N))
    sa, sb = {"A": (2.0 ** -24, 2.0 ** 10), "B": (2.0 ** 10, 2.0 ** -24), "C": (2.0 ** -12, 2.0 ** -12)}[subnormal]
    A16, B16 = (ai * sa).astype(np.float16), (bi * sb).astype(np.float16)
    exact = (ai @ bi) * (sa * sb)
    want = exact.astype(np.float16)
    assert np.array_equal(want.astype(np.float64), exact) and np.any(want != 0)
    tiny = {"A": A16, "B": B16, "C": want}[subnormal]
    sub = (tiny != 0) & (np.abs(tiny.astype(np.float64)) < 2.0 ** -14)
    assert (np.all(sub == (tiny != 0)) if subnormal != "C" else sub.mean() > 0.5)
    A = _to_dev(A16.view(np.uint16).ravel(), (M, K))
    B = _to_dev(B16.view(np.uint16).ravel(), (K, N))
    want_bits = want.view(np.uint16).ravel()
    for v in G.variants():
        assert v.divides(M, N, K)
        got = _bits(_run(v.index, A, B, M, N, K))
        bad = int(np.count_nonzero(got != want_bits))
        assert bad == 0, "%s, subnormal %s: %d of %d outputs differ" % (v.label(), subnormal, bad, M * N)


def test_python_gemm_on_offset_views():
    """gemm() on contiguous views that start inside a larger buffer: a 16-byte
    aligned start gives the same bits as a fresh tensor; a start 2 bytes off is
    refused by the launcher (hipErrorInvalidValue) and raised, never launched."""
    M, N, K = 256, 256, 128
    Ab, Bb, want = _exact_case(M, N, K, -3, 3, 99)
    A = _to_dev(Ab.ravel(), (M, K))
    B = _to_dev(Bb.ravel(), (K, N))
    idx = G.find_variant(256, 256, 32, 128, 64, 3, 4)
    for offset, ok in ((8, True), (1, False)):
        buf = torch.zeros(M * K + 64, dtype=torch.float16, device=DEV)
        view = buf[offset:offset + M * K].view(M, K)
        view.copy_(A)
        if ok:
            C = G.gemm(view, B, idx)
            torch.cuda.synchronize()
            assert np.array_equal(_bits(C), want)
        else:
            with pytest.raises(G.RidgeGemmError, match="hipError 1"):
                G.gemm(view, B, idx)


def test_inf_nan_and_overflow_follow_ieee():
    """Special values, every variant. One +inf in A (row 5, k 7) and one NaN in B
    (k 9, column 11) over small integers: column 11 is NaN; the rest of row 5 is
    +inf or -inf with the sign of B[7, j], or NaN where B[7, j] = 0 (inf x 0);
    every other output is the exact integer. A = B = 16 with K = 256 sums to
    65536, which rounds to +inf in FP16."""
    M, N, K = 256, 256, 128
    rng = np.random.default_rng(2718)
    ai = rng.integers(-3, 4, (M, K)).astype(np.float64)
    bi = rng.integers(-3, 4, (K, N)).astype(np.float64)
    finite = ai @ bi
    a16, b16 = ai.astype(np.float16), bi.astype(np.float16)
    a16[5, 7] = np.inf
    b16[9, 11] = np.nan
    want = finite.astype(np.float16)
    want[5, :] = np.where(bi[7] > 0, np.inf, np.where(bi[7] < 0, -np.inf, np.nan))
    want[:, 11] = np.nan
    A = _to_dev(a16.view(np.uint16).ravel(), (M, K))
    B = _to_dev(b16.view(np.uint16).ravel(), (K, N))
    Kb = 256
    big = torch.full((M, Kb), 16.0, dtype=torch.float16, device=DEV)
    bigB = torch.full((Kb, N), 16.0, dtype=torch.float16, device=DEV)
    for v in G.variants():
        got = _bits(_run(v.index, A, B, M, N, K)).view(np.float16).reshape(M, N)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan), "%s: NaN positions differ" % v.label()
        assert np.array_equal(got[~nan].view(np.uint16), want[~nan].view(np.uint16)), (
            "%s: %d finite or infinite outputs differ" % (v.label(), int(np.count_nonzero(got[~nan] != want[~nan]))))
        over = _bits(_run(v.index, big, bigB, M, N, Kb)).view(np.float16)
        assert np.all(np.isposinf(over)), "%s: 65536 did not round to +inf" % v.label()


@pytest.mark.parametrize("key", [(256, 256, 32, 128, 64, 3, 4), (256, 256, 32, 128, 64, 4, 4)])
def test_headline_4096_exact_integers_and_identity(key):
    """The bench's default variant (s3 g4) and its s4 neighbour at the headline shape."""
    M = N = K = 4096
    best = G.find_variant(*key)
    assert best >= 0
    Ab, Bb, want = _exact_case(M, N, K, -2, 2, 4096)
    A, B = _to_dev(Ab.ravel(), (M, K)), _to_dev(Bb.ravel(), (K, N))
    got = _bits(_run(best, A, B, M, N, K))
    assert np.array_equal(got, want)
    # A = I gives C = B exactly (one exact product per output).
    eye = torch.eye(M, dtype=torch.float16, device=DEV)
    Bu = torch.empty((K, N), dtype=torch.float16, device=DEV)
    G.fill_uniform(Bu, 9)
    C = _run(best, eye, Bu, M, N, K)
    assert torch.equal(C.view(torch.int16), Bu.view(torch.int16))


@pytest.mark.parametrize("M,N,K", [(8192, 8192, 128), (16384, 128, 8192)])
def test_baseline_small_k_and_tall_skinny_exact_every_variant(M, N, K):
    """The two HBM-bound BASELINE configs at full size, every variant that divides
    them (the persistent rows among them), on integers in [-2, 2]: every partial
    sum is exact in FP32 (|C| <= 4K <= 32768), so the FP16 output must equal the
    exact product rounded once, bit for bit."""
    Ab, Bb, want = _exact_case(M, N, K, -2, 2, M ^ (N << 4) ^ K)
    A, B = _to_dev(Ab.ravel(), (M, K)), _to_dev(Bb.ravel(), (K, N))
    rows = [v for v in G.variants() if v.divides(M, N, K)]
    assert any(v.schedule == 2 for v in rows)
    for v in rows:
        print("  %s %dx%dx%d" % (v.label(), M, N, K), flush=True)
        got = _bits(_run(v.index, A, B, M, N, K))
        bad = int(np.count_nonzero(got != want))
        assert bad == 0, "%s: %d of %d outputs differ" % (v.label(), bad, M * N)


def _random_shapes(n, seed):
    """Seeded shapes every row divides (M, N multiples of 256, K of 128) whose
    grids are rarely a multiple of 8 or of the rows' GroupM: partial groups,
    uneven XCD shares and single-tile-row grids."""
    rng = np.random.default_rng(seed)
    return [(256 * int(rng.integers(1, 9)), 256 * int(rng.integers(1, 9)), 128 * int(rng.integers(1, 17)))
            for _ in range(n)]


# Six shapes by default; RIDGE_RANDOM_SHAPES=n draws n (the first six are the same).
RANDOM_SHAPES = int(os.environ.get("RIDGE_RANDOM_SHAPES", "6"))


@pytest.mark.parametrize("M,N,K", _random_shapes(RANDOM_SHAPES, 20261202))
def test_random_divisible_shapes_exact_every_variant(M, N, K):
    """Every row of the table on seeded odd-sized grids, small-integer inputs:
    the FP16 output equals the exact product rounded once, and no output is
    left unwritten (C starts as NaN)."""
    Ab, Bb, want = _exact_case(M, N, K, -3, 3, M * 31 + N * 7 + K)
    A, B = _to_dev(Ab.ravel(), (M, K)), _to_dev(Bb.ravel(), (K, N))
    rows = [v for v in G.variants() if v.divides(M, N, K)]
    assert len(rows) == G.num_variants()
    for v in rows:
        got = _bits(_run(v.index, A, B, M, N, K))
        bad = int(np.count_nonzero(got != want))
        assert bad == 0, "%s on %dx%dx%d: %d of %d outputs differ" % (v.label(), M, N, K, bad, M * N)


# Random-data twin of the test above: 3 shapes by default, RIDGE_RANDOM_UNIFORM_SHAPES=n
# draws n (another seed).
RANDOM_UNIFORM_SHAPES = int(os.environ.get("RIDGE_RANDOM_UNIFORM_SHAPES", "3"))


@pytest.mark.parametrize("M,N,K", _random_shapes(RANDOM_UNIFORM_SHAPES, 20261203))
def test_random_divisible_shapes_uniform_inputs_every_variant(M, N, K):
    """Every row of the table on seeded odd-sized grids with U[-1,1) inputs,
    against the f64 oracle under the reference's gates and the FP16-output gate
    (every element within FP32 accumulation plus one rounding). All rows of C up
    to 2^30 multiply-adds, 128 evenly spaced rows beyond."""
    A = torch.empty((M, K), dtype=torch.float16, device=DEV)
    B = torch.empty((K, N), dtype=torch.float16, device=DEV)
    G.fill_uniform(A, M * 131 + N * 17 + K)
    G.fill_uniform(B, M * 7 + N * 131 + K + 1)
    Ab, Bb = _bits(A), _bits(B)
    rows = np.arange(M) if M * N * K <= 2 ** 30 else np.linspace(0, M - 1, 128).astype(int)
    Arows = Ab.reshape(M, K)[rows].ravel()
    ref = O.gemm_f64(Arows, Bb, len(rows), N, K)
    absprod = O.gemm_f64(O.abs_bits(Arows), O.abs_bits(Bb), len(rows), N, K)
    max_a, max_b = _max_abs(Ab), _max_abs(Bb)
    worst_row = (0.0, 0.0, "")
    for v in G.variants():
        assert v.divides(M, N, K)
        got = O.f16_bits_to_f32(_bits(_run(v.index, A, B, M, N, K))).reshape(M, N)[rows]
        ok, frob, mx, ne = O.passes(got, ref, max_a, max_b, K)
        assert ok, "%s on %dx%dx%d: frob %.3e maxRel %.3e norm %.3e" % (v.label(), M, N, K, frob, mx, ne)
        ok, frob, worst = O.passes_fp16(got, ref, absprod, K)
        assert ok, "%s on %dx%dx%d: FP16-output gate frob %.3e, worst element at %.2f of its bound" % (
            v.label(), M, N, K, frob, worst)
        worst_row = max(worst_row, (worst, frob, v.label()))
    print("  uniform %dx%dx%d, %d rows checked: worst element at %.3f of its bound (%s), frob %.3e" % (
        M, N, K, len(rows), worst_row[0], worst_row[2], worst_row[1]), flush=True)


def _persistent_edge_shapes(v):
    """Shapes that drive the persistent schedule's control flow to its edges."""
    BM, BN, BK, S = v.BM, v.BN, v.BK, v.stages
    return [
        (BM, BN, BK),                        # one output tile, one K tile
        (BM, BN, BK * max(1, S - 2)),         # fewer K tiles than the ring prefetches
        (2 * BM, 3 * BN, 5 * BK),             # six tiles: a grid far below one per CU
        (4096, 4096, BK),                     # many tiles per workgroup, one K tile each
        (37 * BM, 11 * BN, 3 * BK),           # 407 tiles: some workgroups walk one more
        (800 * BM, 3 * BN, 2 * BK),           # 2400 tiles: 9-10 per workgroup
        (2048, 1024, (2 * S + 1) * BK),       # K tiles wrap the ring more than twice
    ]


def test_persistent_rows_edge_shapes_bit_exact():
    """Every persistent (store-behind) row on its edge shapes, small-integer
    inputs: the FP16 output equals the exact product rounded once, and no output
    is left unwritten (C starts as NaN, which would not compare equal)."""
    rows = [v for v in G.variants() if v.schedule == 2]
    assert rows
    for v in rows:
        for (M, N, K) in _persistent_edge_shapes(v):
            assert v.divides(M, N, K), (v.label(), M, N, K)
            print("  %s %dx%dx%d" % (v.label(), M, N, K), flush=True)
            Ab, Bb, want = _exact_case(M, N, K, -3, 3, M + 7 * N + 13 * K)
            A, B = _to_dev(Ab.ravel(), (M, K)), _to_dev(Bb.ravel(), (K, N))
            got = _bits(_run(v.index, A, B, M, N, K))
            bad = int(np.count_nonzero(got != want))
            assert bad == 0, "%s on %dx%dx%d: %d of %d outputs differ" % (v.label(), M, N, K, bad, M * N)


# The launcher admits a shape only while its 32-bit in-kernel byte offsets cannot
# overflow (BM * K and BK * N below 2^31). At the largest K it admits for 256-row
# tiles, an A tile's last row starts (BM - 1) * K * 2 bytes, just under 2^32, into
# the tile's row panel.
K_LIMIT_BM256 = (0x7FFFFFFF // 256) // 64 * 64


def _offset_limit_case(M, N, K):
    """A[i, k] = 1 where k = i (mod 4099) and B[k, j] = 1 where k = j (mod 3), else
    0. C[i, j] counts the k < K in both classes: with k = i + 4099 t and
    4099 = 1 (mod 3), those are the t < T_i = ceil((K - i) / 4099) with
    t = j - i (mod 3). Every count is near 682, exact in FP16, and a wrapped
    offset reads another row's or another K slice's classes."""
    k = torch.arange(K, device=DEV, dtype=torch.int32)
    A = (k[None, :] % 4099 == torch.arange(M, device=DEV, dtype=torch.int32)[:, None]).to(torch.float16)
    rows = (torch.arange(3, device=DEV)[:, None] - torch.arange(N, device=DEV)[None, :]) % 3 == 0
    B = rows.to(torch.float16).index_select(0, (k % 3).long())
    del k
    i = np.arange(M)[:, None]
    j = np.arange(N)[None, :]
    T = (K - i + 4098) // 4099
    r = (j - i) % 3
    count = np.where(r < T, (T - r + 2) // 3, 0)
    return A, B, count.astype(np.float16).view(np.uint16).ravel()


def test_largest_k_the_offset_guard_admits_is_exact():
    M = N = 256
    K = K_LIMIT_BM256
    rows = [v for v in G.variants() if v.BM == 256 and v.divides(M, N, K)]
    assert rows, "no 256-row variant admits the limit shape"
    print("  K = %d, %d variants" % (K, len(rows)), flush=True)
    A, B, want = _offset_limit_case(M, N, K)
    for v in rows:
        print("  variant %d %s" % (v.index, v.label()), flush=True)
        got = _bits(_run(v.index, A, B, M, N, K))
        bad = int(np.count_nonzero(got != want))
        assert bad == 0, "%s at K = %d: %d of %d outputs differ" % (v.label(), K, bad, M * N)
    del A, B
    torch.cuda.empty_cache()


def test_largest_n_the_offset_guard_admits_is_exact_on_bk128_persistent_rows():
    """The BK = 128 persistent rows at the largest N the guard admits (BK * N just
    under 2^31, so a B tile's last row starts just under 2^32 bytes from its first),
    with two row panels and K = 2 BK, so the loaders' staggered K start reads the
    second K tile first on one panel. A[i, k] = 1 where k = i (mod BK): row i sums
    B rows i % BK and i % BK + BK. B[k, j] = 1 where k + j = 0 (mod 3), so every
    output is 0, 1 or 2 and exact, and a wrapped or misplaced offset (a shift of a
    whole K slice, or of 2^31 halves) reads another class. Checked on the device,
    every output; B is about 8.6 GB and C about 4.3 GB."""
    rows = [v for v in G.variants() if v.schedule == 2 and v.BK == 128]
    assert len(rows) == 2
    for v in rows:
        M, K = 2 * v.BM, 2 * v.BK
        N = (0x7FFFFFFF // v.BK) // v.BN * v.BN
        assert v.divides(M, N, K) and not v.divides(M, N + v.BN, K)
        print("  %s at %dx%dx%d" % (v.label(), M, N, K), flush=True)
        k = torch.arange(K, device=DEV)
        A = (k[None, :] % v.BK == torch.arange(M, device=DEV)[:, None] % v.BK).to(torch.float16)
        jm3 = torch.arange(N, device=DEV, dtype=torch.int32) % 3
        B = torch.empty((K, N), dtype=torch.float16, device=DEV)
        for kk in range(K):
            B[kk] = (jm3 == (-kk) % 3).to(torch.float16)
        C = _run(v.index, A, B, M, N, K)
        del B
        bad = 0
        for i in range(M):
            r = i % v.BK
            want = ((jm3 + r) % 3 == 0).to(torch.int32) + ((jm3 + r + v.BK) % 3 == 0).to(torch.int32)
            bad += int((C[i].to(torch.int32) != want).sum().item())
        assert bad == 0, "%s at N = %d: %d of %d outputs differ" % (v.label(), N, bad, M * N)
        del A, C, jm3
        torch.cuda.empty_cache()


@pytest.mark.parametrize("M,N,K", [(1024, 1024, 1024), (4096, 4096, 4096), (8192, 8192, 128),
                                   (16384, 128, 8192)])
def test_baseline_configs_uniform_inputs(M, N, K):
    """BASELINE.json configs with U[-1,1) inputs: every dividing variant against an
    f64 reference on sampled rows (all rows at 1024^3)."""
    print("baseline %dx%dx%d" % (M, N, K), flush=True)
    A = torch.empty((M, K), dtype=torch.float16, device=DEV)
    B = torch.empty((K, N), dtype=torch.float16, device=DEV)
    G.fill_uniform(A, 1)
    G.fill_uniform(B, 2)
    Ab, Bb = _bits(A), _bits(B)
    rows = np.arange(M) if M <= 1024 else np.linspace(0, M - 1, 64).astype(int)
    Arows = Ab.reshape(M, K)[rows].ravel()
    ref = O.gemm_f64(Arows, Bb, len(rows), N, K)
    absprod = O.gemm_f64(O.abs_bits(Arows), O.abs_bits(Bb), len(rows), N, K)
    max_a, max_b = _max_abs(Ab), _max_abs(Bb)
    for v in G.variants():
        if not v.divides(M, N, K):
            continue
        C = _run(v.index, A, B, M, N, K)
        got = O.f16_bits_to_f32(_bits(C)).reshape(M, N)[rows]
        ok, frob, mx, ne = O.passes(got, ref, max_a, max_b, K)
        assert ok, "%s on %dx%dx%d: frob %.3e maxRel %.3e norm %.3e" % (v.label(), M, N, K, frob, mx, ne)
        ok, frob, worst = O.passes_fp16(got, ref, absprod, K)
        assert ok, "%s on %dx%dx%d: FP16-output gate frob %.3e, worst element at %.2f of its bound" % (
            v.label(), M, N, K, frob, worst)


def test_headline_variant_every_output_at_4096_cubed():
    """The bench's variant at 4096^3 on U[-1,1) inputs: all 16.8 M outputs against
    the f64 oracle under the reference's gates and the FP16-output gate (every
    element within its FP32-accumulation-plus-one-rounding bound, Frobenius
    <= 1e-3)."""
    M = N = K = 4096
    idx = G.find_variant(256, 256, 32, 128, 64, 3, 4)
    assert idx >= 0
    print("headline %s every output" % G.variant(idx).label(), flush=True)
    A = torch.empty((M, K), dtype=torch.float16, device=DEV)
    B = torch.empty((K, N), dtype=torch.float16, device=DEV)
    G.fill_uniform(A, 1)
    G.fill_uniform(B, 2)
    Ab, Bb = _bits(A), _bits(B)
    got = O.f16_bits_to_f32(_bits(_run(idx, A, B, M, N, K))).reshape(M, N)
    ref = O.gemm_f64(Ab, Bb, M, N, K)
    ok, frob, mx, ne = O.passes(got, ref, _max_abs(Ab), _max_abs(Bb), K)
    assert ok, "reference gates: frob %.3e maxRel %.3e norm %.3e" % (frob, mx, ne)
    absprod = O.gemm_f64(O.abs_bits(Ab), O.abs_bits(Bb), M, N, K)
    ok, frob, worst = O.passes_fp16(got, ref, absprod, K)
    print("  frob %.3e, worst element at %.3f of its bound" % (frob, worst), flush=True)
    assert ok, "FP16-output gate: frob %.3e, worst element at %.2f of its bound" % (frob, worst)


def _max_abs(bits):
    """max |x| over FP16 bit patterns (the reference's normalisation,
    check-gemm.cu:110-135, taken from the operands actually used)."""
    return float(np.max(np.abs(O.f16_bits_to_f32(bits))))


# The best row of each BASELINE config other than the headline (whose every
# output the test above checks). The persistent rows start each output tile's K
# loop at a tile-dependent K tile and wrap, so their FP32 sums round in another
# order than the other rows'; small-integer inputs (exact sums) cannot see that.
REPORTED_ROWS = [
    ((1024, 1024, 1024), (64, 64, 64, 32, 32, 4, 8)),
    ((8192, 8192, 128), (256, 128, 32, 64, 64, 6, 4)),
    ((16384, 128, 8192), (64, 128, 128, 32, 64, 3, 8)),
]


@pytest.mark.parametrize("shape,key", REPORTED_ROWS, ids=["1024cube", "8192sq_k128", "tall_skinny"])
def test_reported_rows_every_output(shape, key):
    """Every output of the reported row on U[-1,1) inputs against the f64 oracle,
    under the reference's gates (bench/check-gemm.cu:277-322 compares the whole C)
    and the FP16-output gate (each element within FP32 accumulation plus one
    rounding)."""
    M, N, K = shape
    idx = G.find_variant(*key)
    assert idx >= 0, key
    print("reported row %s at %dx%dx%d, every output" % (G.variant(idx).label(), M, N, K), flush=True)
    A = torch.empty((M, K), dtype=torch.float16, device=DEV)
    B = torch.empty((K, N), dtype=torch.float16, device=DEV)
    G.fill_uniform(A, 1)
    G.fill_uniform(B, 2)
    Ab, Bb = _bits(A), _bits(B)
    got = O.f16_bits_to_f32(_bits(_run(idx, A, B, M, N, K))).reshape(M, N)
    del A, B
    torch.cuda.empty_cache()
    ref = O.gemm_f64(Ab, Bb, M, N, K)
    ok, frob, mx, ne = O.passes(got, ref, _max_abs(Ab), _max_abs(Bb), K)
    print("  reference gates: frob %.3e maxRel %.3e norm %.3e" % (frob, mx, ne), flush=True)
    assert ok, "reference gates: frob %.3e maxRel %.3e norm %.3e" % (frob, mx, ne)
    absprod = O.gemm_f64(O.abs_bits(Ab), O.abs_bits(Bb), M, N, K)
    ok, frob, worst = O.passes_fp16(got, ref, absprod, K)
    print("  FP16-output gate over %d outputs: frob %.3e, worst element at %.3f of its bound"
          % (M * N, frob, worst), flush=True)
    assert ok, "FP16-output gate: frob %.3e, worst element at %.2f of its bound" % (frob, worst)


# Row split: the 256x256 s3 row on the rows of whole rounds of tiles and another
# row on the rest (two launches, ridge_gemm_launch_split).
SPLIT_BODY = (256, 256, 32, 128, 64, 3, 4)
SPLIT_TAILS = [(128, 128, 64, 64, 64, 4, 8), (256, 128, 64, 64, 64, 3, 8), (64, 64, 64, 32, 32, 4, 8),
               (128, 64, 128, 64, 32, 3, 8)]


def test_row_split_small_integers_bit_exact_and_nothing_outside_c():
    """6144 x 3072 x 256 on integers in [-3, 3] (exact sums): the split gives the
    exact product rounded once, bit for bit, with the planner's split (5376 body
    rows on 256 CUs) for four tails, a 64-row tail and a one-panel body; C is a
    view of a buffer with 64 guard rows after it, which keep their bits; one case
    runs on a side stream."""
    M, N, K = 6144, 3072, 256
    body = G.find_variant(*SPLIT_BODY)
    assert body >= 0 and G.split_rows(body, M, N, K, 256) == 5376
    Ab, Bb, want = _exact_case(M, N, K, -3, 3, 6144 + 3072 + 256)
    A, B = _to_dev(Ab.ravel(), (M, K)), _to_dev(Bb.ravel(), (K, N))
    cases = [(G.find_variant(*t), 5376) for t in SPLIT_TAILS]
    cases += [(G.find_variant(64, 64, 64, 32, 32, 4, 8), M - 256), (G.find_variant(*SPLIT_TAILS[0]), 256)]
    side = torch.cuda.Stream()
    for n, (tail, rows) in enumerate(cases):
        assert tail >= 0
        on_side = n == 1
        print("split %s | %s at %d rows%s" % (G.variant(body).label(), G.variant(tail).label(), rows,
                                              " (side stream)" if on_side else ""), flush=True)
        buf = torch.full((M + 64, N), float("nan"), dtype=torch.float16, device=DEV)
        C = buf[:M]
        if on_side:
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                rc = G.launch_split(body, tail, rows, A, B, C, M, N, K, stream=side)
            side.synchronize()
        else:
            rc = G.launch_split(body, tail, rows, A, B, C, M, N, K)
            torch.cuda.synchronize()
        assert rc == 0
        got = _bits(C)
        bad = int(np.count_nonzero(got != want))
        assert bad == 0, "%d of %d outputs differ (first at row %d)" % (
            bad, M * N, int(np.flatnonzero(got != want)[0]) // N if bad else -1)
        guard = _bits(buf[M:])
        assert np.all(guard == guard[0]) and np.isnan(O.f16_bits_to_f32(guard[:1]))[0], "guard rows written"


def test_row_split_halves_equal_their_own_launches_and_the_oracle():
    """12288 x 3072 x 3072 on U[-1,1) inputs with the planner's split for this
    device: the body rows equal the body row's single launch over the whole shape
    bit for bit (a tile's sum does not depend on the grid), the tail rows equal
    the tail row launched alone on A's last rows, and every tail row plus 128
    body rows pass the FP16-output gate against the f64 oracle. Tails: a
    one-tile-per-workgroup row and a persistent row (whose K loop starts at a
    tile-dependent K tile, so it is compared with its own launch)."""
    M, N, K = 12288, 3072, 3072
    body = G.find_variant(*SPLIT_BODY)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    rows = G.split_rows(body, M, N, K, cus)
    print("device CUs %d, body rows %d" % (cus, rows), flush=True)
    if not 0 < rows < M:
        pytest.skip("no split of %dx%dx%d on %d CUs" % (M, N, K, cus))
    A = torch.empty((M, K), dtype=torch.float16, device=DEV)
    B = torch.empty((K, N), dtype=torch.float16, device=DEV)
    G.fill_uniform(A, 11)
    G.fill_uniform(B, 12)
    single = _bits(_run(body, A, B, M, N, K)).reshape(M, N)
    Ab, Bb = _bits(A), _bits(B)
    sample = np.concatenate([np.linspace(0, rows - 1, 128).astype(int), np.arange(rows, M)])
    Abs = Ab.reshape(M, K)[sample].ravel()
    ref = O.gemm_f64(Abs, Bb, len(sample), N, K)
    absprod = O.gemm_f64(O.abs_bits(Abs), O.abs_bits(Bb), len(sample), N, K)
    for key in ((256, 128, 64, 64, 64, 3, 8), (256, 128, 32, 64, 64, 6, 4)):
        tail = G.find_variant(*key)
        print("  tail %s, %d rows" % (G.variant(tail).label(), M - rows), flush=True)
        C = torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV)
        assert G.launch_split(body, tail, rows, A, B, C, M, N, K) == 0
        torch.cuda.synchronize()
        got = _bits(C).reshape(M, N)
        assert np.array_equal(got[:rows], single[:rows]), "body rows differ from the single launch"
        alone = _bits(_run(tail, A[rows:], B, M - rows, N, K)).reshape(M - rows, N)
        assert np.array_equal(got[rows:], alone), "tail rows differ from the tail row's own launch"
        ok, frob, worst = O.passes_fp16(O.f16_bits_to_f32(got[sample].ravel()).reshape(len(sample), N),
                                        ref, absprod, K)
        print("  FP16-output gate on %d rows: frob %.3e, worst element at %.3f of its bound"
              % (len(sample), frob, worst), flush=True)
        assert ok, "FP16-output gate: frob %.3e, worst element at %.2f of its bound" % (frob, worst)


def test_hipblaslt_comparator_agrees_with_oracle():
    M, N, K = 512, 768, 256
    Ab = O.lcg_fill_f16(M * K, 5)
    Bb = O.lcg_fill_f16(K * N, 6)
    A, B = _to_dev(Ab, (M, K)), _to_dev(Bb, (K, N))
    ref = O.gemm_f64(Ab, Bb, M, N, K)
    blas = G.BlasLt()
    C16 = torch.empty((M, N), dtype=torch.float16, device=DEV)
    C32 = torch.empty((M, N), dtype=torch.float32, device=DEV)
    blas.gemm(A, B, C16, M, N, K)
    blas.gemm(A, B, C32, M, N, K, c_is_f32=True)
    torch.cuda.synchronize()
    assert O.passes(O.f16_bits_to_f32(_bits(C16)), ref, 0.5, 0.5, K)[0]
    assert O.passes(C32.cpu().numpy(), ref, 0.5, 0.5, K)[0]
    blas.close()


def _registered_sweep_shapes():
    import os
    path = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "data", "sweep",
                        "mi355x-registered.csv")
    shapes = []
    with open(path) as f:
        for line in f:
            if line.startswith("#") or not line.strip():
                continue
            m, n, k = (int(x) for x in line.split(",")[:3])
            shapes.append((m, n, k))
    return shapes


@pytest.mark.parametrize("M,N,K", _registered_sweep_shapes())
def test_registered_sweep_shapes_every_variant(M, N, K):
    """Every registered sweep shape x every variant (the measured cross product):
    no output left unwritten (C starts as NaN) and 16 rows spread over M, first and
    last included, within the reference's tolerances of the f64 oracle."""
    print("sweep shape %dx%dx%d" % (M, N, K), flush=True)
    A = torch.empty((M, K), dtype=torch.float16, device=DEV)
    B = torch.empty((K, N), dtype=torch.float16, device=DEV)
    G.fill_uniform(A, 11)
    G.fill_uniform(B, 12)
    rows = np.linspace(0, M - 1, 16).astype(int)
    Ab = A[torch.from_numpy(rows).to(DEV)].cpu().view(torch.int16).numpy().view(np.uint16).ravel()
    Bb = _bits(B)
    ref = O.gemm_f64(Ab, Bb, len(rows), N, K)
    absprod = O.gemm_f64(O.abs_bits(Ab), O.abs_bits(Bb), len(rows), N, K)
    max_a, max_b = _max_abs(_bits(A)), _max_abs(Bb)
    idx = torch.from_numpy(rows).to(DEV)
    for v in G.variants():
        assert v.divides(M, N, K), v.label()
        C = _run(v.index, A, B, M, N, K)
        assert not bool(torch.isnan(C).any()), "%s left outputs unwritten at %dx%dx%d" % (v.label(), M, N, K)
        got = O.f16_bits_to_f32(C[idx].cpu().view(torch.int16).numpy().view(np.uint16)).reshape(len(rows), N)
        ok, frob, mx, ne = O.passes(got, ref, max_a, max_b, K)
        assert ok, "%s on %dx%dx%d: frob %.3e maxRel %.3e norm %.3e" % (v.label(), M, N, K, frob, mx, ne)
        ok, frob, worst = O.passes_fp16(got, ref, absprod, K)
        assert ok, "%s on %dx%dx%d: FP16-output gate frob %.3e, worst element at %.2f of its bound" % (
            v.label(), M, N, K, frob, worst)
        del C


def test_concurrent_host_threads_launch_persistent_rows():
    """Four host threads, each with its own stream and buffers, launch a persistent
    row 20 times at once (the first launches fill the per-device grid cache
    concurrently); every result is the exact product of small integers."""
    import threading
    v = [w for w in G.variants() if w.schedule == 2][0]
    M, N, K = 8 * v.BM, 4 * v.BN, 4 * v.BK
    Ab, Bb, want = _exact_case(M, N, K, -3, 3, 77)
    jobs = []
    for t in range(4):
        A, B = _to_dev(Ab.ravel(), (M, K)), _to_dev(Bb.ravel(), (K, N))
        C = torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV)
        jobs.append((A, B, C, torch.cuda.Stream()))
    torch.cuda.synchronize()
    errors = []

    def work(A, B, C, s):
        for _ in range(20):
            rc = G.launch(v.index, A, B, C, M, N, K, s)
            if rc != 0:
                errors.append(rc)
                return

    threads = [threading.Thread(target=work, args=j) for j in jobs]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    torch.cuda.synchronize()
    assert not errors
    for (_, _, C, _) in jobs:
        assert np.array_equal(_bits(C), want)


def test_launches_replay_from_a_captured_hip_graph():
    """The launcher allocates nothing and never synchronises, so a caller can
    capture kernel-table launches into a HIP graph and replay them (the way a
    serving loop removes per-launch host cost). One row of each schedule is
    captured on one stream; three replays, with the inputs refilled eagerly
    between them, must each equal eager launches bit for bit."""
    M, N, K = 1024, 1024, 1024
    picks = []
    for sched in (0, 1, 2):
        cand = [v for v in G.variants() if v.schedule == sched and v.divides(M, N, K)]
        assert cand, "no row of schedule %d divides %dx%dx%d" % (sched, M, N, K)
        picks.append(cand[0])
    A = torch.empty((M, K), dtype=torch.float16, device=DEV)
    B = torch.empty((K, N), dtype=torch.float16, device=DEV)
    G.fill_uniform(A, 5)
    G.fill_uniform(B, 6)
    Cg = [torch.full((M, N), float("nan"), dtype=torch.float16, device=DEV) for _ in picks]
    for v in picks:  # eager first launches (the persistent launcher caches its grid)
        _run(v.index, A, B, M, N, K)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for v, C in zip(picks, Cg):
            assert G.launch(v.index, A, B, C, M, N, K) == 0
    torch.cuda.synchronize()
    for rep in range(3):
        print("replay %d" % rep, flush=True)
        G.fill_uniform(A, 100 + rep)
        G.fill_uniform(B, 200 + rep)
        graph.replay()
        torch.cuda.synchronize()
        for v, C in zip(picks, Cg):
            eager = _run(v.index, A, B, M, N, K)
            assert torch.equal(C, eager), "%s replay %d differs from the eager launch" % (v.label(), rep)
