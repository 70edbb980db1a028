"""ctypes binding of the CPU oracle (oracle/ridge_oracle.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, by __graft_entry__.smoke() as the
checker, and by bench.py's cpu_baseline leg. The product never imports it.
"""

import ctypes
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError("%s missing: run `make -C oracle`" % LIB_PATH)
    L = ctypes.CDLL(LIB_PATH)
    P = np.ctypeslib.ndpointer
    u16 = P(dtype=np.uint16, flags="C_CONTIGUOUS")
    f32 = P(dtype=np.float32, flags="C_CONTIGUOUS")
    f64 = P(dtype=np.float64, flags="C_CONTIGUOUS")
    sz = ctypes.c_size_t
    L.oracle_f32_to_f16.restype = ctypes.c_uint16
    L.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    L.oracle_f16_to_f32.restype = ctypes.c_float
    L.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    L.oracle_lcg_fill_f16.restype = None
    L.oracle_lcg_fill_f16.argtypes = [u16, sz, ctypes.c_uint32]
    L.oracle_uniform_fill_f16.restype = None
    L.oracle_uniform_fill_f16.argtypes = [u16, sz, ctypes.c_uint64]
    L.oracle_splitmix64_at.restype = ctypes.c_uint64
    L.oracle_splitmix64_at.argtypes = [ctypes.c_uint64, ctypes.c_uint64]
    L.oracle_gemm_f64.restype = None
    L.oracle_gemm_f64.argtypes = [u16, u16, f64, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L.oracle_gemm_f64_omp.restype = ctypes.c_int
    L.oracle_gemm_f64_omp.argtypes = [u16, u16, f64, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    L.oracle_error_stats.restype = None
    L.oracle_error_stats.argtypes = [f32, f64, sz, ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]
    L.oracle_normalized_max_err.restype = ctypes.c_double
    L.oracle_normalized_max_err.argtypes = [f32, f64, sz, ctypes.c_double, ctypes.c_double, ctypes.c_int]
    L.oracle_selftest_ref.restype = None
    L.oracle_selftest_ref.argtypes = [f64, sz]
    L.oracle_f16_array_to_f32.restype = None
    L.oracle_f16_array_to_f32.argtypes = [u16, f32, sz]
    _lib = L
    return L


# Tolerances (check-gemm.cu:28-37 and the north star's normalised bound).
REL_FROB_TOL = 1e-2
MAX_ELEM_TOL = 5e-2
NORM_MAX_ERR_TOL = 1e-3


def f32_to_f16(x):
    return lib().oracle_f32_to_f16(float(x))


def f16_to_f32(h):
    return lib().oracle_f16_to_f32(int(h))


def f16_bits_to_f32(bits):
    bits = np.ascontiguousarray(bits, dtype=np.uint16).ravel()
    out = np.empty(bits.size, dtype=np.float32)
    lib().oracle_f16_array_to_f32(bits, out, bits.size)
    return out


def lcg_fill_f16(n, seed):
    out = np.empty(n, dtype=np.uint16)
    lib().oracle_lcg_fill_f16(out, n, seed & 0xffffffff)
    return out


def uniform_fill_f16(n, seed):
    out = np.empty(n, dtype=np.uint16)
    lib().oracle_uniform_fill_f16(out, n, seed & 0xffffffffffffffff)
    return out


def splitmix64_at(seed, i):
    return lib().oracle_splitmix64_at(seed, i)


def gemm_f64(A_bits, B_bits, M, N, K, threads=0, naive=False):
    """f64 reference C (M x N) from FP16 bit patterns of row-major A and B."""
    A_bits = np.ascontiguousarray(A_bits, dtype=np.uint16).ravel()
    B_bits = np.ascontiguousarray(B_bits, dtype=np.uint16).ravel()
    assert A_bits.size == M * K and B_bits.size == K * N
    C = np.empty(M * N, dtype=np.float64)
    if naive:
        lib().oracle_gemm_f64(A_bits, B_bits, C, M, N, K)
    else:
        used = lib().oracle_gemm_f64_omp(A_bits, B_bits, C, M, N, K, threads)
        if used < 0:
            raise MemoryError("oracle_gemm_f64_omp could not allocate")
    return C.reshape(M, N)


def error_stats(got, ref):
    got = np.ascontiguousarray(got, dtype=np.float32).ravel()
    ref = np.ascontiguousarray(ref, dtype=np.float64).ravel()
    assert got.size == ref.size
    frob, mx = ctypes.c_double(), ctypes.c_double()
    lib().oracle_error_stats(got, ref, ref.size, ctypes.byref(frob), ctypes.byref(mx))
    return frob.value, mx.value


def normalized_max_err(got, ref, max_abs_a, max_abs_b, K):
    got = np.ascontiguousarray(got, dtype=np.float32).ravel()
    ref = np.ascontiguousarray(ref, dtype=np.float64).ravel()
    return lib().oracle_normalized_max_err(got, ref, ref.size, float(max_abs_a), float(max_abs_b), int(K))


def passes(got, ref, max_abs_a, max_abs_b, K):
    """All three criteria: relative Frobenius, max element (check-gemm.cu:28-37),
    and max|err| / (max|A| max|B| K). Returns (ok, frob, maxRel, normErr)."""
    frob, mx = error_stats(got, ref)
    ne = normalized_max_err(got, ref, max_abs_a, max_abs_b, K)
    ok = frob <= REL_FROB_TOL and mx <= MAX_ELEM_TOL and ne <= NORM_MAX_ERR_TOL
    return ok, frob, mx, ne


# FP16-output gate (this build's, tighter than the reference's): FP16 x FP16
# products are exact in FP32; an FP32 sum of K of them is within
# K * 2^-24 * sum_k |a_ik| |b_kj| of the exact sum (the a-priori bound
# gamma_K = K u / (1 - K u), u = 2^-24, whose denominator is below 1.001 for
# K <= 2^14); rounding that sum to FP16 adds at most 2^-11 of its magnitude, or
# 2^-25 absolute below the normal range. Any kernel that accumulates in FP32
# and rounds once meets the bound element by element; its relative Frobenius
# error is then of order 2^-11 / sqrt(3), about 3e-4, hence the 1e-3 gate.
FP16_FROB_TOL = 1e-3
_U32 = 2.0 ** -24
_U16 = 2.0 ** -11


def abs_bits(bits):
    """FP16 bit patterns with the sign bit cleared (|x| for every half)."""
    return np.ascontiguousarray(bits, dtype=np.uint16) & np.uint16(0x7FFF)


def fp16_output_bound(ref, absprod, K):
    """Per-element bound |got - ref| for an FP32-accumulated, once-rounded FP16
    result: ref = A B and absprod = |A| |B| (both f64, from gemm_f64)."""
    accum = 1.001 * K * _U32 * np.asarray(absprod, dtype=np.float64)
    return _U16 * (np.abs(ref) + accum) + accum + 2.0 ** -25


def passes_fp16(got, ref, absprod, K):
    """The FP16-output gate: relative Frobenius <= 1e-3 and every element within
    fp16_output_bound. Returns (ok, frob, worst), worst = max |err| / bound."""
    got = np.asarray(got, dtype=np.float64).reshape(np.shape(ref))
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    den = np.sqrt(np.sum(ref * ref))
    frob = float(np.sqrt(np.sum(err * err)) / den) if den > 0 else float(np.any(err > 0))
    worst = float(np.max(err / fp16_output_bound(ref, absprod, K))) if err.size else 0.0
    return frob <= FP16_FROB_TOL and worst <= 1.0, frob, worst


def selftest_ref(n=4096):
    out = np.empty(n, dtype=np.float64)
    lib().oracle_selftest_ref(out, n)
    return out
