"""Host-side mirror of the reference's kernel table, over the C ABI in
include/ridge_gemm.h (libridge_gemm.so).

The reference's operator API is a table of KernelVariant rows with a launch
function each (bench/kernels/gemm-mma.cuh:368-387); its callers walk the table,
skip variants that do not divide the shape, launch, and compare. This module
exposes the same surface in Python:

    variants()                 -> list of Variant (the table, in order)
    variant(i)                 -> Variant
    find_variant(BM, BN, ...)  -> index or -1
    launch(i, A, B, C, M, N, K, stream) -> hipError_t value (0 = success)
    gemm(A, B, i)              -> C, raising on any error

Device buffers are torch tensors (or raw device addresses); torch provides device
memory and streams only. There is no fallback: if the native library is missing,
every entry point raises.
"""

import ctypes
import os
from dataclasses import dataclass, asdict

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libridge_gemm.so")

HIP_SUCCESS = 0
HIP_ERROR_INVALID_VALUE = 1

_lib = None


class RidgeGemmError(RuntimeError):
    pass


class _VariantStruct(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int) for n in (
        "BM", "BN", "BK", "WM", "WN", "stages", "groupM", "ldsBytes", "threads", "regsPerThread",
        "waves", "vgprs", "agprs", "sgprs", "scratchBytes", "occupancy", "pingPong", "schedule")]

SCHEDULES = {0: "uniform", 1: "ping-pong", 2: "persistent"}


@dataclass(frozen=True)
class Variant:
    index: int
    BM: int
    BN: int
    BK: int
    WM: int
    WN: int
    stages: int
    groupM: int
    ldsBytes: int
    threads: int
    regsPerThread: int
    waves: int
    vgprs: int
    agprs: int
    sgprs: int
    scratchBytes: int
    occupancy: int
    pingPong: int
    schedule: int

    @property
    def smemBytes(self):
        """The reference's name for the per-workgroup on-chip buffer size."""
        return self.ldsBytes

    def divides(self, M, N, K):
        return bool(lib().ridge_gemm_divides(self.index, M, N, K))

    def key(self):
        return (self.BM, self.BN, self.BK, self.WM, self.WN, self.stages, self.groupM)

    @property
    def schedule_name(self):
        return SCHEDULES.get(self.schedule, "unknown")

    def label(self):
        """BMxBNxBK wWMxWN sS gG, with " persistent" for the store-behind rows."""
        base = "%dx%dx%d w%dx%d s%d g%d" % self.key()
        return base + " persistent" if self.schedule == 2 else base

    def as_dict(self):
        return asdict(self)


def lib():
    """Loads libridge_gemm.so once. Raises if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RidgeGemmError("%s is missing: run `python -m ridge_amd.build` (or "
                             "__graft_entry__.build()) first" % LIB_PATH)
    L = ctypes.CDLL(LIB_PATH)
    c_int, c_void_p, c_size_t = ctypes.c_int, ctypes.c_void_p, ctypes.c_size_t
    L.ridge_gemm_num_variants.restype = c_int
    L.ridge_gemm_num_variants.argtypes = []
    L.ridge_gemm_get_variant.restype = c_int
    L.ridge_gemm_get_variant.argtypes = [c_int, ctypes.POINTER(_VariantStruct)]
    L.ridge_gemm_find_variant.restype = c_int
    L.ridge_gemm_find_variant.argtypes = [c_int] * 7
    L.ridge_gemm_divides.restype = c_int
    L.ridge_gemm_divides.argtypes = [c_int] * 4
    L.ridge_gemm_launch.restype = c_int
    L.ridge_gemm_launch.argtypes = [c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_void_p]
    L.ridge_gemm_split_rows.restype = c_int
    L.ridge_gemm_split_rows.argtypes = [c_int] * 5
    L.ridge_gemm_launch_split.restype = c_int
    L.ridge_gemm_launch_split.argtypes = [c_int, c_int, c_int, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                          c_void_p]
    L.ridge_gemm_variant_table_csv.restype = c_size_t
    L.ridge_gemm_variant_table_csv.argtypes = [ctypes.c_char_p, c_size_t]
    L.ridge_fill_uniform_f16.restype = c_int
    L.ridge_fill_uniform_f16.argtypes = [c_void_p, c_size_t, ctypes.c_uint64, c_void_p]
    L.ridge_fill_lcg_f16.restype = c_int
    L.ridge_fill_lcg_f16.argtypes = [c_void_p, c_size_t, ctypes.c_uint32, c_void_p]
    L.ridge_blaslt_create.restype = c_int
    L.ridge_blaslt_create.argtypes = [ctypes.POINTER(c_void_p)]
    L.ridge_blaslt_destroy.restype = c_int
    L.ridge_blaslt_destroy.argtypes = [c_void_p]
    L.ridge_blaslt_prepare.restype = c_int
    L.ridge_blaslt_prepare.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int,
                                       c_int, c_int, c_void_p]
    L.ridge_blaslt_gemm.restype = c_int
    L.ridge_blaslt_gemm.argtypes = [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_void_p]
    L.ridge_gemm_build_info.restype = ctypes.c_char_p
    L.ridge_gemm_build_info.argtypes = []
    L.ridge_gemm_variant_struct_size.restype = c_size_t
    L.ridge_gemm_variant_struct_size.argtypes = []
    if L.ridge_gemm_variant_struct_size() != ctypes.sizeof(_VariantStruct):
        raise RidgeGemmError("ridge_gemm_variant_t is %d bytes in %s but %d in this binding: rebuild or update "
                             "_VariantStruct" % (L.ridge_gemm_variant_struct_size(), LIB_PATH,
                                                 ctypes.sizeof(_VariantStruct)))
    _lib = L
    return L


def num_variants():
    return lib().ridge_gemm_num_variants()


def variant(i):
    s = _VariantStruct()
    rc = lib().ridge_gemm_get_variant(i, ctypes.byref(s))
    if rc != HIP_SUCCESS:
        raise IndexError("variant index %d out of range" % i)
    return Variant(i, *[getattr(s, f) for f, _ in _VariantStruct._fields_])


def variants():
    return [variant(i) for i in range(num_variants())]


def find_variant(BM, BN, BK, WM, WN, stages, groupM):
    return lib().ridge_gemm_find_variant(BM, BN, BK, WM, WN, stages, groupM)


def variant_table_csv():
    L = lib()
    n = L.ridge_gemm_variant_table_csv(None, 0)
    buf = ctypes.create_string_buffer(n + 1)
    L.ridge_gemm_variant_table_csv(buf, n + 1)
    return buf.value.decode()


def _ptr(x):
    if x is None:
        return None
    if isinstance(x, int):
        return x
    return x.data_ptr()


def _stream_handle(stream):
    if stream is None:
        import torch
        return torch.cuda.current_stream().cuda_stream
    if isinstance(stream, int):
        return stream
    return stream.cuda_stream


def launch(i, A, B, C, M, N, K, stream=None):
    """Enqueues C = A B with variant i; returns the hipError_t value."""
    return lib().ridge_gemm_launch(i, _ptr(A), _ptr(B), _ptr(C), M, N, K, _stream_handle(stream))


def bound_launch(i, A, B, C, M, N, K, stream=None):
    """A zero-argument callable that enqueues C = A B with variant i, its
    arguments converted once: the per-call host cost is one foreign call, for
    timing loops whose launches are shorter than Python's argument handling."""
    f = lib().ridge_gemm_launch
    args = (i, _ptr(A), _ptr(B), _ptr(C), M, N, K, _stream_handle(stream))
    # The closure holds the operands (and the stream object), so the raw
    # pointers in `args` stay valid for as long as the callable exists.
    keep = (A, B, C, stream)

    def call():
        assert keep is not None
        rc = f(*args)
        if rc != HIP_SUCCESS:
            raise RidgeGemmError("ridge_gemm_launch(variant %d, %dx%dx%d) returned hipError %d" % (i, M, N, K, rc))
    return call


def split_rows(body, M, N, K, num_cus=256):
    """Rows of C a row split gives the body row: whole rounds of its resident
    workgroups on num_cus CUs (M when the grid already is whole rounds, 0 when it
    is less than one, -1 for a bad index or a shape the row does not divide)."""
    return lib().ridge_gemm_split_rows(body, M, N, K, num_cus)


def launch_split(body, tail, body_rows, A, B, C, M, N, K, stream=None):
    """Enqueues C = A B as two launches: variant `body` on rows [0, body_rows),
    variant `tail` on the rest. Returns the hipError_t value; a refused call
    enqueues nothing."""
    return lib().ridge_gemm_launch_split(body, tail, body_rows, _ptr(A), _ptr(B), _ptr(C), M, N, K,
                                         _stream_handle(stream))


def bound_launch_split(body, tail, body_rows, A, B, C, M, N, K, stream=None):
    """launch_split with its arguments converted once (see bound_launch)."""
    f = lib().ridge_gemm_launch_split
    args = (body, tail, body_rows, _ptr(A), _ptr(B), _ptr(C), M, N, K, _stream_handle(stream))
    keep = (A, B, C, stream)

    def call():
        assert keep is not None
        rc = f(*args)
        if rc != HIP_SUCCESS:
            raise RidgeGemmError("ridge_gemm_launch_split(%d, %d, %d rows, %dx%dx%d) returned hipError %d"
                                 % (body, tail, body_rows, M, N, K, rc))
    return call


def _check_operands(A, B, C=None):
    import torch
    if A.dtype != torch.float16 or B.dtype != torch.float16:
        raise RidgeGemmError("A and B must be float16")
    if not (A.is_cuda and B.is_cuda):
        raise RidgeGemmError("A and B must be device tensors")
    if A.dim() != 2 or B.dim() != 2 or A.shape[1] != B.shape[0]:
        raise RidgeGemmError("shapes %s x %s do not chain" % (tuple(A.shape), tuple(B.shape)))
    if not (A.is_contiguous() and B.is_contiguous()):
        raise RidgeGemmError("A and B must be row-major contiguous")
    if A.device != B.device:
        raise RidgeGemmError("A is on %s but B on %s" % (A.device, B.device))
    if C is not None:
        if C.dtype != torch.float16 or not C.is_contiguous() or tuple(C.shape) != (A.shape[0], B.shape[1]):
            raise RidgeGemmError("C must be a contiguous float16 tensor of shape (M, N)")
        if C.device != A.device:
            raise RidgeGemmError("C is on %s but A and B on %s" % (C.device, A.device))


def gemm(A, B, index=0, out=None, stream=None):
    """C = A @ B with variant `index`, FP16 out. Raises on any launch error."""
    import torch
    _check_operands(A, B, out)
    M, K = A.shape
    N = B.shape[1]
    C = out if out is not None else torch.empty((M, N), dtype=torch.float16, device=A.device)
    # The library launches on the current device; make it the operands' one.
    with torch.cuda.device(A.device):
        rc = launch(index, A, B, C, M, N, K, stream)
    if rc != HIP_SUCCESS:
        raise RidgeGemmError("ridge_gemm_launch(variant %d, %dx%dx%d) returned hipError %d" % (index, M, N, K, rc))
    return C


def fill_uniform(t, seed, stream=None):
    """U[-1,1) FP16 fill of a contiguous device tensor (element i from (seed, i))."""
    rc = lib().ridge_fill_uniform_f16(_ptr(t), t.numel(), seed, _stream_handle(stream))
    if rc != HIP_SUCCESS:
        raise RidgeGemmError("ridge_fill_uniform_f16 returned %d" % rc)
    return t


def fill_lcg(t, seed, stream=None):
    """The reference's LCG fill (U[-0.5,0.5] in FP16) of a contiguous device tensor."""
    rc = lib().ridge_fill_lcg_f16(_ptr(t), t.numel(), seed & 0xffffffff, _stream_handle(stream))
    if rc != HIP_SUCCESS:
        raise RidgeGemmError("ridge_fill_lcg_f16 returned %d" % rc)
    return t


class BlasLt:
    """hipBLASLt comparator (row-major via operand swap), best-of heuristic picks."""

    def __init__(self):
        h = ctypes.c_void_p()
        rc = lib().ridge_blaslt_create(ctypes.byref(h))
        if rc != 0:
            raise RidgeGemmError("ridge_blaslt_create returned %d" % rc)
        self._h = h

    def prepare(self, A, B, C, M, N, K, c_is_f32=False, candidates=8, iters=10, stream=None):
        rc = lib().ridge_blaslt_prepare(self._h, _ptr(A), _ptr(B), _ptr(C), M, N, K, int(c_is_f32),
                                        candidates, iters, _stream_handle(stream))
        if rc != 0:
            raise RidgeGemmError("ridge_blaslt_prepare(%dx%dx%d) returned %d" % (M, N, K, rc))

    def gemm(self, A, B, C, M, N, K, c_is_f32=False, stream=None):
        if not self._h:
            raise RidgeGemmError("the hipBLASLt handle is closed")
        rc = lib().ridge_blaslt_gemm(self._h, _ptr(A), _ptr(B), _ptr(C), M, N, K, int(c_is_f32),
                                     _stream_handle(stream))
        if rc != 0:
            raise RidgeGemmError("ridge_blaslt_gemm(%dx%dx%d) returned %d" % (M, N, K, rc))

    def bound_gemm(self, A, B, C, M, N, K, c_is_f32=False, stream=None):
        """gemm() as a zero-argument callable with its arguments converted once."""
        if not self._h:
            raise RidgeGemmError("the hipBLASLt handle is closed")
        f = lib().ridge_blaslt_gemm
        args = (self._h, _ptr(A), _ptr(B), _ptr(C), M, N, K, int(c_is_f32), _stream_handle(stream))
        # The closure holds the operands and this object; a call after close()
        # is refused instead of reaching a destroyed handle.
        keep = (A, B, C, stream)

        def call():
            assert keep is not None
            if not self._h:
                raise RidgeGemmError("the hipBLASLt handle is closed")
            rc = f(*args)
            if rc != 0:
                raise RidgeGemmError("ridge_blaslt_gemm(%dx%dx%d) returned %d" % (M, N, K, rc))
        return call

    def close(self):
        if self._h:
            lib().ridge_blaslt_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
