"""Python binding of the cost model (libridge_model.so, include/ridge_model.h)
and a runner for the ridge-predict CLI.

The reference keeps a single copy of the model math in C++ and has its Python
tools reach it through `ridge-predict --batch` (tools/ridge-autotune.py:53-62,
bench/validate.py:221-231). The same holds here: predict() calls the C++ model
through its C ABI and predict_batch() runs the CLI; nothing re-implements the
model in Python.
"""

import ctypes
import os
import subprocess

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libridge_model.so")
PREDICT_BIN = os.path.join(_PKG, "bin", "ridge-predict")

BOTTLENECKS = ["TENSOR_CORE", "SMEM", "HBM", "OCC", "WAVES", "ENVELOPE", "DOES_NOT_FIT"]


class _Config(ctypes.Structure):
    _fields_ = [("M", ctypes.c_longlong), ("N", ctypes.c_longlong), ("K", ctypes.c_longlong)] + \
               [(n, ctypes.c_int) for n in ("BM", "BN", "BK", "warpM", "warpN", "mmaM", "mmaN", "mmaK",
                                           "stages", "regsPerThread", "groupM", "schedule")]


_PRED_FIELDS = [("predictedTFLOPS", ctypes.c_double), ("bottleneck", ctypes.c_int)] + \
    [(n, ctypes.c_double) for n in ("computeTFLOPS", "hbmTFLOPS", "peakTensorTFLOPS", "smEfficiency", "occFactor",
                                    "arithmeticIntensity", "baseIntensity", "l2ReuseFactor", "waveEfficiency",
                                    "totalCtas", "ctaSlots", "wavesExact", "envelopeEfficiency",
                                    "tPrologueCycles", "tEpilogueCycles", "tBodyCycles", "kSteps")] + \
    [("numWarps", ctypes.c_int), ("ctasPerSM", ctypes.c_int)] + \
    [(n, ctypes.c_double) for n in ("tComputeCycles", "tSmemCycles", "tStepCycles", "reuseTilesM", "reuseTilesN",
                                    "compulsoryIntensity", "tailClockFactor", "l2HitBytes", "powerClockFactor",
                                    "fillRounds", "refillMissShare", "mallLoad", "mallStretch",
                                    "kernelSeconds", "dramReadBytes", "dramWriteBytes", "dramShare", "bodyFactor",
                                    "bodyShare", "cuShare", "mfmaShare", "ldsShare", "matrixLoad",
                                    "observedClockHz")]


class _Prediction(ctypes.Structure):
    _fields_ = _PRED_FIELDS


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError("%s is missing: run `python -m ridge_amd.build`" % LIB_PATH)
    L = ctypes.CDLL(LIB_PATH)
    L.ridge_model_default_config.argtypes = [ctypes.POINTER(_Config)]
    L.ridge_model_default_config.restype = None
    L.ridge_model_hw_load.argtypes = [ctypes.c_char_p, ctypes.c_char_p, ctypes.c_size_t]
    L.ridge_model_hw_load.restype = ctypes.c_void_p
    L.ridge_model_hw_free.argtypes = [ctypes.c_void_p]
    L.ridge_model_hw_free.restype = None
    L.ridge_model_hw_calibrated.argtypes = [ctypes.c_void_p]
    L.ridge_model_hw_calibrated.restype = ctypes.c_int
    L.ridge_model_hw_name.argtypes = [ctypes.c_void_p]
    L.ridge_model_hw_name.restype = ctypes.c_char_p
    L.ridge_model_predict.argtypes = [ctypes.c_void_p, ctypes.POINTER(_Config), ctypes.POINTER(_Prediction)]
    L.ridge_model_predict.restype = ctypes.c_int
    L.ridge_model_bottleneck_name.argtypes = [ctypes.c_int]
    L.ridge_model_bottleneck_name.restype = ctypes.c_char_p
    for fn, struct in ((L.ridge_model_config_size, _Config), (L.ridge_model_prediction_size, _Prediction)):
        fn.argtypes = []
        fn.restype = ctypes.c_size_t
        if fn() != ctypes.sizeof(struct):
            raise RuntimeError("%s: %d bytes in %s but %d in this binding" % (fn.__name__, fn(), LIB_PATH,
                                                                             ctypes.sizeof(struct)))
    _lib = L
    return L


class Hardware:
    """A loaded hardware model: "a100", "mi355x" or a calibration JSON path."""

    def __init__(self, spec):
        err = ctypes.create_string_buffer(512)
        h = lib().ridge_model_hw_load(spec.encode(), err, len(err))
        if not h:
            raise ValueError(err.value.decode())
        self._h = h
        self.spec = spec

    @property
    def calibrated(self):
        return bool(lib().ridge_model_hw_calibrated(self._h))

    @property
    def name(self):
        return lib().ridge_model_hw_name(self._h).decode()

    def close(self):
        if self._h:
            lib().ridge_model_hw_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def default_config():
    c = _Config()
    lib().ridge_model_default_config(ctypes.byref(c))
    return {f: getattr(c, f) for f, _ in _Config._fields_}


def predict(hw, **cfg):
    """Runs the model on one config (GemmConfig field names; unspecified fields
    take the reference defaults). Returns a dict of the Prediction fields with
    the bottleneck as its label string."""
    c = _Config()
    lib().ridge_model_default_config(ctypes.byref(c))
    for k, v in cfg.items():
        if not hasattr(c, k):
            raise KeyError(k)
        setattr(c, k, int(v))
    p = _Prediction()
    if lib().ridge_model_predict(hw._h, ctypes.byref(c), ctypes.byref(p)) != 0:
        raise RuntimeError("ridge_model_predict failed")
    out = {f: getattr(p, f) for f, _ in _PRED_FIELDS}
    out["bottleneck"] = BOTTLENECKS[out["bottleneck"]]
    return out


def predict_batch(in_csv, out_csv, hw="a100", binary=PREDICT_BIN):
    """`ridge-predict --batch`: hw is "a100", "mi355x" or a JSON path. Returns the
    CLI's stderr line; raises on failure."""
    if not os.path.exists(binary):
        raise RuntimeError("%s is missing: run `python -m ridge_amd.build`" % binary)
    cmd = [binary]
    cmd += ["--gpu", hw] if hw in ("a100", "mi355x") else ["--hw", hw]
    cmd += ["--batch", in_csv, "--out", out_csv]
    p = subprocess.run(cmd, capture_output=True, text=True)
    if p.returncode != 0:
        raise RuntimeError("ridge-predict failed: %s" % p.stderr)
    return p.stderr
