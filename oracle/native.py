"""ctypes view of oracle/liboracle_moe.so (fp64 brute force + generator).

TEST INFRASTRUCTURE ONLY."""
import ctypes
import os

import numpy as np

from . import build as _build

_lib = None


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(_build.LIB):
            _build.build()
        lib = ctypes.CDLL(_build.LIB)
        vp, u32 = ctypes.c_void_p, ctypes.c_uint32
        lib.oracle_dequant_matvec_f64.argtypes = [vp, vp, vp, vp, vp, u32, u32]
        lib.oracle_dequant_matvec_f64.restype = None
        lib.oracle_bf16_matvec_f64.argtypes = [vp, vp, vp, vp, u32, u32]
        lib.oracle_bf16_matvec_f64.restype = None
        lib.oracle_synth_key.argtypes = [u32, u32, u32]
        lib.oracle_synth_key.restype = u32
        lib.oracle_synth_region.argtypes = [u32, u32, vp, ctypes.c_size_t]
        lib.oracle_synth_region.restype = None
        _lib = lib
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def dequant_matvec_f64(W, S, x):
    """fp64 y and absacc of an MXFP4 matvec (test_glm_mxfp4.cu:46-67)."""
    W = np.ascontiguousarray(W, np.uint8)
    S = np.ascontiguousarray(S, np.uint8)
    x = np.ascontiguousarray(x, np.float32)
    N, K = W.shape[0], W.shape[1] * 2
    y = np.empty(N, np.float64)
    a = np.empty(N, np.float64)
    load().oracle_dequant_matvec_f64(_p(W), _p(S), _p(x), _p(y), _p(a), N, K)
    return y, a


def bf16_matvec_f64(W, x):
    W = np.ascontiguousarray(W, np.uint16)
    x = np.ascontiguousarray(x, np.float32)
    N, K = W.shape
    y = np.empty(N, np.float64)
    a = np.empty(N, np.float64)
    load().oracle_bf16_matvec_f64(_p(W), _p(x), _p(y), _p(a), N, K)
    return y, a


def synth_key(seed, layer, expert):
    return int(load().oracle_synth_key(seed, layer, expert))


def synth_region(key, r, nbytes):
    out = np.empty(nbytes, np.uint8)
    load().oracle_synth_region(key, r, _p(out), nbytes)
    return out
