"""ctypes binding of the oracle's C restatement (exact_c.c). Test infrastructure only.

install() routes the oracle's group-128 linear through oc_group_linear (the numpy path stays the
default); weights(), scales() and embed() are fast equivalents of exact_amd.synth.weights_np /
scales_np / embed_np.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "libexact_oracle_c.so")
_LIB = None


def load(build=True):
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH) and build:
        subprocess.run(["make", "-C", HERE], check=True, capture_output=True)
    lib = ctypes.CDLL(LIB_PATH)
    P, I64, U64 = ctypes.c_void_p, ctypes.c_int64, ctypes.c_uint64
    lib.oc_weights.argtypes = [U64, P, I64, I64, I64, I64, P]
    lib.oc_scales.argtypes = [U64, I64, I64, I64, I64, P]
    lib.oc_group_linear.argtypes = [P, ctypes.c_int, I64, I64, P, I64, P, P]
    lib.oc_embed.argtypes = [P, P, I64, I64, P]
    for f in (lib.oc_weights, lib.oc_scales, lib.oc_group_linear, lib.oc_embed):
        f.restype = None
    _LIB = lib
    return lib


def _p(a):
    return ctypes.c_void_p(a.ctypes.data)


def weights(key, thr, N, K, n0=0, n1=None):
    n1 = N if n1 is None else n1
    out = np.empty((K, n1 - n0), np.int8)
    thr = np.ascontiguousarray(thr, np.uint32)
    load().oc_weights(key, _p(thr), N, K, n0, n1, _p(out))
    return out


def scales(key, N, K, lo, hi):
    G = K // 128
    out = np.empty((G, N), np.int64)
    load().oc_scales(key, lo, hi, N, G, _p(out))
    return out


def embed(w_kn, M_gn):
    """exact_amd.synth.embed_np: Q16 rows (V, D) = rint(w * M / 2^12), ties to even."""
    D, V = w_kn.shape
    w = np.ascontiguousarray(w_kn, np.int8)
    M = np.ascontiguousarray(M_gn, np.int64)
    out = np.empty((V, D), np.int64)
    load().oc_embed(_p(w), _p(M), D, V, _p(out))
    return out


def group_t(xq, w, Mg):
    """t (R, N) int64 = sum_g M_g * (xq[:, g] @ w[g]) for xq int16/int8-valued (R, K), w (K, N) int8."""
    R, K = xq.shape
    N = w.shape[1]
    xb = 2 if np.abs(xq).max(initial=0) > 127 else 1
    x = np.ascontiguousarray(xq, np.int16 if xb == 2 else np.int8)
    w = np.ascontiguousarray(w, np.int8)
    M = np.ascontiguousarray(Mg, np.int64)
    t = np.empty((R, N), np.int64)
    load().oc_group_linear(_p(x), xb, R, K, _p(w), N, _p(M), _p(t))
    return t


def install():
    import exact_oracle
    load()
    exact_oracle.set_group_kernel(group_t)


def uninstall():
    import exact_oracle
    exact_oracle.set_group_kernel(None)
