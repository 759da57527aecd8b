"""ctypes wrapper of oracle/_build/liboracle_attn.so (tiled_ref.c).  Test use only."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "liboracle_attn.so")
_lib = None

_f = ctypes.POINTER(ctypes.c_float)


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        _lib = ctypes.CDLL(_LIB_PATH)
        i = ctypes.c_int
        fl = ctypes.c_float
        sigs = {
            "oracle_qkv_split_fwd": [_f, _f, _f, _f, i, i, i, i],
            "oracle_qkv_split_bwd": [_f, _f, _f, _f, i, i, i, i],
            "oracle_head_merge_fwd": [_f, _f, i, i, i, i],
            "oracle_head_merge_bwd": [_f, _f, i, i, i, i],
            "oracle_causal_softmax_fwd": [_f, _f, i, i, i, fl],
            "oracle_causal_softmax_bwd": [_f, _f, _f, i, i, i, fl],
            "oracle_tiled_fwd": [_f, _f, _f, _f, i, i, i, i, fl, _f, _f],
            "oracle_dot_do_o": [_f, _f, _f, ctypes.c_int64, i],
            "oracle_tiled_bwd_dq": [_f, _f, _f, _f, _f, _f, _f, _f, i, i, i, i, fl],
            "oracle_tiled_bwd_dkdv": [_f, _f, _f, _f, _f, _f, _f, _f, _f, i, i, i, i, fl],
        }
        for name, argtypes in sigs.items():
            fn = getattr(_lib, name)
            fn.argtypes = argtypes
            fn.restype = None
    return _lib


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"]
    return a.ctypes.data_as(_f)


def _c(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def qkv_split_fwd(qkv, B, T, H, d):
    qkv = _c(qkv)
    q, k, v = (np.empty((B, H, T, d), np.float32) for _ in range(3))
    lib().oracle_qkv_split_fwd(_p(qkv), _p(q), _p(k), _p(v), B, T, H, d)
    return q, k, v


def qkv_split_bwd(dq, dk, dv, B, T, H, d):
    dq, dk, dv = _c(dq), _c(dk), _c(dv)
    out = np.empty((B, T, 3 * H * d), np.float32)
    lib().oracle_qkv_split_bwd(_p(dq), _p(dk), _p(dv), _p(out), B, T, H, d)
    return out


def head_merge_fwd(x, B, H, T, d):
    x = _c(x)
    out = np.empty((B, T, H * d), np.float32)
    lib().oracle_head_merge_fwd(_p(x), _p(out), B, H, T, d)
    return out


def head_merge_bwd(dout, B, H, T, d):
    dout = _c(dout)
    out = np.empty((B, H, T, d), np.float32)
    lib().oracle_head_merge_bwd(_p(dout), _p(out), B, H, T, d)
    return out


def causal_softmax_fwd(scores, B, H, T, scale):
    scores = _c(scores)
    probs = np.empty_like(scores)
    lib().oracle_causal_softmax_fwd(_p(scores), _p(probs), B, H, T, scale)
    return probs


def causal_softmax_bwd(dprobs, probs, B, H, T, scale):
    dprobs, probs = _c(dprobs), _c(probs)
    ds = np.empty_like(probs)
    lib().oracle_causal_softmax_bwd(_p(dprobs), _p(probs), _p(ds), B, H, T, scale)
    return ds


def tiled_fwd(q, k, v, scale):
    q, k, v = _c(q), _c(k), _c(v)
    B, H, T, d = q.shape
    out = np.empty_like(q)
    m = np.empty((B, H, T), np.float32)
    l = np.empty((B, H, T), np.float32)
    lib().oracle_tiled_fwd(_p(q), _p(k), _p(v), _p(out), B, H, T, d, scale, _p(m), _p(l))
    return out, m, l


def dot_do_o(do, o):
    do, o = _c(do), _c(o)
    d = do.shape[-1]
    rows = do.size // d
    D = np.empty(do.shape[:-1], np.float32)
    lib().oracle_dot_do_o(_p(do), _p(o), _p(D), rows, d)
    return D


def tiled_bwd(q, k, v, o, do, m, l, scale):
    q, k, v, o, do, m, l = (_c(x) for x in (q, k, v, o, do, m, l))
    B, H, T, d = q.shape
    D = dot_do_o(do, o)
    dq, dk, dv = (np.empty_like(q) for _ in range(3))
    lib().oracle_tiled_bwd_dq(_p(q), _p(k), _p(v), _p(do), _p(m), _p(l), _p(D), _p(dq), B, H,
                              T, d, scale)
    lib().oracle_tiled_bwd_dkdv(_p(q), _p(k), _p(v), _p(do), _p(m), _p(l), _p(D), _p(dk),
                                _p(dv), B, H, T, d, scale)
    return dq, dk, dv, D
