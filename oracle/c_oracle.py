"""ctypes loader of the C oracle (oracle/_build/libhc_oracle.so).

TEST INFRASTRUCTURE ONLY (tests/, smoke(), bench.py cpu_baseline).
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "_build", "libhc_oracle.so")
_lib = None


def build():
    r = subprocess.run(["make", "-s", "-C", HERE], capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + r.stdout + r.stderr)
    return LIB


def load():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        lib = ctypes.CDLL(LIB)
        vp, i32, i64, f32 = ctypes.c_void_p, ctypes.c_int32, ctypes.c_int64, ctypes.c_float
        lib.hco_decode_attention.argtypes = [ctypes.c_int, vp, vp, vp, vp, vp, ctypes.c_int, ctypes.c_int, f32,
                                             ctypes.c_int, vp]
        lib.hco_decode_attention.restype = None
        lib.hco_topk_select.argtypes = [vp, ctypes.c_int, ctypes.c_int, vp]
        lib.hco_topk_select.restype = ctypes.c_int
        lib.hco_num_threads.restype = ctypes.c_int
        lib.hco_set_threads.argtypes = [ctypes.c_int]
        _lib = lib
    return _lib


def _p(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def decode_attention(q, k, v, row_off, row_len, scale, dtype_code, chunk=4096):
    """q [rows, G, 128] (float32 or bf16 bits as uint16), k/v flat natural layout."""
    lib = load()
    rows, G, _ = q.shape
    out = np.zeros((rows, G, 128), dtype=np.float32)
    row_off = np.ascontiguousarray(row_off, dtype=np.int64)
    row_len = np.ascontiguousarray(row_len, dtype=np.int32)
    lib.hco_decode_attention(dtype_code, _p(np.ascontiguousarray(q)), _p(np.ascontiguousarray(k)),
                             _p(np.ascontiguousarray(v)), _p(row_off), _p(row_len), rows, G, float(scale), chunk,
                             _p(out))
    return out


def topk_select(scores, cap):
    lib = load()
    s = np.ascontiguousarray(scores, dtype=np.float32)
    out = np.zeros(max(cap, 1), dtype=np.int32)
    n = lib.hco_topk_select(_p(s), len(s), int(cap), _p(out))
    return out[:n].astype(np.int64)


def set_threads(n):
    load().hco_set_threads(int(n))


def num_threads():
    return load().hco_num_threads()
