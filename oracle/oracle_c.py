"""ctypes wrapper of the C oracle (bc_oracle.c) for numpy arrays.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker, never by the product path.
FP16 arrays are numpy float16; integer arrays int32.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libbc_oracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        _lib = ctypes.CDLL(str(LIB_PATH))
        _lib.oracle_max_abs_error.restype = ctypes.c_float
        _lib.oracle_h2f.restype = ctypes.c_float
        _lib.oracle_h2f.argtypes = [ctypes.c_uint16]
        _lib.oracle_f2h.restype = ctypes.c_uint16
        _lib.oracle_f2h.argtypes = [ctypes.c_float]
        _lib.oracle_packed_decode.argtypes = [ctypes.c_int] * 5 + [ctypes.c_void_p] * 4 + \
            [ctypes.c_longlong] * 4 + [ctypes.c_double, ctypes.c_void_p, ctypes.c_void_p,
                                        ctypes.c_int]
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    assert a.flags["C_CONTIGUOUS"], "oracle inputs must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


def _h(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float16)


def _i(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.int32)


def f2h(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    lib().oracle_f2h_array(_p(x), _p(out), ctypes.c_size_t(x.size))
    return out


def h2f(bits: np.ndarray) -> np.ndarray:
    bits = np.ascontiguousarray(bits, dtype=np.uint16)
    out = np.empty(bits.shape, dtype=np.float32)
    lib().oracle_h2f_array(_p(bits), _p(out), ctypes.c_size_t(bits.size))
    return out


def decode(q, k, v, pages, lengths, threads: int = 1) -> np.ndarray:
    """q [B,Hq,D]; k, v [P,16,Hkv,D]; pages [B,max_pages]; lengths [B]."""
    q, k, v, pages, lengths = _h(q), _h(k), _h(v), _i(pages), _i(lengths)
    b, hq, d = q.shape
    hkv = k.shape[2]
    out = np.empty((b, hq, d), dtype=np.float32)
    lib().oracle_decode(b, hq, hkv, d, pages.shape[1], _p(q), _p(k), _p(v), _p(pages),
                        _p(lengths), _p(out), threads)
    return out


def packed_decode(q, cache, pages, lengths, strides, hkv, scale, threads: int = 1):
    """cache: FP16 buffer read through element strides = (block, head, slot,
    kv); returns (fp32 result, fp16 result)."""
    q, pages, lengths = _h(q), _i(pages), _i(lengths)
    flat = _h(cache).reshape(-1)
    b, hq, d = q.shape
    bs, hs, ss, kvs = (int(x) for x in strides)
    out32 = np.empty((b, hq, d), dtype=np.float32)
    out16 = np.empty((b, hq, d), dtype=np.uint16)
    lib().oracle_packed_decode(b, hq, hkv, d, pages.shape[1], _p(q), _p(flat), _p(pages),
                               _p(lengths), bs, hs, ss, kvs, float(scale), _p(out32),
                               _p(out16), threads)
    return out32, out16.view(np.float16)


def tree(k, v, pages, lengths, draft_q, draft_k, draft_v, parent, threads: int = 1):
    """k, v [P,16,Hkv,D]; draft_q [B,N,Hq,D]; draft_k/v [B,N,Hkv,D]; parent [B,N]."""
    k, v, dq, dk, dv = _h(k), _h(v), _h(draft_q), _h(draft_k), _h(draft_v)
    pages, lengths, parent = _i(pages), _i(lengths), _i(parent)
    b, n, hq, d = dq.shape
    hkv = k.shape[2]
    out = np.empty((b, n, hq, d), dtype=np.float32)
    lib().oracle_tree(b, n, hq, hkv, d, pages.shape[1], _p(k), _p(v), _p(pages),
                      _p(lengths), _p(dq), _p(dk), _p(dv), _p(parent), _p(out), threads)
    return out


def commit(cache_k, cache_v, draft_k, draft_v, path, dest_pages, dest_slots, request):
    """In-place on copies; returns (new_k, new_v)."""
    ck, cv = _h(cache_k).copy(), _h(cache_v).copy()
    dk, dv = _h(draft_k), _h(draft_v)
    path, dp, ds = _i(path), _i(dest_pages), _i(dest_slots)
    b, n, hkv, d = dk.shape
    lib().oracle_commit(b, n, hkv, d, ck.shape[0], _p(dk), _p(dv), _p(ck), _p(cv),
                        _p(path), _p(dp), _p(ds), request, len(path))
    return ck, cv


def copy_pages(cache_k, cache_v, src, dst):
    ck, cv = _h(cache_k).copy(), _h(cache_v).copy()
    src, dst = _i(src), _i(dst)
    _, _, hkv, d = ck.shape
    lib().oracle_copy_pages(hkv, d, ck.shape[0], _p(ck), _p(cv), _p(src), _p(dst), len(src))
    return ck, cv


def expand_tree(k, v, pages, lengths, draft_k, draft_v, parent):
    """Expanded-prefix fixture (src/main.cu:375-423): returns
    (lengths [B*N], pages [B*N, max_pages], k, v)."""
    k, v, dk, dv = _h(k), _h(v), _h(draft_k), _h(draft_v)
    pages, lengths, parent = _i(pages), _i(lengths), _i(parent)
    b, n, hkv, d = dk.shape
    smax = ctypes.c_int(0)
    total = ctypes.c_int(0)
    L = lib()
    L.oracle_expand_tree(b, n, hkv, d, pages.shape[1], _p(k), _p(v), _p(pages), _p(lengths),
                         _p(dk), _p(dv), _p(parent), ctypes.byref(smax), ctypes.byref(total),
                         None, None, None, None)
    out_len = np.empty(b * n, dtype=np.int32)
    out_pages = np.empty((b * n, max(smax.value, 1)), dtype=np.int32)
    out_k = np.empty((total.value + 7, 16, hkv, d), dtype=np.float16)
    out_v = np.empty_like(out_k)
    L.oracle_expand_tree(b, n, hkv, d, pages.shape[1], _p(k), _p(v), _p(pages), _p(lengths),
                         _p(dk), _p(dv), _p(parent), ctypes.byref(smax), ctypes.byref(total),
                         _p(out_len), _p(out_pages), _p(out_k), _p(out_v))
    return out_len, out_pages, out_k, out_v


def max_abs_error(a, b) -> float:
    a = np.ascontiguousarray(a, dtype=np.float32).reshape(-1)
    b = np.ascontiguousarray(b, dtype=np.float32).reshape(-1)
    assert a.size == b.size
    return float(lib().oracle_max_abs_error(_p(a), _p(b), ctypes.c_size_t(a.size)))
