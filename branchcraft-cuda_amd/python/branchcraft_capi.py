"""ctypes view of the Branchcraft C ABI (``include/branchcraft.h``).

This is the binding a Python caller (or a maintainer porting the reference's
``branchcraft::`` calls) uses to reach ``libbranchcraft_hip.so`` without
PyTorch.  Pointers are plain integers (device addresses), streams are
``hipStream_t`` values as integers; every call returns the HIP error code.
Loading the library never touches the GPU.
"""

from __future__ import annotations

import ctypes
from ctypes import (POINTER, Structure, c_char_p, c_float, c_int, c_int32,
                    c_longlong, c_size_t, c_uint16, c_void_p)
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent.parent / "lib" / "libbranchcraft_hip.so"

BC_SUCCESS = 0
BC_ERROR_INVALID_VALUE = 1
BC_ERROR_OUT_OF_MEMORY = 2
BC_STATIC_SCRATCH_BYTES = 16 << 20
BC_SCRATCH_SLOTS = 4
BC_SCRATCH_SLOT_BYTES = 18 << 20
BC_PAGE_SIZE = 16
BC_MAX_SPLITS = 256
BC_MAX_TREE_NODES = 256

# Every entry point include/branchcraft.h declares.
EXPORTED = (
    "bc_decode", "bc_auto_splits", "bc_tree_verify",
    "bc_tree_verify_workspace_size", "bc_tree_verify_ws", "bc_commit_path", "bc_commit_paths", "bc_copy_pages", "bc_packed_decode", "bc_packed_decode_workspace_size",
    "bc_packed_decode_ws", "bc_packed_decode_noalloc", "bc_version",
)


class Shape(Structure):
    _fields_ = [("batch", c_int), ("query_heads", c_int), ("kv_heads", c_int),
                ("dim", c_int), ("max_pages", c_int), ("physical_pages", c_int)]


class Inputs(Structure):
    _fields_ = [("q", c_void_p), ("k", c_void_p), ("v", c_void_p),
                ("pages", c_void_p), ("lengths", c_void_p), ("output", c_void_p)]


class Scratch(Structure):
    _fields_ = [("partial_a", c_void_p), ("partial_ml", c_void_p)]


class TreeInputs(Structure):
    _fields_ = [("prefix", Inputs), ("draft_q", c_void_p), ("draft_k", c_void_p),
                ("draft_v", c_void_p), ("parent", c_void_p), ("output", c_void_p)]


_lib = None


def load(path: str | Path | None = None) -> ctypes.CDLL:
    """Load the library (once) and declare every prototype."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path else LIB_PATH
    if not p.exists():
        raise ImportError(f"{p} is missing; build it with branchcraft-cuda_amd/build.py")
    lib = ctypes.CDLL(str(p))
    lib.bc_decode.argtypes = [Shape, Inputs, Scratch, c_int, c_void_p]
    lib.bc_decode.restype = c_int
    lib.bc_auto_splits.argtypes = [Shape, c_int, c_int]
    lib.bc_auto_splits.restype = c_int
    lib.bc_tree_verify.argtypes = [Shape, TreeInputs, c_int, c_void_p]
    lib.bc_tree_verify.restype = c_int
    lib.bc_tree_verify_workspace_size.argtypes = [Shape, c_int]
    lib.bc_tree_verify_workspace_size.restype = c_size_t
    lib.bc_tree_verify_ws.argtypes = [Shape, TreeInputs, c_int, c_void_p, c_size_t, c_void_p]
    lib.bc_tree_verify_ws.restype = c_int
    lib.bc_commit_path.argtypes = [Shape, c_void_p, c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_void_p, c_void_p, c_int, c_int, c_int,
                                   c_void_p]
    lib.bc_commit_path.restype = c_int
    lib.bc_commit_paths.argtypes = [Shape, c_void_p, c_void_p, c_void_p, c_void_p,
                                    c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int,
                                    c_void_p]
    lib.bc_commit_paths.restype = c_int
    lib.bc_copy_pages.argtypes = [Shape, c_void_p, c_void_p, c_void_p, c_void_p,
                                  c_int, c_void_p]
    lib.bc_copy_pages.restype = c_int
    lib.bc_packed_decode.argtypes = [Shape, c_void_p, c_void_p, c_void_p, c_void_p,
                                     c_void_p, c_longlong, c_longlong, c_longlong,
                                     c_longlong, c_float, c_void_p]
    lib.bc_packed_decode.restype = c_int
    lib.bc_packed_decode_workspace_size.argtypes = [Shape]
    lib.bc_packed_decode_workspace_size.restype = c_size_t
    lib.bc_packed_decode_ws.argtypes = [Shape, c_void_p, c_void_p, c_void_p, c_void_p,
                                        c_void_p, c_longlong, c_longlong, c_longlong,
                                        c_longlong, c_float, c_void_p, c_size_t,
                                        c_void_p]
    lib.bc_packed_decode_ws.restype = c_int
    lib.bc_packed_decode_noalloc.argtypes = [Shape, c_void_p, c_void_p, c_void_p, c_void_p,
                                             c_void_p, c_longlong, c_longlong, c_longlong,
                                             c_longlong, c_float, c_void_p]
    lib.bc_packed_decode_noalloc.restype = c_int
    lib.bc_version.argtypes = []
    lib.bc_version.restype = c_char_p
    if path is None:
        _lib = lib
    return lib


def shape(batch, query_heads, kv_heads, dim, max_pages, physical_pages) -> Shape:
    return Shape(batch, query_heads, kv_heads, dim, max_pages, physical_pages)


__all__ = ["BC_SUCCESS", "BC_ERROR_INVALID_VALUE", "BC_ERROR_OUT_OF_MEMORY",
           "BC_STATIC_SCRATCH_BYTES", "BC_PAGE_SIZE", "BC_MAX_SPLITS",
           "BC_MAX_TREE_NODES", "EXPORTED", "Shape", "Inputs", "Scratch",
           "TreeInputs", "load", "shape", "LIB_PATH", "POINTER", "c_int32",
           "c_uint16"]
