"""Calls into libbranchcraft_hip.so through the C ABI with torch-owned
device memory (torch is only the allocator and stream provider here)."""

from __future__ import annotations

import math

import numpy as np
import torch

import branchcraft_capi as capi

PAGE = 16


def lib():
    return capi.load()


def stream() -> int:
    return torch.cuda.current_stream().cuda_stream


def dev(a, dtype=None) -> torch.Tensor:
    t = torch.from_numpy(np.ascontiguousarray(a))
    if dtype is not None:
        t = t.to(dtype)
    return t.to("cuda")


def dev_at(a, shift: int) -> torch.Tensor:
    """Device copy of `a` starting `shift` bytes past a 16-byte boundary (the
    caching allocator's blocks are 512-byte aligned); shift 0 is dev(a)."""
    t = torch.from_numpy(np.ascontiguousarray(a))
    if shift == 0:
        return t.to("cuda")
    es = t.element_size()
    assert shift % es == 0 and 0 < shift < 16
    buf = torch.empty(t.numel() + 16 // es, device="cuda", dtype=t.dtype)
    view = buf[shift // es:][:t.numel()]
    view.copy_(t.reshape(-1))
    assert view.data_ptr() % 16 == shift
    return view.view(t.shape)


def nan_out(shape, shift: int, dtype=torch.float32) -> torch.Tensor:
    """Output buffer filled with NaN, `shift` bytes off 16-byte alignment."""
    n = math.prod(shape)
    buf = torch.full((n + 8,), float("nan"), device="cuda", dtype=dtype)
    es = buf.element_size()
    assert shift % es == 0 and 0 <= shift < 16
    view = buf[shift // es:][:n]
    assert view.data_ptr() % 16 == shift
    return view.view(shape)


def check(err: int, what: str) -> None:
    assert err == capi.BC_SUCCESS, f"{what} returned {err}"


def decode(q, k, v, pages, lengths, splits, *, shift=0, out_shift=None, scratch_shift=0):
    """bc_decode on numpy inputs; returns the FP32 output as numpy.  shift
    places Q, K and V that many bytes off 16-byte alignment (the element-wise
    path), out_shift the output (default: 4 bytes when shift is set) and
    scratch_shift the split partials."""
    b, hq, d = q.shape
    P, _, hkv, _ = k.shape
    tq, tk, tv = dev_at(q, shift), dev_at(k, shift), dev_at(v, shift)
    tp, tl = dev(pages.astype(np.int32)), dev(lengths.astype(np.int32))
    o = nan_out((b, hq, d), 4 * (shift > 0) if out_shift is None else out_shift)
    pa = nan_out((max(1, splits * b * hq * d),), scratch_shift)
    pml = torch.empty(max(1, splits * b * hq * 2), device="cuda", dtype=torch.float32)
    shape = capi.Shape(b, hq, hkv, d, pages.shape[1], P)
    ins = capi.Inputs(tq.data_ptr(), tk.data_ptr(), tv.data_ptr(), tp.data_ptr(),
                      tl.data_ptr(), o.data_ptr())
    scr = capi.Scratch(pa.data_ptr(), pml.data_ptr())
    check(lib().bc_decode(shape, ins, scr, splits, stream()), "bc_decode")
    torch.cuda.synchronize()
    return o.cpu().numpy()


def tree(k, v, pages, lengths, dq, dk, dv, parent, *, workspace=True, ws_offset=0, shift=0,
         phys_pages=None):
    """bc_tree_verify_ws (workspace) or bc_tree_verify.  ws_offset shifts the
    workspace pointer by that many bytes (the size passed stays the required
    one); shift places the FP16 tensors and the output that many bytes off
    16-byte alignment (the element-wise path); phys_pages overrides the
    shape's pool size (default: k.shape[0])."""
    b, n, hq, d = dq.shape
    P, _, hkv, _ = k.shape
    if phys_pages is not None:
        P = phys_pages
    tk, tv = dev_at(k, shift), dev_at(v, shift)
    tp, tl = dev(pages.astype(np.int32)), dev(lengths.astype(np.int32))
    tq, tdk, tdv = dev_at(dq, shift), dev_at(dk, shift), dev_at(dv, shift)
    tpar = dev(parent.astype(np.int32))
    o = nan_out((b, n, hq, d), 4 * (shift > 0))
    shape = capi.Shape(b, hq, hkv, d, pages.shape[1], P)
    prefix = capi.Inputs(None, tk.data_ptr(), tv.data_ptr(), tp.data_ptr(), tl.data_ptr(),
                         None)
    ins = capi.TreeInputs(prefix, tq.data_ptr(), tdk.data_ptr(), tdv.data_ptr(),
                          tpar.data_ptr(), o.data_ptr())
    L = lib()
    if workspace:
        nbytes = L.bc_tree_verify_workspace_size(shape, n)
        ws = torch.empty(max(1, nbytes + ws_offset), device="cuda", dtype=torch.uint8)
        check(L.bc_tree_verify_ws(shape, ins, n, ws.data_ptr() + ws_offset, nbytes, stream()),
              "bc_tree_verify_ws")
    else:
        check(L.bc_tree_verify(shape, ins, n, stream()), "bc_tree_verify")
    torch.cuda.synchronize()
    return o.cpu().numpy()


def packed(q, cache: torch.Tensor, strides, hkv, phys_pages, pages, lengths, scale, *,
           workspace=True, ws_offset=0, out_shift=0):
    """cache: a GPU FP16 tensor whose storage holds the packed pool; strides
    are element strides relative to cache.data_ptr().  ws_offset shifts the
    workspace pointer by that many bytes, out_shift the FP16 output."""
    b, hq, d = q.shape
    tq = dev(q)
    tp, tl = dev(pages.astype(np.int32)), dev(lengths.astype(np.int32))
    o = nan_out((b, hq, d), out_shift, torch.float16)
    shape = capi.Shape(b, hq, hkv, d, pages.shape[1], phys_pages)
    bs, hs, ss, kvs = (int(x) for x in strides)
    L = lib()
    if workspace:
        nbytes = L.bc_packed_decode_workspace_size(shape)
        ws = torch.empty(max(1, nbytes + ws_offset), device="cuda", dtype=torch.uint8)
        check(L.bc_packed_decode_ws(shape, tq.data_ptr(), cache.data_ptr(), tp.data_ptr(),
                                    tl.data_ptr(), o.data_ptr(), bs, hs, ss, kvs,
                                    float(scale), ws.data_ptr() + ws_offset, nbytes,
                                    stream()),
              "bc_packed_decode_ws")
    else:
        check(L.bc_packed_decode(shape, tq.data_ptr(), cache.data_ptr(), tp.data_ptr(),
                                 tl.data_ptr(), o.data_ptr(), bs, hs, ss, kvs,
                                 float(scale), stream()), "bc_packed_decode")
    torch.cuda.synchronize()
    return o.cpu().numpy()


def commit(cache_k: torch.Tensor, cache_v: torch.Tensor, dk: torch.Tensor,
           dv: torch.Tensor, path, dest_pages, dest_slots, request: int, *,
           phys_pages=None, kv_heads=None):
    """bc_commit_path; phys_pages and kv_heads override the shape's fields
    (defaults: the cache's page count and the drafts' head count)."""
    b, n, hkv, d = dk.shape
    tpath = torch.tensor(path, device="cuda", dtype=torch.int32)
    tdp = torch.tensor(dest_pages, device="cuda", dtype=torch.int32)
    tds = torch.tensor(dest_slots, device="cuda", dtype=torch.int32)
    kvh = hkv if kv_heads is None else kv_heads
    shape = capi.Shape(b, kvh, kvh, d, 1, cache_k.shape[0] if phys_pages is None else phys_pages)
    check(lib().bc_commit_path(shape, dk.data_ptr(), dv.data_ptr(), cache_k.data_ptr(),
                               cache_v.data_ptr(), tpath.data_ptr(), tdp.data_ptr(),
                               tds.data_ptr(), request, n, len(path), stream()),
          "bc_commit_path")
    torch.cuda.synchronize()


def commit_paths(cache_k: torch.Tensor, cache_v: torch.Tensor, dk: torch.Tensor,
                 dv: torch.Tensor, requests, nodes, dest_pages, dest_slots):
    b, n, hkv, d = dk.shape
    tr, tn, tdp, tds = (torch.tensor(x, device="cuda", dtype=torch.int32)
                        for x in (requests, nodes, dest_pages, dest_slots))
    shape = capi.Shape(b, hkv, hkv, d, 1, cache_k.shape[0])
    check(lib().bc_commit_paths(shape, dk.data_ptr(), dv.data_ptr(), cache_k.data_ptr(),
                                cache_v.data_ptr(), tr.data_ptr(), tn.data_ptr(),
                                tdp.data_ptr(), tds.data_ptr(), n, len(requests), stream()),
          "bc_commit_paths")
    torch.cuda.synchronize()


def copy_pages(cache_k: torch.Tensor, cache_v: torch.Tensor, src, dst):
    _, _, hkv, d = cache_k.shape
    ts = torch.tensor(src, device="cuda", dtype=torch.int32)
    td = torch.tensor(dst, device="cuda", dtype=torch.int32)
    shape = capi.Shape(1, hkv, hkv, d, 1, cache_k.shape[0])
    check(lib().bc_copy_pages(shape, cache_k.data_ptr(), cache_v.data_ptr(), ts.data_ptr(),
                              td.data_ptr(), len(src), stream()), "bc_copy_pages")
    torch.cuda.synchronize()


def f16_tolerance(expected: np.ndarray, atol: float) -> np.ndarray:
    """Allowed |fp16 result - fp32 oracle|: the kernel tolerance plus half an
    FP16 ulp of the expected value (round-to-nearest of the output)."""
    ulp = np.spacing(np.abs(expected).astype(np.float16)).astype(np.float32)
    return atol + 0.5 * ulp


def gate(actual, expected, atol, what):
    err = float(np.max(np.abs(actual.astype(np.float64) - expected.astype(np.float64)))) \
        if actual.size else 0.0
    assert np.all(np.isfinite(actual)), f"{what}: non-finite output"
    assert err <= atol, f"{what}: max abs error {err:.3e} > {atol:.1e}"
    return err


def rsqrt(d):
    return 1.0 / math.sqrt(d)
