#!/usr/bin/env python3
"""Benchmark of the Branchcraft paged-attention hot path on one MI355X.

Headline (`value`): benchmark config 5 -- packed-KV decode, batch 64, ragged
contexts U[128, 4096], 32/8 heads, D=128, cache [20000, 2, 16, 8, 128] FP16
-- as algorithmic HBM GB/s (each attended token's K+V once, plus Q, output,
used page-table entries and lengths) over one call of bc_packed_decode_ws
(the kernels behind torch.ops.branchcraft.packed_decode_out).  A step is
one call over the whole batch; inputs are resident in HBM before timing.

Also reported (`results`), each with the reference's timing protocol (5
warm-ups, 7 trials x 20 launches, median; src/main.cu:354-373):
  C1 paged decode B=1 L=512;  C2 tree_verify 1 x 2048 + 7 nodes;
  C3 tree_verify 8 x (2048+5) shared prefix vs the expanded-prefix decode,
     plus the copy-on-write commit;  C4 split-K decode B=4, L~U[16K, 32K];
  C5 packed decode through the reference's signature (bc_packed_decode,
     whose split scratch is a slot of the library's pool), and 20 calls
     captured in one HIP graph and replayed (per-call time); paged decode
     (bc_decode, separate K and V) on the same C5 sequences; one 32K-token
     packed sequence through both calls.
  Tree results time bc_tree_verify_ws and the reference's signature
  bc_tree_verify (whose split scratch is a pool slot).
The CPU baseline times the C oracle (oracle/bc_oracle.c) on the whole C5
workload on this host's cores.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT / "branchcraft-cuda_amd" / "python"))

HBM_PEAK_GBS = 8000.0
# HBM bytes per config-5 call measured with rocprofv3 counters: attention
# FETCH 264,747.3 KiB x 2 + WRITE 3,021.5 KiB, merge FETCH 1,595.0 KiB x 2 +
# WRITE 448.0 KiB (FETCH_SIZE reads half of a 512 MiB copy's bytes).
C5_HBM_TRAFFIC_BYTES = (264747.3 * 2 + 3021.5 + 1595.0 * 2 + 448.0) * 1024
MFMA_F16_PEAK_TFLOPS = 2500.0
PAGE = 16


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    ap.add_argument("--only", default="",
                    help="comma list of configs to run (c1..c5; tl = a 256-node tree; "
                         "long = one 32K-token packed sequence)")
    ap.add_argument("--calibrate", action="store_true",
                    help="also run a plain 512 MiB device copy, the known-size reference "
                         "for scaling FETCH_SIZE / WRITE_SIZE counters")
    return ap.parse_args()


# ---------------------------------------------------------------------------
# timing


def median_us(torch, fn, trials=7, repeats=20, warmup=5):
    """Reference protocol: warm-ups, then trials of back-to-back launches
    bracketed by events on the launch stream; median per-launch time."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(trials):
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(repeats):
            fn()
        stop.record()
        stop.synchronize()
        times.append(start.elapsed_time(stop) * 1000.0 / repeats)
    return statistics.median(times)


def paired_median_us(torch, fns, rounds=3):
    """median_us of several calls that run the same work, taken in alternating
    rounds (the median of each call's per-round medians), so that a drift of
    the GPU's speed over the run (after a fixture is written, say) does not
    favour whichever call is timed first."""
    per = [[] for _ in fns]
    for _ in range(rounds):
        for i, fn in enumerate(fns):
            per[i].append(median_us(torch, fn))
    return [statistics.median(v) for v in per]


def graph_replay_us(torch, make_call, out, calls=20, replays=20):
    """Per-call time of `calls` back-to-back calls captured in one HIP graph
    (torch.cuda.CUDAGraph on ROCm) and replayed `replays` times, as a serving
    loop runs a captured decode step.  `make_call` must read the current
    stream when it is called.  Every replay's `out` must equal the eager
    result."""
    make_call()()
    torch.cuda.synchronize()
    eager = out.clone()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        fn = make_call()
        for _ in range(calls):
            fn()
    times = []
    for _ in range(replays):
        out.zero_()
        torch.cuda.synchronize()
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        graph.replay()
        stop.record()
        stop.synchronize()
        times.append(start.elapsed_time(stop) * 1000.0 / calls)
        if not torch.equal(out, eager):
            raise RuntimeError("graph replay differs from the eager call")
    del graph
    return statistics.median(times)


# ---------------------------------------------------------------------------
# workloads (synthetic, seeded)


def block_table(rng, lengths, max_pages, pool):
    perm = rng.permutation(pool).astype(np.int32)
    pages = np.full((len(lengths), max_pages), -1, dtype=np.int32)
    cur = 0
    for i, n in enumerate(lengths):
        c = -(-int(n) // PAGE)
        pages[i, :c] = perm[cur:cur + c]
        cur += c
    return pages


def decode_bytes(lengths, hq, hkv, d, out_bytes):
    b = len(lengths)
    used = sum(-(-int(n) // PAGE) for n in lengths)
    return int(sum(int(n) for n in lengths) * hkv * d * 2 * 2 + b * hq * d * 2
               + b * hq * d * out_bytes + used * 4 + b * 4)


class Ctx:
    def __init__(self):
        import torch
        import branchcraft_capi as capi
        self.torch = torch
        self.capi = capi
        self.lib = capi.load()

    def stream(self):
        return self.torch.cuda.current_stream().cuda_stream

    def check(self, err, what):
        if err != 0:
            raise RuntimeError(f"{what} failed with HIP error {err}")


def make_decode_call(cx, q, k, v, pages, lengths, out, splits, scratch):
    capi = cx.capi
    b, hq, d = q.shape
    shape = capi.Shape(b, hq, k.shape[2], d, pages.shape[1], k.shape[0])
    ins = capi.Inputs(q.data_ptr(), k.data_ptr(), v.data_ptr(), pages.data_ptr(),
                      lengths.data_ptr(), out.data_ptr())
    scr = capi.Scratch(scratch[0].data_ptr(), scratch[1].data_ptr())
    lib, st = cx.lib, cx.stream()

    def call():
        err = lib.bc_decode(shape, ins, scr, splits, st)
        if err:
            raise RuntimeError(f"bc_decode error {err}")
    return call


def decode_scratch(cx, b, hq, d, splits):
    t = cx.torch
    return (t.empty(max(1, splits * b * hq * d), device="cuda", dtype=t.float32),
            t.empty(max(1, splits * b * hq * 2), device="cuda", dtype=t.float32))


def bench_c1(cx):
    t = cx.torch
    rng = np.random.default_rng(1)
    pages = rng.permutation(64).astype(np.int32)[:32].reshape(1, 32)
    g = t.Generator(device="cuda").manual_seed(1)
    q = t.randn((1, 32, 128), generator=g, device="cuda", dtype=t.float16)
    k = t.randn((64, 16, 8, 128), generator=g, device="cuda", dtype=t.float16)
    v = t.randn((64, 16, 8, 128), generator=g, device="cuda", dtype=t.float16)
    tp = t.from_numpy(pages).cuda()
    tl = t.tensor([512], device="cuda", dtype=t.int32)
    out = t.empty((1, 32, 128), device="cuda", dtype=t.float32)
    shape = cx.capi.Shape(1, 32, 8, 128, 32, 64)
    res = {}
    for splits in sorted({1, cx.lib.bc_auto_splits(shape, 512, cx.cus), 8}):
        scr = decode_scratch(cx, 1, 32, 128, splits)
        us = median_us(t, make_decode_call(cx, q, k, v, tp, tl, out, splits, scr))
        res[f"splits{splits}_us"] = round(us, 3)
    nbytes = decode_bytes([512], 32, 8, 128, 4)
    best = min(res.values())
    res.update(bytes=nbytes, best_us=best, gbs=round(nbytes / best / 1e3, 1),
               workload="paged decode B=1 L=512 Hq=32 Hkv=8 D=128, pool 64 pages")
    return res


def bench_c4(cx):
    t = cx.torch
    rng = np.random.default_rng(4)
    lengths = rng.integers(16384, 32769, size=4).astype(np.int32)
    used = sum(-(-int(n) // PAGE) for n in lengths)
    pool = used + 16
    pages = block_table(rng, lengths, int(-(-lengths.max() // PAGE)), pool)
    g = t.Generator(device="cuda").manual_seed(4)
    q = t.randn((4, 32, 128), generator=g, device="cuda", dtype=t.float16)
    k = t.randn((pool, 16, 8, 128), generator=g, device="cuda", dtype=t.float16)
    v = t.randn((pool, 16, 8, 128), generator=g, device="cuda", dtype=t.float16)
    tp, tl = t.from_numpy(pages).cuda(), t.from_numpy(lengths).cuda()
    out = t.empty((4, 32, 128), device="cuda", dtype=t.float32)
    shape = cx.capi.Shape(4, 32, 8, 128, pages.shape[1], pool)
    auto = cx.lib.bc_auto_splits(shape, int(lengths.max()), cx.cus)
    nbytes = decode_bytes(lengths, 32, 8, 128, 4)
    res = {"auto_splits": auto}
    for splits in sorted({16, auto, 64}):
        scr = decode_scratch(cx, 4, 32, 128, splits)
        us = median_us(t, make_decode_call(cx, q, k, v, tp, tl, out, splits, scr))
        res[f"splits{splits}_us"] = round(us, 3)
        res[f"splits{splits}_gbs"] = round(nbytes / us / 1e3, 1)
    best = min(v for kk, v in res.items() if kk.endswith("_us"))
    res.update(bytes=nbytes, best_us=best, gbs=round(nbytes / best / 1e3, 1),
               pct_peak=round(100 * nbytes / best / 1e3 / HBM_PEAK_GBS, 1),
               lengths=[int(x) for x in lengths],
               workload="split-K paged decode B=4 L~U[16384,32768] Hq=32 Hkv=8 D=128")
    return res


class C5:
    """Config 5 inputs, resident on the GPU."""

    def __init__(self, cx):
        t = cx.torch
        rng = np.random.default_rng(5)
        self.B, self.hq, self.hkv, self.d, self.nb, self.maxp = 64, 32, 8, 128, 20000, 256
        self.lengths = rng.integers(128, 4097, size=self.B).astype(np.int32)
        self.pages = block_table(rng, self.lengths, self.maxp, self.nb)
        g = t.Generator(device="cuda").manual_seed(5)
        self.cache = t.randn((self.nb, 2, 16, self.hkv, self.d), generator=g, device="cuda",
                             dtype=t.float16)
        self.q = t.randn((self.B, self.hq, self.d), generator=g, device="cuda",
                         dtype=t.float16)
        self.out = t.empty_like(self.q)
        self.tp = t.from_numpy(self.pages).cuda()
        self.tl = t.from_numpy(self.lengths).cuda()
        c = self.cache
        self.strides = (c.stride(0), c.stride(3), c.stride(2), c.stride(1))
        self.scale = 1.0 / math.sqrt(self.d)
        self.shape = cx.capi.Shape(self.B, self.hq, self.hkv, self.d, self.maxp, self.nb)
        self.ws_bytes = cx.lib.bc_packed_decode_workspace_size(self.shape)
        self.ws = t.empty(max(1, self.ws_bytes), device="cuda", dtype=t.uint8)
        self.bytes = decode_bytes(self.lengths, self.hq, self.hkv, self.d, 2)

    def call(self, cx, workspace=True):
        return packed_call(cx, self, "ws" if workspace else "reference")


def packed_call(cx, p, mode):
    """One packed-decode call on p's inputs: "ws" is bc_packed_decode_ws with
    a caller workspace, "reference" the reference's signature
    (bc_packed_decode: a split shape borrows a slot of the library's scratch
    pool)."""
    lib, st = cx.lib, cx.stream()
    bs, hs, ss, kvs = p.strides
    args = (p.shape, p.q.data_ptr(), p.cache.data_ptr(), p.tp.data_ptr(),
            p.tl.data_ptr(), p.out.data_ptr(), bs, hs, ss, kvs, p.scale)
    if mode == "ws":
        ws, nb = p.ws.data_ptr(), p.ws_bytes

        def f():
            err = lib.bc_packed_decode_ws(*args, ws, nb, st)
            if err:
                raise RuntimeError(f"bc_packed_decode_ws error {err}")
    else:
        def f():
            err = lib.bc_packed_decode(*args, st)
            if err:
                raise RuntimeError(f"bc_packed_decode error {err}")
    return f


class LongPacked:
    """One 32K-token sequence in a [P, 2, 16, 8, 128] cache: the reference's
    named next problem for packed decode (long sequences, CONTRIBUTING.md:20-23)."""

    def __init__(self, cx, tokens=32768):
        t = cx.torch
        rng = np.random.default_rng(32)
        self.hq, self.hkv, self.d = 32, 8, 128
        npg = tokens // PAGE
        self.nb = npg + 64
        self.lengths = np.array([tokens], dtype=np.int32)
        self.pages = block_table(rng, self.lengths, npg, self.nb)
        g = t.Generator(device="cuda").manual_seed(32)
        self.cache = t.randn((self.nb, 2, 16, self.hkv, self.d), generator=g, device="cuda",
                             dtype=t.float16)
        self.q = t.randn((1, self.hq, self.d), generator=g, device="cuda", dtype=t.float16)
        self.out = t.empty_like(self.q)
        self.tp = t.from_numpy(self.pages).cuda()
        self.tl = t.from_numpy(self.lengths).cuda()
        c = self.cache
        self.strides = (c.stride(0), c.stride(3), c.stride(2), c.stride(1))
        self.scale = 1.0 / math.sqrt(self.d)
        self.shape = cx.capi.Shape(1, self.hq, self.hkv, self.d, npg, self.nb)
        self.ws_bytes = cx.lib.bc_packed_decode_workspace_size(self.shape)
        self.ws = t.empty(max(1, self.ws_bytes), device="cuda", dtype=t.uint8)
        self.bytes = decode_bytes(self.lengths, self.hq, self.hkv, self.d, 2)


def bench_packed_modes(cx, p, workload):
    """Both packed-decode calls on p: per-call time, GB/s, and the reference
    signature's time over the workspace call's."""
    t = cx.torch
    res = {}
    outs = {}
    modes = ("ws", "reference")
    fns = [packed_call(cx, p, mode) for mode in modes]
    for mode, fn, us in zip(modes, fns, paired_median_us(t, fns)):
        res[f"{mode}_us"] = round(us, 3)
        res[f"{mode}_gbs"] = round(p.bytes / us / 1e3, 1)
        fn()
        t.cuda.synchronize()
        outs[mode] = p.out.clone()
    if not t.equal(outs["ws"], outs["reference"]):
        raise RuntimeError("reference-signature packed call differs from the workspace call")
    res["ref_over_ws"] = round(res["reference_us"] / res["ws_us"], 3)
    res["reference_pct_peak"] = round(100 * p.bytes / res["reference_us"] / 1e3 / HBM_PEAK_GBS,
                                      1)
    res.update(bytes=p.bytes, workload=workload)
    return res


def bench_c5_paged(cx, c5):
    """bc_decode (separate [P, 16, Hkv, D] K and V, FP32 output) on the config-5
    sequences: the same lengths, page table, Q and K/V values as the packed
    call, so its output must match the packed output up to FP16 rounding."""
    t = cx.torch
    k = c5.cache[:, 0].contiguous()
    v = c5.cache[:, 1].contiguous()
    out = t.empty((c5.B, c5.hq, c5.d), device="cuda", dtype=t.float32)
    shape = cx.capi.Shape(c5.B, c5.hq, c5.hkv, c5.d, c5.maxp, c5.nb)
    auto = cx.lib.bc_auto_splits(shape, int(c5.lengths.max()), cx.cus)
    nbytes = decode_bytes(c5.lengths, c5.hq, c5.hkv, c5.d, 4)
    res = {"auto_splits": auto}
    for splits in sorted({1, auto}):
        scr = decode_scratch(cx, c5.B, c5.hq, c5.d, splits)
        call = make_decode_call(cx, c5.q, k, v, c5.tp, c5.tl, out, splits, scr)
        us = median_us(t, call)
        res[f"splits{splits}_us"] = round(us, 3)
    call()
    c5.call(cx, workspace=True)()
    t.cuda.synchronize()
    diff = float((out - c5.out.float()).abs().max())
    if diff > 2e-3:
        raise RuntimeError(f"paged and packed decode differ by {diff}")
    us = res[f"splits{auto}_us"]
    res.update(bytes=nbytes, us=us, gbs=round(nbytes / us / 1e3, 1),
               pct_peak=round(100 * nbytes / us / 1e3 / HBM_PEAK_GBS, 1),
               max_abs_diff_vs_packed=diff,
               workload="paged decode (bc_decode, auto splits) on the config-5 sequences, "
                        "FP32 output")
    del k, v
    return res


def tree_setup(cx, batch, prefix, seed, nodes=7):
    """Shared-prefix tree fixture on the GPU: every request's page-table row
    names the same physical pages (random permutation of the pool), and the
    rows hold two unused entries (-1) past the prefix's pages, as the
    reference's fixture does (src/main.cu:152-158)."""
    t = cx.torch
    rng = np.random.default_rng(seed)
    hq, hkv, d, n = 32, 8, 128, nodes
    npg = -(-prefix // PAGE)
    pool = npg + 2 * batch + 2
    perm = rng.permutation(pool).astype(np.int32)
    pages = np.full((batch, npg + 2), -1, dtype=np.int32)
    pages[:, :npg] = perm[:npg]
    parent = np.full((batch, n), -1, dtype=np.int32)
    for b in range(batch):
        for i in range(1, n):
            parent[b, i] = rng.integers(0, i)
    g = t.Generator(device="cuda").manual_seed(seed)
    f = dict(
        k=t.randn((pool, 16, hkv, d), generator=g, device="cuda", dtype=t.float16),
        v=t.randn((pool, 16, hkv, d), generator=g, device="cuda", dtype=t.float16),
        dq=t.randn((batch, n, hq, d), generator=g, device="cuda", dtype=t.float16),
        dk=t.randn((batch, n, hkv, d), generator=g, device="cuda", dtype=t.float16),
        dv=t.randn((batch, n, hkv, d), generator=g, device="cuda", dtype=t.float16),
        pages=t.from_numpy(pages).cuda(), parent_np=parent,
        parent=t.from_numpy(parent).cuda(),
        lengths=t.full((batch,), prefix, device="cuda", dtype=t.int32),
        batch=batch, prefix=prefix, hq=hq, hkv=hkv, d=d, n=n, pool=pool, pages_np=pages,
        free_pages=[int(x) for x in perm[npg:]])
    f["out"] = t.empty((batch, n, hq, d), device="cuda", dtype=t.float32)
    return f


def tree_call(cx, f, workspace=True):
    """bc_tree_verify_ws (workspace) or bc_tree_verify (the reference's
    signature: a plan that splits borrows a slot of the library's scratch
    pool)."""
    capi = cx.capi
    shape = capi.Shape(f["batch"], f["hq"], f["hkv"], f["d"], f["pages"].shape[1], f["pool"])
    prefix = capi.Inputs(None, f["k"].data_ptr(), f["v"].data_ptr(), f["pages"].data_ptr(),
                         f["lengths"].data_ptr(), None)
    ins = capi.TreeInputs(prefix, f["dq"].data_ptr(), f["dk"].data_ptr(), f["dv"].data_ptr(),
                          f["parent"].data_ptr(), f["out"].data_ptr())
    lib, st, n = cx.lib, cx.stream(), f["n"]
    if workspace:
        nb = lib.bc_tree_verify_workspace_size(shape, n)
        f["ws"] = cx.torch.empty(max(1, nb), device="cuda", dtype=cx.torch.uint8)
        ws = f["ws"].data_ptr()

        def call():
            err = lib.bc_tree_verify_ws(shape, ins, n, ws, nb, st)
            if err:
                raise RuntimeError(f"tree_verify workspace call error {err}")
    else:
        def call():
            err = lib.bc_tree_verify(shape, ins, n, st)
            if err:
                raise RuntimeError(f"bc_tree_verify error {err}")
    return call


def ancestors(parent_row, node):
    out, cur = [], node
    while 0 <= cur < len(parent_row) and len(out) < len(parent_row):
        out.append(cur)
        cur = int(parent_row[cur])
    return out


def tree_metrics(f):
    b, n, hq, hkv, d, L = f["batch"], f["n"], f["hq"], f["hkv"], f["d"], f["prefix"]
    depth_sum = sum(len(ancestors(f["parent_np"][bi], x)) for bi in range(b) for x in range(n))
    unique = (L * hkv * d * 2 * 2 + b * n * hkv * d * 2 * 2 + b * n * hq * d * 2
              + b * n * hq * d * 4 + b * (-(-L // PAGE)) * 4 + b * 4 + b * n * 4)
    flops = 4 * d * hq * (b * n * L + depth_sum)
    return unique, flops


def expanded_fixture(cx, f):
    """Each (request, node) becomes its own paged sequence: the prefix then
    the root-to-node path (src/main.cu:375-423), built on the GPU."""
    t = cx.torch
    b, n, hkv, d, L = f["batch"], f["n"], f["hkv"], f["d"], f["prefix"]
    pool_rows = f["k"].shape[0] * PAGE
    kflat = t.cat([f["k"].reshape(-1, hkv, d), f["dk"].reshape(-1, hkv, d)])
    vflat = t.cat([f["v"].reshape(-1, hkv, d), f["dv"].reshape(-1, hkv, d)])
    lens, rows = [], []
    tok = np.arange(L)
    for bi in range(b):
        prow = f["pages_np"][bi][tok // PAGE] * PAGE + tok % PAGE
        for x in range(n):
            path = ancestors(f["parent_np"][bi], x)[::-1]
            src = np.concatenate([prow, pool_rows + bi * n + np.asarray(path)])
            pad = (-len(src)) % PAGE
            lens.append(len(src))
            rows.append(np.concatenate([src, np.zeros(pad, dtype=src.dtype)]))
    maxp = max(len(r) for r in rows) // PAGE
    pages = np.full((b * n, maxp), -1, dtype=np.int32)
    cur = 0
    for s, r in enumerate(rows):
        c = len(r) // PAGE
        pages[s, :c] = np.arange(cur, cur + c)
        cur += c
    idx = t.from_numpy(np.concatenate(rows).astype(np.int64)).cuda()
    ek = kflat.index_select(0, idx).reshape(cur, PAGE, hkv, d).contiguous()
    ev = vflat.index_select(0, idx).reshape(cur, PAGE, hkv, d).contiguous()
    q = f["dq"].reshape(b * n, f["hq"], d).contiguous()
    return (q, ek, ev, t.from_numpy(pages).cuda(),
            t.tensor(lens, device="cuda", dtype=t.int32), lens)


def bench_tree(cx, batch, prefix, seed, with_expanded, nodes=7):
    t = cx.torch
    f = tree_setup(cx, batch, prefix, seed, nodes)
    res = {}
    calls = {"ws": tree_call(cx, f, True), "ref": tree_call(cx, f, False)}
    outs = {}
    times = paired_median_us(t, list(calls.values()))
    for (name, fn), us in zip(calls.items(), times):
        res[f"tree_{name}_us"] = round(us, 3)
        fn()
        t.cuda.synchronize()
        outs[name] = f["out"].clone()
    res["tree_ws_vs_ref_maxdiff"] = float((outs["ws"] - outs["ref"]).abs().max())
    res["tree_ref_over_ws"] = round(res["tree_ref_us"] / res["tree_ws_us"], 3)
    unique, flops = tree_metrics(f)
    tree_us = min(res["tree_ws_us"], res["tree_ref_us"])
    res.update(tree_us=tree_us, tree_bytes=unique, tree_gflop=round(flops / 1e9, 4),
               tree_gbs=round(unique / tree_us / 1e3, 1),
               tree_mfma_pct=round(100 * flops / tree_us / 1e6 / MFMA_F16_PEAK_TFLOPS, 3))
    if with_expanded:
        q, ek, ev, ep, el, lens = expanded_fixture(cx, f)
        out = t.empty((q.shape[0], q.shape[1], q.shape[2]), device="cuda", dtype=t.float32)
        exp_bytes = decode_bytes(lens, f["hq"], f["hkv"], f["d"], 4)
        shape = cx.capi.Shape(q.shape[0], f["hq"], f["hkv"], f["d"], ep.shape[1], ek.shape[0])
        auto = cx.lib.bc_auto_splits(shape, max(lens), cx.cus)
        # The baseline is the best of the heuristic's split count, its
        # neighbours and the unsplit kernel, so the tree is not compared with
        # an unlucky split.
        for splits in sorted({1, max(1, auto - 1), auto, auto + 1}):
            scr = decode_scratch(cx, q.shape[0], f["hq"], f["d"], splits)
            fn = make_decode_call(cx, q, ek, ev, ep, el, out, splits, scr)
            us = median_us(t, fn)
            res[f"expanded_splits{splits}_us"] = round(us, 3)
            fn()
            t.cuda.synchronize()
            diff = float((out.reshape(outs["ws"].shape) - outs["ws"]).abs().max())
            res[f"expanded_splits{splits}_maxdiff_vs_tree"] = diff
            if diff > 3e-4:
                raise RuntimeError(f"tree and expanded decode disagree: {diff}")
        exp_us = min(v for kk, v in res.items() if kk.startswith("expanded") and kk.endswith("_us"))
        res.update(expanded_us=exp_us, expanded_bytes=exp_bytes,
                   expanded_gbs=round(exp_bytes / exp_us / 1e3, 1),
                   expanded_over_tree=round(exp_us / tree_us, 2))
        del ek, ev
        res["commit"] = bench_commit(cx, f)
    res["workload"] = (f"tree_verify {batch} req x {prefix} shared prefix + {nodes} nodes "
                       "(random parents), Hq=32 Hkv=8 D=128")
    return res


def bench_commit(cx, f):
    """Commit after verification: each request writes a random root-to-leaf
    path at the end of the shared prefix.  A prefix that ends inside a page
    (config 3, 2,053 tokens) clones that shared page per request first; one
    that fills its last page (config 2, 2,048 tokens) writes the path into a
    fresh page.  The launches are the ones PagedTreeCache.commit_many issues:
    every clone (bc_copy_pages), then every accepted node of every request
    (bc_commit_paths)."""
    t = cx.torch
    capi = cx.capi
    rng = np.random.default_rng(303)
    b, n, hkv, d, L = f["batch"], f["n"], f["hkv"], f["d"], f["prefix"]
    partial = L % PAGE != 0
    last = int(f["pages_np"][0, (L - 1) // PAGE])
    fresh = f["free_pages"][:b]
    src = t.tensor([last] * b, device="cuda", dtype=t.int32)
    dst = t.tensor(fresh, device="cuda", dtype=t.int32)
    shape = capi.Shape(b, hkv, hkv, d, 1, f["pool"])
    k, v = f["k"].clone(), f["v"].clone()
    rows = []
    for bi in range(b):
        par = f["parent_np"][bi]
        leaves = [x for x in range(n) if x not in set(par.tolist())]
        path = ancestors(par, int(rng.choice(leaves)))[::-1]
        for j, node in enumerate(path):
            pos = L + j
            if pos // PAGE != L // PAGE:
                raise RuntimeError("accepted path must fit the page that follows the prefix")
            rows.append((bi, node, fresh[bi], pos % PAGE))
    reqs, nodes, pages, slots = (t.tensor([r[j] for r in rows], device="cuda", dtype=t.int32)
                                 for j in range(4))
    lib, st = cx.lib, cx.stream()

    def call():
        err = 0
        if partial:
            err |= lib.bc_copy_pages(shape, k.data_ptr(), v.data_ptr(), src.data_ptr(),
                                     dst.data_ptr(), b, st)
        err |= lib.bc_commit_paths(shape, f["dk"].data_ptr(), f["dv"].data_ptr(),
                                   k.data_ptr(), v.data_ptr(), reqs.data_ptr(),
                                   nodes.data_ptr(), pages.data_ptr(), slots.data_ptr(),
                                   n, len(rows), st)
        if err:
            raise RuntimeError("commit failed")
    us = median_us(t, call)
    cloned = b if partial else 0
    moved = 2 * cloned * PAGE * hkv * d * 2 * 2 + 2 * len(rows) * hkv * d * 2 * 2
    return {"us": round(us, 3), "bytes": moved, "launches": 2 if partial else 1,
            "cloned_pages": cloned, "accepted_nodes": len(rows)}


# ---------------------------------------------------------------------------


def cpu_baseline(c5_host):
    """C oracle on the whole config-5 workload: one thread (the reference's
    oracle is single-threaded), 16 threads (a one-GPU box's CPU share) and
    every core this process may run on (os.sched_getaffinity), which gives
    `value`; os.cpu_count() is reported beside it."""
    sys.path.insert(0, str(ROOT))
    from oracle import oracle_c
    q, cache, pages, lengths, strides, nbytes = c5_host
    host_cpus = os.cpu_count() or 1
    try:
        cores = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        cores = host_cpus
    res = {}
    for threads in sorted({1, min(16, cores), cores}):
        reps = 1 if threads == 1 else 3
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            oracle_c.packed_decode(q, cache, pages, lengths, strides, 8, 1 / math.sqrt(128),
                                   threads=threads)
            times.append(time.perf_counter() - t0)
        res[threads] = statistics.median(times)
    return {
        "value": round(nbytes / res[cores] / 1e9, 3), "unit": "GB/s", "cores": cores,
        "kind": "port",
        "sample": ("whole config-5 workload (64 sequences, "
                   f"{int(lengths.sum())} tokens) through oracle/bc_oracle.c, "
                   f"median of 3 at {cores} threads (every core in this process's "
                   "affinity mask)"),
        "host_cpu_count": host_cpus,
        "single_thread_gbs": round(nbytes / res[1] / 1e9, 3),
        "sixteen_thread_gbs": round(nbytes / res[min(16, cores)] / 1e9, 3),
        "single_thread_s": round(res[1], 3), "multi_thread_s": round(res[cores], 3),
    }


def main():
    args = parse()
    if args.gpus != 1:
        print(json.dumps({"error": "this build measures one GPU only; run with --gpus 1",
                          "n_gpus": args.gpus}))
        sys.exit(2)
    cx = Ctx()
    t = cx.torch
    torch = t
    torch.cuda.set_device(0)
    props = torch.cuda.get_device_properties(0)
    cx.cus = props.multi_processor_count
    only = set(filter(None, args.only.split(",")))

    def want(name):
        return not only or name in only

    if args.calibrate:
        src = torch.empty(256 * 1024 * 1024, device="cuda", dtype=torch.float16).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print("[bench] calibration copy: 5 x 512 MiB read + 512 MiB written",
              file=sys.stderr, flush=True)
        del src, dst

    c5 = C5(cx)
    call = c5.call(cx, workspace=True)
    # The other C5 measurements run first, so the timed loop below starts from
    # back-to-back calls (as in serving) rather than right after the 655 MB
    # fixture was generated; they follow a warm-up of their own.
    for _ in range(50):
        call()
    torch.cuda.synchronize()
    side = bench_packed_modes(cx, c5, "config 5 (the headline workload)")
    side.pop("workload")
    side.pop("bytes")
    side["reference_protocol_us"] = side["ws_us"]
    side["graph_replay_us"] = round(graph_replay_us(torch, lambda: c5.call(cx, workspace=True),
                                                    c5.out), 3)
    for _ in range(args.warmup):
        call()
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    stop = torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(args.steps):
        call()
    stop.record()
    torch.cuda.synchronize()
    ms = start.elapsed_time(stop) / args.steps
    gbs = c5.bytes / (ms * 1e-3) / 1e9
    print(f"[bench] C5 packed decode: {ms * 1e3:.2f} us/call, {gbs:.0f} GB/s "
          f"({100 * gbs / HBM_PEAK_GBS:.1f}% of 8 TB/s)", file=sys.stderr, flush=True)

    results = {}
    results["c5_packed_decode"] = {
        "us": round(ms * 1e3, 3), "bytes": c5.bytes, "gbs": round(gbs, 1),
        "pct_peak": round(100 * gbs / HBM_PEAK_GBS, 1), **side,
    }
    results["c5_paged_decode"] = bench_c5_paged(cx, c5)
    print(f"[bench] C5 paged {results['c5_paged_decode']}", file=sys.stderr, flush=True)
    if want("long"):
        lp = LongPacked(cx)
        results["packed_1x32k"] = bench_packed_modes(
            cx, lp, "packed decode, one sequence of 32768 tokens, 32/8 heads, D=128")
        print(f"[bench] packed 1 x 32K {results['packed_1x32k']}", file=sys.stderr, flush=True)
        del lp
    if want("c1"):
        results["c1_decode"] = bench_c1(cx)
        print(f"[bench] C1 {results['c1_decode']}", file=sys.stderr, flush=True)
    if want("c2"):
        results["c2_tree"] = bench_tree(cx, 1, 2048, 2, with_expanded=True)
        print(f"[bench] C2 {results['c2_tree']}", file=sys.stderr, flush=True)
    if want("c3"):
        results["c3_tree"] = bench_tree(cx, 8, 2053, 3, with_expanded=True)
        print(f"[bench] C3 {results['c3_tree']}", file=sys.stderr, flush=True)
    if want("tl"):
        # A large draft tree (beyond the benchmark configs): 8 requests x 256
        # nodes over a 2048-token shared prefix, where tree_rows_kernel shares
        # each K/V tile between four row tiles.
        results["tree_large"] = bench_tree(cx, 8, 2048, 4, with_expanded=False, nodes=256)
        print(f"[bench] tree 8 x 2048 x 256 nodes {results['tree_large']}", file=sys.stderr,
              flush=True)
    if want("c4"):
        results["c4_decode"] = bench_c4(cx)
        print(f"[bench] C4 {results['c4_decode']}", file=sys.stderr, flush=True)

    cpu = None
    if not args.no_cpu:
        host = (c5.q.cpu().numpy(), c5.cache.cpu().numpy(), c5.pages, c5.lengths,
                c5.strides, c5.bytes)
        cpu = cpu_baseline(host)
        print(f"[bench] CPU oracle {cpu}", file=sys.stderr, flush=True)

    line = {
        "metric": "decode µs/call + HBM GB/s (% peak); tree_verify µs at 8 req × 2048 prefix",
        "value": round(gbs, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) FP16 K/V/Q, random block tables)",
        "config": {
            "workload": ("benchmark config 5: packed-KV decode, batch 64, contexts "
                         "U[128,4096], 32 Q / 8 KV heads, D=128, cache [20000,2,16,8,128] "
                         "FP16, FP16 output"),
            "decode_us_per_call": round(ms * 1e3, 3),
            "pct_hbm_peak": round(100 * gbs / HBM_PEAK_GBS, 1),
            "tree_verify_us_8x2048": results.get("c3_tree", {}).get("tree_us"),
            "device": props.name,
            "cus": cx.cus,
        },
        "roofline": {
            "bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": C5_HBM_TRAFFIC_BYTES,
            "traffic_source": "rocprofv3 FETCH_SIZE (x2) + WRITE_SIZE (x1) per call, scaled "
                              "by a 512 MiB copy; profiles/packed_decode_c5_hbm_traffic.md",
            "kernel": ("paged_attn_kernel<128,_Float16,true,4> + merge_kernel<128,_Float16,1,false,false> "
                       "(one bc_packed_decode_ws call; achieved = algorithmic bytes / "
                       "HIP-event time per call on the launch stream)"),
            "algorithmic_bytes_per_launch": c5.bytes,
        },
        "cpu_baseline": cpu,
        "results": results,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
