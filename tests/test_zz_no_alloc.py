"""bc_packed_decode_noalloc: bc_packed_decode_ws with its split workspace in
the library's static device array (no allocation in the call).

Two calls in a row through the C ABI -- benchmark config 5's shape, then a
smaller batch that reuses (and must not be disturbed by) the first call's
scratch contents -- each bit-identical to bc_packed_decode_ws on the same
inputs with a workspace from the caching allocator, and within the packed
decode tolerance of the CPU oracle.  The use the entry point is for, HIP
graph capture, runs in a fresh process whose first noalloc call is made
inside the capture (so the device address of the static array is looked up
there): every replay equals the eager workspace call bit for bit.
"""

import math
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest
import torch

import branchcraft_capi as capi
from oracle import oracle_c
import gpu_helpers as G

pytestmark = pytest.mark.gpu


def _case(rng, batch, pool, hkv=8, hq=32, d=128, lo=128, hi=4096):
    lens = rng.integers(lo, hi + 1, size=batch).astype(np.int32)
    maxp = int(-(-lens.max() // 16))
    perm = rng.permutation(pool).astype(np.int32)
    pages = np.full((batch, maxp), -1, dtype=np.int32)
    cur = 0
    for i, n in enumerate(lens):
        c = -(-int(n) // 16)
        pages[i, :c] = perm[cur:cur + c]
        cur += c
    q = rng.standard_normal((batch, hq, d)).astype(np.float16)
    return q, pages, lens


def _run(entry, shape, q, cache, pages, lens, strides, scale):
    tq, tp, tl = G.dev(q), G.dev(pages), G.dev(lens)
    out = torch.full(q.shape, float("nan"), device="cuda", dtype=torch.float16)
    L = G.lib()
    if entry == "noalloc":
        err = L.bc_packed_decode_noalloc(shape, tq.data_ptr(), cache.data_ptr(), tp.data_ptr(),
                                         tl.data_ptr(), out.data_ptr(), *strides, scale,
                                         G.stream())
    else:
        nbytes = L.bc_packed_decode_workspace_size(shape)
        ws = torch.empty(max(1, nbytes), device="cuda", dtype=torch.uint8)
        err = L.bc_packed_decode_ws(shape, tq.data_ptr(), cache.data_ptr(), tp.data_ptr(),
                                    tl.data_ptr(), out.data_ptr(), *strides, scale,
                                    ws.data_ptr(), nbytes, G.stream())
    G.check(err, entry)
    torch.cuda.synchronize()
    return out.cpu().numpy()


def test_noalloc_matches_workspace_entry_point_twice():
    rng = np.random.default_rng(55)
    pool, hkv, d = 20000, 8, 128
    cache = torch.randn((pool, 2, 16, hkv, d), device="cuda", dtype=torch.float16)
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    scale = 1 / math.sqrt(d)
    host_cache = None
    for batch in (64, 16):  # the second call is smaller
        q, pages, lens = _case(rng, batch, pool)
        shape = capi.Shape(batch, 32, hkv, d, pages.shape[1], pool)
        need = G.lib().bc_packed_decode_workspace_size(shape)
        assert 0 < need <= capi.BC_STATIC_SCRATCH_BYTES, need
        got = _run("noalloc", shape, q, cache, pages, lens, strides, scale)
        ref = _run("ws", shape, q, cache, pages, lens, strides, scale)
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), f"batch {batch}"
        if host_cache is None:
            host_cache = cache.cpu().numpy()
        exp32, _ = oracle_c.packed_decode(q, host_cache, pages, lens, strides, hkv, scale,
                                          threads=16)
        tol = G.f16_tolerance(exp32, 2e-3)
        assert np.all(np.abs(got.astype(np.float32) - exp32) <= tol), f"batch {batch}"


def test_noalloc_large_batches_use_pair_slots():
    """Batches above the 128 flat ranges (32/8 heads) split with two partial
    slots per range, 4.3 MB of the static array whatever the batch: 600
    short sequences, then 200 longer ones, each bit-identical to the
    workspace entry point and within tolerance of the oracle."""
    rng = np.random.default_rng(57)
    pool, hkv, d = 30000, 8, 128
    cache = torch.randn((pool, 2, 16, hkv, d), device="cuda", dtype=torch.float16)
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    scale = 1 / math.sqrt(d)
    host_cache = cache.cpu().numpy()
    for batch, lo, hi in ((600, 0, 300), (200, 100, 1500)):
        q, pages, lens = _case(rng, batch, pool, lo=lo, hi=hi)
        shape = capi.Shape(batch, 32, hkv, d, pages.shape[1], pool)
        need = G.lib().bc_packed_decode_workspace_size(shape)
        assert 0 < need <= capi.BC_STATIC_SCRATCH_BYTES, need
        got = _run("noalloc", shape, q, cache, pages, lens, strides, scale)
        ref = _run("ws", shape, q, cache, pages, lens, strides, scale)
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), f"batch {batch}"
        exp32, _ = oracle_c.packed_decode(q, host_cache, pages, lens, strides, hkv, scale,
                                          threads=16)
        tol = G.f16_tolerance(exp32, 2e-3)
        assert np.all(np.abs(got.astype(np.float32) - exp32) <= tol), f"batch {batch}"


def test_noalloc_unsplit_shape_and_oversize_rejection():
    """A short table runs unsplit (no scratch); an oversize shape returns
    hipErrorOutOfMemory and leaves the output untouched."""
    rng = np.random.default_rng(56)
    pool, hkv, d = 64, 2, 64
    cache = torch.randn((pool, 2, 16, hkv, d), device="cuda", dtype=torch.float16)
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    q, pages, lens = _case(rng, 3, pool, hkv=hkv, hq=8, d=d, lo=1, hi=300)
    shape = capi.Shape(3, 8, hkv, d, pages.shape[1], pool)
    assert G.lib().bc_packed_decode_workspace_size(shape) == 0
    got = _run("noalloc", shape, q, cache, pages, lens, strides, 0.125)
    ref = _run("ws", shape, q, cache, pages, lens, strides, 0.125)
    assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    big = capi.Shape(200, 128, 8, 128, 256, 20000)
    # The rejection happens before any launch only while the shape's split
    # workspace exceeds the static array; on a device where the shape would
    # run unsplit (workspace 0) the call would launch on the tiny buffers
    # below, so it is not made there.
    if G.lib().bc_packed_decode_workspace_size(big) <= capi.BC_STATIC_SCRATCH_BYTES:
        pytest.skip("the oversize shape does not split on this device")
    out = torch.full((4,), 7.0, device="cuda", dtype=torch.float16)
    err = G.lib().bc_packed_decode_noalloc(big, out.data_ptr(), out.data_ptr(), out.data_ptr(),
                                           out.data_ptr(), out.data_ptr(), 1, 1, 1, 1, 0.1,
                                           G.stream())
    assert err == capi.BC_ERROR_OUT_OF_MEMORY
    torch.cuda.synchronize()
    assert torch.all(out == 7.0)


_CAPTURE_SCRIPT = r"""
import math, sys
import numpy as np
import torch
sys.path[:0] = [sys.argv[1], sys.argv[2]]
import branchcraft_capi as capi
L = capi.load()
print("capture: inputs", flush=True)
rng = np.random.default_rng(57)
pool, hkv, hq, d, batch = 20000, 8, 32, 128, 64
cache = torch.randn((pool, 2, 16, hkv, d), device="cuda", dtype=torch.float16)
strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
lens = rng.integers(128, 4097, size=batch).astype(np.int32)
maxp = int(-(-lens.max() // 16))
perm = rng.permutation(pool).astype(np.int32)
pages = np.full((batch, maxp), -1, dtype=np.int32)
cur = 0
for i, n in enumerate(lens):
    c = -(-int(n) // 16)
    pages[i, :c] = perm[cur:cur + c]
    cur += c
q = torch.from_numpy(rng.standard_normal((batch, hq, d)).astype(np.float16)).cuda()
tp, tl = torch.from_numpy(pages).cuda(), torch.from_numpy(lens).cuda()
shape = capi.Shape(batch, hq, hkv, d, maxp, pool)
need = L.bc_packed_decode_workspace_size(shape)
assert 0 < need <= capi.BC_STATIC_SCRATCH_BYTES, need
scale = 1 / math.sqrt(d)
out = torch.full((batch, hq, d), float("nan"), device="cuda", dtype=torch.float16)
ref = torch.full_like(out, float("nan"))
ws = torch.empty(need, device="cuda", dtype=torch.uint8)
torch.cuda.synchronize()
print("capture: first noalloc call, inside the capture", flush=True)
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):
    err = L.bc_packed_decode_noalloc(shape, q.data_ptr(), cache.data_ptr(), tp.data_ptr(),
                                     tl.data_ptr(), out.data_ptr(), *strides, scale,
                                     torch.cuda.current_stream().cuda_stream)
assert err == capi.BC_SUCCESS, err
err = L.bc_packed_decode_ws(shape, q.data_ptr(), cache.data_ptr(), tp.data_ptr(),
                            tl.data_ptr(), ref.data_ptr(), *strides, scale, ws.data_ptr(), need,
                            torch.cuda.current_stream().cuda_stream)
assert err == capi.BC_SUCCESS, err
torch.cuda.synchronize()
want = ref.cpu().numpy().view(np.uint16)
for r in range(4):
    out.fill_(float("nan"))   # eager work between the replays
    g.replay()
    torch.cuda.synchronize()
    assert np.array_equal(out.cpu().numpy().view(np.uint16), want), f"replay {r}"
    print(f"capture: replay {r} matches", flush=True)
print("CAPTURE_OK", flush=True)
"""


def test_noalloc_first_call_inside_graph_capture_replays_bit_exact():
    """A fresh process makes its first bc_packed_decode_noalloc call inside
    torch.cuda.graph on the capture stream (benchmark config 5's shape, a
    split shape); four replays, with eager work between them, each equal
    bc_packed_decode_ws's output bit for bit."""
    root = Path(__file__).resolve().parent.parent
    env = dict(os.environ)
    proc = subprocess.run(
        [sys.executable, "-c", _CAPTURE_SCRIPT, str(root / "branchcraft-cuda_amd" / "python"),
         str(root)], capture_output=True, text=True, timeout=110, env=env)
    print(proc.stdout[-2000:], proc.stderr[-2000:])
    assert proc.returncode == 0 and "CAPTURE_OK" in proc.stdout
