"""The reference-signature calls (no workspace argument) run the split path
through the library's scratch pool.

bc_packed_decode and bc_tree_verify have the reference's signatures
(include/branchcraft.hpp:55-56,70-74), which take no workspace.  Shapes that
split borrow a slot of the library's per-device scratch pool, so their
results are the workspace calls' bit for bit.  Overlapping calls on several
streams (more streams than slots) and from two host threads give the bits of
serial calls, and a call captured into a HIP graph runs the single pass
(no slot) within the oracle's tolerance on every replay.
"""

import math
import threading

import numpy as np
import pytest
import torch

from oracle import oracle_np
import branchcraft_capi as capi
import gpu_helpers as G

pytestmark = pytest.mark.gpu

HKV, HQ, D = 8, 32, 128


class Packed:
    """A packed-decode problem on the GPU: [P, 2, 16, Hkv, D] cache."""

    def __init__(self, rng, batch, lo, hi, pool):
        self.cache = torch.randn((pool, 2, 16, HKV, D), device="cuda", dtype=torch.float16)
        lens = rng.integers(lo, hi + 1, size=batch).astype(np.int32)
        maxp = int(-(-lens.max() // 16))
        perm = rng.permutation(pool).astype(np.int32)
        pages = np.full((batch, maxp), -1, dtype=np.int32)
        cur = 0
        for i, n in enumerate(lens):
            c = -(-int(n) // 16)
            pages[i, :c] = perm[cur:cur + c]
            cur += c
        self.q = G.dev(rng.standard_normal((batch, HQ, D)).astype(np.float16))
        self.pages, self.lens = G.dev(pages), G.dev(lens)
        self.strides = (self.cache.stride(0), self.cache.stride(3), self.cache.stride(2),
                        self.cache.stride(1))
        self.shape = capi.Shape(batch, HQ, HKV, D, maxp, pool)
        self.host = (rng, pages, lens)

    def out(self):
        return torch.full(tuple(self.q.shape), float("nan"), device="cuda", dtype=torch.float16)

    def call(self, out, stream, ws=None):
        L = G.lib()
        args = (self.shape, self.q.data_ptr(), self.cache.data_ptr(), self.pages.data_ptr(),
                self.lens.data_ptr(), out.data_ptr(), *self.strides, 1 / math.sqrt(D))
        if ws is None:
            G.check(L.bc_packed_decode(*args, stream), "bc_packed_decode")
        else:
            G.check(L.bc_packed_decode_ws(*args, ws.data_ptr(), ws.numel(), stream),
                    "bc_packed_decode_ws")


class Tree:
    def __init__(self, rng, batch, prefix):
        k, v, pages, lengths, dq, dk, dv, par = oracle_np.tree_fixture(
            rng, batch, prefix, 7, sigma=1.0, parents="random")
        self.np = (k, v, pages, lengths, dq, dk, dv, par)
        self.t = [G.dev(x) for x in (k, v, pages, lengths, dq, dk, dv, par)]
        b, n, hq, d = dq.shape
        self.shape = capi.Shape(b, hq, k.shape[2], d, pages.shape[1], k.shape[0])
        self.nodes = n

    def out(self):
        b, n, hq, d = self.np[4].shape
        return torch.full((b, n, hq, d), float("nan"), device="cuda", dtype=torch.float32)

    def call(self, out, stream, ws=None):
        tk, tv, tp, tl, tq, tdk, tdv, tpar = self.t
        prefix = capi.Inputs(None, tk.data_ptr(), tv.data_ptr(), tp.data_ptr(), tl.data_ptr(),
                             None)
        ins = capi.TreeInputs(prefix, tq.data_ptr(), tdk.data_ptr(), tdv.data_ptr(),
                              tpar.data_ptr(), out.data_ptr())
        L = G.lib()
        if ws is None:
            G.check(L.bc_tree_verify(self.shape, ins, self.nodes, stream), "bc_tree_verify")
        else:
            G.check(L.bc_tree_verify_ws(self.shape, ins, self.nodes, ws.data_ptr(), ws.numel(),
                                        stream), "bc_tree_verify_ws")


def _ws(nbytes):
    return torch.empty(max(1, nbytes), device="cuda", dtype=torch.uint8)


def _bits(t):
    return t.cpu().numpy().view(np.uint16 if t.dtype == torch.float16 else np.uint32)


@pytest.mark.parametrize("case", ["c5", "one_32k", "c4_like"])
def test_packed_reference_signature_equals_workspace_call(case):
    rng = np.random.default_rng({"c5": 51, "one_32k": 52, "c4_like": 53}[case])
    if case == "c5":
        p = Packed(rng, 64, 128, 4096, 20000)
    elif case == "one_32k":
        p = Packed(rng, 1, 32768, 32768, 4096)
    else:
        p = Packed(rng, 4, 16384, 32768, 8192)
    need = G.lib().bc_packed_decode_workspace_size(p.shape)
    assert 0 < need <= capi.BC_SCRATCH_SLOT_BYTES
    a, b = p.out(), p.out()
    p.call(a, G.stream())
    p.call(b, G.stream(), ws=_ws(need))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(a), _bits(b))
    assert torch.isfinite(a.float()).all()


@pytest.mark.parametrize("batch,prefix", [(1, 2048), (8, 2053), (12, 2048)])
def test_tree_reference_signature_equals_workspace_call(batch, prefix, oracle):
    rng = np.random.default_rng(batch * 7 + prefix)
    t = Tree(rng, batch, prefix)
    need = G.lib().bc_tree_verify_workspace_size(t.shape, t.nodes)
    assert 0 < need <= capi.BC_SCRATCH_SLOT_BYTES
    a, b = t.out(), t.out()
    t.call(a, G.stream())
    t.call(b, G.stream(), ws=_ws(need))
    torch.cuda.synchronize()
    assert np.array_equal(_bits(a), _bits(b))
    k, v, pages, lengths, dq, dk, dv, par = t.np
    expected = oracle.tree(k, v, pages, lengths, dq, dk, dv, par, threads=16)
    G.gate(a.cpu().numpy(), expected, 3e-4, "reference signature")


def _oracle_ok(p, t, out_p, out_t, oracle):
    """Both outputs within the oracle's tolerance (packed FP16: 2e-3 plus
    half an FP16 ulp; tree: 3e-4)."""
    _, pages, lens = p.host
    exp32, _ = oracle.packed_decode(p.q.cpu().numpy(), p.cache.cpu().numpy(), pages, lens,
                                    p.strides, HKV, 1 / math.sqrt(D), threads=16)
    got = out_p.cpu().numpy().astype(np.float32)
    assert np.all(np.abs(got - exp32) <= G.f16_tolerance(exp32, 2e-3))
    k, v, pages, lengths, dq, dk, dv, par = t.np
    G.gate(out_t.cpu().numpy(), oracle.tree(k, v, pages, lengths, dq, dk, dv, par, threads=16),
           3e-4, "tree")


def _stream_rounds(nstreams, rounds, seed):
    """nstreams streams, each with its own packed and tree problem: serial
    reference bits (default stream), then `rounds` rounds of back-to-back
    launches on every stream without synchronisation.  Returns the problems,
    per round and stream whether each output equals the serial bits, and
    every round's outputs."""
    rng = np.random.default_rng(seed)
    packs = [Packed(rng, 16, 1024, 4096, 4096) for _ in range(nstreams)]
    trees = [Tree(rng, 8, 2053) for _ in range(nstreams)]
    ref = []
    for p, t in zip(packs, trees):
        o1, o2 = p.out(), t.out()
        p.call(o1, G.stream())
        t.call(o2, G.stream())
        torch.cuda.synchronize()
        ref.append((_bits(o1), _bits(o2)))
    streams = [torch.cuda.Stream() for _ in range(nstreams)]
    same, all_outs = [], []
    for _ in range(rounds):
        outs = [(p.out(), t.out()) for p, t in zip(packs, trees)]
        all_outs.append(outs)
        torch.cuda.synchronize()
        for i, (p, t) in enumerate(zip(packs, trees)):
            s = streams[i].cuda_stream
            p.call(outs[i][0], s)
            t.call(outs[i][1], s)
        torch.cuda.synchronize()
        same.append([(np.array_equal(_bits(o[0]), ref[i][0]),
                      np.array_equal(_bits(o[1]), ref[i][1])) for i, o in enumerate(outs)])
    return packs, trees, same, all_outs


@pytest.mark.parametrize("nstreams", [2, 6])
def test_overlapping_calls_on_streams_are_correct(nstreams, oracle):
    """Overlapping reference-signature calls on several streams.  Each
    output either equals the serial call's bits (the split path through a
    slot) or, where the pool had no slot for that stream (every slot owned
    by another stream of this process, with no recorded use), is the single
    pass within the oracle's tolerance; a race on a slot would fit neither."""
    packs, trees, same, outs = _stream_rounds(nstreams, 3, 60 + nstreams)
    for rnd, row in enumerate(same):
        for i, (sp, st) in enumerate(row):
            if not (sp and st):
                _oracle_ok(packs[i], trees[i], outs[rnd][i][0], outs[rnd][i][1], oracle)


_SCHEDULE_SCRIPT = r"""
import sys
sys.path[:0] = sys.argv[1:4]
import numpy as np
import test_ref_signature_gpu as T
packs, trees, same, _ = T._stream_rounds(6, 4, 66)
for rnd, row in enumerate(same):
    print("round", rnd, [int(a and b) for a, b in row], flush=True)
# Fresh pool: the default stream owns slot 0 (serial phase), streams 0-2 take
# the free slots 1-3, stream 3 finds every slot owned and runs the single
# pass, which turns event recording on (streams 4 and 5 likewise); from
# round 1 on, slots pass between streams through their events.
assert [a and b for a, b in same[0][:3]] == [True] * 3, same[0]
for row in same[1:]:
    assert all(a and b for a, b in row), row
print("SCHEDULE_OK", flush=True)
"""


def test_slot_schedule_in_a_fresh_process():
    """From a fresh pool (a child process): six streams against four slots.
    The first round gives the serial bits on the three streams that find a
    free slot; every later round gives the serial bits on all six, the slots
    now passing between streams through their events."""
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parent.parent
    proc = subprocess.run(
        [sys.executable, "-c", _SCHEDULE_SCRIPT, str(root / "tests"),
         str(root / "branchcraft-cuda_amd" / "python"), str(root)],
        capture_output=True, text=True, timeout=110, env=dict(os.environ))
    print(proc.stdout[-2000:], proc.stderr[-2000:])
    assert proc.returncode == 0 and "SCHEDULE_OK" in proc.stdout


def test_calls_from_two_host_threads_match_serial_calls():
    rng = np.random.default_rng(71)
    packs = [Packed(rng, 16, 1024, 4096, 4096) for _ in range(2)]
    refs = []
    for p in packs:
        o = p.out()
        p.call(o, G.stream())
        torch.cuda.synchronize()
        refs.append(_bits(o))
    outs = [[p.out() for _ in range(12)] for p in packs]
    streams = [torch.cuda.Stream() for _ in packs]
    torch.cuda.synchronize()
    errors = []

    def work(i):
        try:
            for o in outs[i]:
                packs[i].call(o, streams[i].cuda_stream)
        except Exception as e:  # noqa: BLE001 - reported below
            errors.append(e)

    th = [threading.Thread(target=work, args=(i,)) for i in range(2)]
    for x in th:
        x.start()
    for x in th:
        x.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for i in range(2):
        for j, o in enumerate(outs[i]):
            assert np.array_equal(_bits(o), refs[i]), (i, j)


def test_captured_reference_signature_call_replays(oracle):
    """Under graph capture no slot is taken (its event could not order the
    replays): the captured call runs the single pass.  Every replay, with
    eager calls of the split path in between, equals the first replay's
    bits and the oracle within the packed tolerance."""
    rng = np.random.default_rng(81)
    p = Packed(rng, 16, 1024, 4096, 4096)
    assert G.lib().bc_packed_decode_workspace_size(p.shape) > 0
    out, other = p.out(), p.out()
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        p.call(out, torch.cuda.current_stream().cuda_stream)
    first = None
    for _ in range(3):
        out.fill_(float("nan"))
        g.replay()
        p.call(other, G.stream())  # eager: the split path through a slot
        torch.cuda.synchronize()
        bits = _bits(out)
        if first is None:
            first = bits
        assert np.array_equal(bits, first)
    _, pages, lens = p.host
    host = p.cache.cpu().numpy()
    exp32, _ = oracle.packed_decode(p.q.cpu().numpy(), host, pages, lens, p.strides, HKV,
                                      1 / math.sqrt(D), threads=16)
    got = out.cpu().numpy().astype(np.float32)
    assert np.all(np.abs(got - exp32) <= G.f16_tolerance(exp32, 2e-3))
    got2 = other.cpu().numpy().astype(np.float32)
    assert np.all(np.abs(got2 - exp32) <= G.f16_tolerance(exp32, 2e-3))
