"""torch.ops.branchcraft on PyTorch-ROCm: the reference's operator tests
(tests/test_torch_ops.py:16-114) with the CPU oracle as the expected value.

* tree_verify: ancestor mask against the oracle (D=64/128, lengths [23, 0]),
  torch.compile(inductor) equality and opcheck schema/FakeTensor checks;
  forked requests (one page table, a copied last page, a shorter request) and
  HIP-graph capture of the split kernel and its merge, replayed several times;
* packed_decode_out: HND and NHD-transposed caches and the 5-D
  [P, 2, 16, Hkv, D] layout, output aliasing, and HIP-graph capture replayed
  several times with eager work in between, every replay checked;
* commit_path_: the known-answer test and isolation of untouched slots;
* copy_pages_: bit-exact page clone.
All ops must run the HIP library (no CPU or Python fallback exists).
"""

import math

import numpy as np
import pytest
import torch

import branchcraft_capi as capi
import branchcraft_torch as bc
from oracle import oracle_c
import gpu_helpers as G

pytestmark = pytest.mark.gpu


def _tree_inputs(dim, device="cuda"):
    torch.manual_seed(7)
    batch, nodes, hq, hkv = 2, 7, 4, 2
    q = torch.randn(batch, nodes, hq, dim, device=device, dtype=torch.float16)
    prefix_k = torch.randn(7, 16, hkv, dim, device=device, dtype=torch.float16)
    prefix_v = torch.randn_like(prefix_k)
    pages = torch.tensor([[4, 1], [5, 2]], device=device, dtype=torch.int32)
    lengths = torch.tensor([23, 0], device=device, dtype=torch.int32)
    draft_k = torch.randn(batch, nodes, hkv, dim, device=device, dtype=torch.float16)
    draft_v = torch.randn_like(draft_k)
    parent = torch.tensor([[-1, 0, 0, 1, 1, 2, 2]] * batch, device=device, dtype=torch.int32)
    return q, prefix_k, prefix_v, pages, lengths, draft_k, draft_v, parent


@pytest.mark.parametrize("dim", [64, 128])
def test_tree_mask_compile_and_opcheck(dim):
    args = _tree_inputs(dim)
    actual = bc.tree_verify(*args)
    assert actual.dtype == torch.float32 and actual.shape == args[0].shape
    q, pk, pv, pages, lengths, dk, dv, parent = (a.cpu().numpy() for a in args)
    expected = oracle_c.tree(pk, pv, pages, lengths, q, dk, dv, parent)
    G.gate(actual.cpu().numpy(), expected, 3e-4, "tree_verify op")
    compiled = torch.compile(bc.tree_verify, backend="inductor")
    torch.testing.assert_close(compiled(*args), actual)
    torch.library.opcheck(torch.ops.branchcraft.tree_verify, args,
                          test_utils=("test_schema", "test_faketensor"))


def test_tree_verify_op_on_forked_requests():
    """Ten requests forked from one page table (as PagedTreeCache.fork
    leaves them), one with a copied last page and one shorter, against the
    oracle."""
    torch.manual_seed(8)
    batch, nodes, hq, hkv, dim = 10, 7, 8, 2, 128
    q = torch.randn(batch, nodes, hq, dim, device="cuda", dtype=torch.float16)
    prefix_k = torch.randn(40, 16, hkv, dim, device="cuda", dtype=torch.float16)
    prefix_v = torch.randn_like(prefix_k)
    row = torch.randperm(38, device="cuda").to(torch.int32)[:30]
    pages = row.repeat(batch, 1)
    pages[3, 29] = 38  # a copy-on-write clone of the last page
    lengths = torch.full((batch,), 470, device="cuda", dtype=torch.int32)
    lengths[6] = 301
    draft_k = torch.randn(batch, nodes, hkv, dim, device="cuda", dtype=torch.float16)
    draft_v = torch.randn_like(draft_k)
    parent = torch.tensor([[-1, 0, 0, 1, 1, 2, 2]] * batch, device="cuda", dtype=torch.int32)
    args = (q, prefix_k, prefix_v, pages, lengths, draft_k, draft_v, parent)
    actual = bc.tree_verify(*args)
    assert actual.dtype == torch.float32 and actual.shape == q.shape
    qn, pk, pv, pg, ln, dk, dv, par = (a.cpu().numpy() for a in args)
    expected = oracle_c.tree(pk, pv, pg, ln, qn, dk, dv, par, threads=8)
    G.gate(actual.cpu().numpy(), expected, 3e-4, "tree_verify op, forked requests")


def test_tree_verify_graph_replay():
    """tree_verify captured in a HIP graph: the split kernel and its merge
    (8 requests x 1400 tokens take several parts per (request, KV head)) with
    the output and workspace from the graph's pool, replayed with eager work
    in between; every replay equals the eager call bit for bit, which
    matches the oracle."""
    torch.manual_seed(21)
    batch, nodes, hq, hkv, dim = 8, 7, 32, 8, 128
    q = torch.randn(batch, nodes, hq, dim, device="cuda", dtype=torch.float16)
    prefix_k = torch.randn(92, 16, hkv, dim, device="cuda", dtype=torch.float16)
    prefix_v = torch.randn_like(prefix_k)
    pages = torch.randperm(92, device="cuda").to(torch.int32)[:88].repeat(batch, 1)
    lengths = torch.full((batch,), 1400, device="cuda", dtype=torch.int32)
    draft_k = torch.randn(batch, nodes, hkv, dim, device="cuda", dtype=torch.float16)
    draft_v = torch.randn_like(draft_k)
    parent = torch.tensor([[-1, 0, 0, 1, 1, 2, 2]] * batch, device="cuda", dtype=torch.int32)
    args = (q, prefix_k, prefix_v, pages, lengths, draft_k, draft_v, parent)
    shape = capi.Shape(batch, hq, hkv, dim, pages.shape[1], prefix_k.shape[0])
    assert G.lib().bc_tree_verify_workspace_size(shape, nodes) > 0  # split + merge
    eager = bc.tree_verify(*args)
    qn, pk, pv, pg, ln, dk, dv, par = (a.cpu().numpy() for a in args)
    expected = oracle_c.tree(pk, pv, pg, ln, qn, dk, dv, par, threads=8)
    G.gate(eager.cpu().numpy(), expected, 3e-4, "tree_verify eager")
    bc.tree_verify(*args)  # warm the allocator outside capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = bc.tree_verify(*args)
    for i in range(4):
        captured.fill_(float("nan"))
        junk = torch.randn(1024, 1024, device="cuda").sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager), f"replay {i}"
        del junk


def _packed_case(layout, dim=64):
    torch.manual_seed(11)
    batch, hq, hkv = 3, 8, 2
    if layout == "HND":
        cache = torch.randn(9, hkv, 16, 2 * dim, device="cuda", dtype=torch.float16)
        strides = (cache.stride(0), cache.stride(1), cache.stride(2), dim)
    elif layout == "NHD":
        cache = torch.randn(9, 16, hkv, 2 * dim, device="cuda",
                            dtype=torch.float16).transpose(1, 2)
        strides = (cache.stride(0), cache.stride(1), cache.stride(2), dim)
    else:  # [P, 2, 16, Hkv, D]
        cache = torch.randn(9, 2, 16, hkv, dim, device="cuda", dtype=torch.float16)
        strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    q = torch.randn(batch, hq, dim, device="cuda", dtype=torch.float16)
    pages = torch.tensor([[4, 1], [2, 7], [8, 6]], device="cuda", dtype=torch.int32)
    lengths = torch.tensor([23, 9, 0], device="cuda", dtype=torch.int32)
    # the oracle reads the storage through the same element strides
    storage = cache.as_strided((cache.untyped_storage().nbytes() // 2,), (1,))
    exp32, _ = oracle_c.packed_decode(q.cpu().numpy(), storage.cpu().numpy(),
                                      pages.cpu().numpy(), lengths.cpu().numpy(), strides,
                                      hkv, 1 / math.sqrt(dim))
    return q, cache, pages, lengths, exp32


@pytest.mark.parametrize("layout", ["HND", "NHD", "P2SHD"])
def test_packed_decode_layouts_and_graph_replay(layout):
    q, cache, pages, lengths, exp32 = _packed_case(layout)
    scale = 1 / math.sqrt(q.shape[-1])
    out = torch.empty_like(q)
    res = bc.packed_decode_out(q, cache, pages, lengths, out, scale)
    assert res.data_ptr() == out.data_ptr()
    tol = G.f16_tolerance(exp32, 2e-3)
    assert np.all(np.abs(out.cpu().numpy().astype(np.float32) - exp32) <= tol)
    assert torch.count_nonzero(out[2]) == 0
    # Capture on fixed allocations, then replay with eager work in between.
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        bc.packed_decode_out(q, cache, pages, lengths, out, scale)
    for i in range(4):
        out.fill_(float("nan"))
        junk = torch.randn(1024, 1024, device="cuda").sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        assert np.all(np.abs(out.cpu().numpy().astype(np.float32) - exp32) <= tol), f"replay {i}"
        del junk


def test_packed_decode_concurrent_streams():
    """Calls on two streams at once, each with its own workspace from the
    caching allocator, give the same bits as the same calls one at a time.
    An 80-column page table takes the split path (workspace and merge)."""
    torch.manual_seed(23)
    batch, hq, hkv, dim, pool = 8, 8, 2, 64, 700
    cache = torch.randn(pool, 2, 16, hkv, dim, device="cuda", dtype=torch.float16)
    gen = np.random.default_rng(23)
    pages = torch.from_numpy(
        np.stack([gen.permutation(pool)[:80] for _ in range(batch)]).astype(np.int32)).cuda()
    lengths = torch.from_numpy(gen.integers(1000, 1281, size=batch).astype(np.int32)).cuda()
    qs = [torch.randn(batch, hq, dim, device="cuda", dtype=torch.float16) for _ in range(2)]
    scale = 1 / math.sqrt(dim)
    assert G.lib().bc_packed_decode_workspace_size(
        capi.Shape(batch, hq, hkv, dim, 80, pool)) > 0
    solo = [bc.packed_decode_out(q, cache, pages, lengths, torch.empty_like(q), scale)
            for q in qs]
    torch.cuda.synchronize()
    outs = [torch.full_like(q, float("nan")) for q in qs]
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for st in streams:
        st.wait_stream(torch.cuda.current_stream())
    for _ in range(5):
        for st, q, out in zip(streams, qs, outs):
            with torch.cuda.stream(st):
                bc.packed_decode_out(q, cache, pages, lengths, out, scale)
    torch.cuda.synchronize()
    for i in range(2):
        assert torch.equal(outs[i], solo[i]), f"stream {i}"


def test_packed_decode_opcheck():
    q, cache, pages, lengths, _ = _packed_case("HND")
    out = torch.empty_like(q)
    torch.library.opcheck(torch.ops.branchcraft.packed_decode_out,
                          (q, cache, pages, lengths, out, 0.125),
                          test_utils=("test_schema", "test_faketensor"))


def test_commit_known_answer_and_isolation():
    cache_k = torch.zeros(4, 16, 2, 64, device="cuda", dtype=torch.float16)
    cache_v = torch.zeros_like(cache_k)
    draft_k = torch.arange(3, device="cuda", dtype=torch.float16).view(1, 3, 1, 1) \
        .expand(1, 3, 2, 64).contiguous()
    draft_v = draft_k + 10
    path = torch.tensor([0, 2], device="cuda", dtype=torch.int32)
    dest_pages = torch.tensor([3, 3], device="cuda", dtype=torch.int32)
    dest_slots = torch.tensor([6, 7], device="cuda", dtype=torch.int32)
    bc.commit_path_(cache_k, cache_v, draft_k, draft_v, path, dest_pages, dest_slots, 0)
    torch.testing.assert_close(cache_k[3, 6], draft_k[0, 0])
    torch.testing.assert_close(cache_k[3, 7], draft_k[0, 2])
    torch.testing.assert_close(cache_v[3, 7], draft_v[0, 2])
    assert torch.count_nonzero(cache_k[:3]) == 0
    assert torch.count_nonzero(cache_k[3, 8:]) == 0
    torch.library.opcheck(torch.ops.branchcraft.commit_path_,
                          (cache_k, cache_v, draft_k, draft_v, path, dest_pages, dest_slots, 0),
                          test_utils=("test_schema", "test_faketensor"))


def test_copy_pages_bit_exact():
    torch.manual_seed(3)
    ck = torch.randn(6, 16, 8, 128, device="cuda", dtype=torch.float16)
    cv = torch.randn_like(ck)
    before_k, before_v = ck.clone(), cv.clone()
    bc.copy_pages_(ck, cv, torch.tensor([1, 4], device="cuda", dtype=torch.int32),
                   torch.tensor([5, 0], device="cuda", dtype=torch.int32))
    assert torch.equal(ck[5], before_k[1]) and torch.equal(cv[0], before_v[4])
    assert torch.equal(ck[1:5], before_k[1:5])


def test_op_argument_errors_raise():
    q, pk, pv, pages, lengths, dk, dv, parent = _tree_inputs(64)
    with pytest.raises(RuntimeError):
        bc.tree_verify(q.float(), pk, pv, pages, lengths, dk, dv, parent)  # dtype
    with pytest.raises(RuntimeError):
        bc.tree_verify(q, pk, pv, pages, lengths, dk, dv, parent[:, :3])  # shape
    with pytest.raises(RuntimeError):
        bc.tree_verify(q.cpu(), pk, pv, pages, lengths, dk, dv, parent)  # device


def test_commit_paths_op_and_opcheck():
    cache_k = torch.zeros(5, 16, 2, 64, device="cuda", dtype=torch.float16)
    cache_v = torch.zeros_like(cache_k)
    draft_k = torch.randn(2, 3, 2, 64, device="cuda", dtype=torch.float16)
    draft_v = torch.randn_like(draft_k)
    i32 = dict(device="cuda", dtype=torch.int32)
    args = (cache_k, cache_v, draft_k, draft_v, torch.tensor([0, 1, 1], **i32),
            torch.tensor([2, 0, 1], **i32), torch.tensor([4, 1, 1], **i32),
            torch.tensor([0, 7, 8], **i32))
    bc.commit_paths_(*args)
    assert torch.equal(cache_k[4, 0], draft_k[0, 2]) and torch.equal(cache_v[1, 8], draft_v[1, 1])
    assert torch.equal(cache_k[1, 7], draft_k[1, 0])
    assert torch.count_nonzero(cache_k[2:4]) == 0
    torch.library.opcheck(torch.ops.branchcraft.commit_paths_, args,
                          test_utils=("test_schema", "test_faketensor"))
