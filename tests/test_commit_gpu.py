"""Commit path and copy-on-write page clone: bit-exact against the oracle.

Restates the reference's known-answer commit test
(tests/test_torch_ops.py:99-114), its transaction test
(tests/test_transaction.py:8-29) and the driver's commit / sibling /
rollback case (src/main.cu:264-313), and runs benchmark config 3's commit.
"""

import numpy as np
import pytest
import torch

from oracle import oracle_np
import gpu_helpers as G

pytestmark = pytest.mark.gpu


def test_known_answer_commit():
    cache_k = torch.zeros(4, 16, 2, 64, device="cuda", dtype=torch.float16)
    cache_v = torch.zeros_like(cache_k)
    draft_k = torch.arange(3, device="cuda", dtype=torch.float16).view(1, 3, 1, 1) \
        .expand(1, 3, 2, 64).contiguous()
    draft_v = draft_k + 10
    G.commit(cache_k, cache_v, draft_k, draft_v, [0, 2], [3, 3], [6, 7], 0)
    assert torch.equal(cache_k[3, 6], draft_k[0, 0])
    assert torch.equal(cache_k[3, 7], draft_k[0, 2])
    assert torch.equal(cache_v[3, 7], draft_v[0, 2])
    assert torch.count_nonzero(cache_k[:3]) == 0
    assert torch.count_nonzero(cache_k[3, 8:]) == 0


def test_random_commits_and_page_copies_bit_exact(oracle):
    rng = np.random.default_rng(21)
    P, hkv, d, b, n = 12, 8, 128, 3, 7
    ck = rng.standard_normal((P, 16, hkv, d)).astype(np.float16)
    cv = rng.standard_normal((P, 16, hkv, d)).astype(np.float16)
    dk = rng.standard_normal((b, n, hkv, d)).astype(np.float16)
    dv = rng.standard_normal((b, n, hkv, d)).astype(np.float16)
    tk, tv = G.dev(ck), G.dev(cv)
    tdk, tdv = G.dev(dk), G.dev(dv)
    # page clone first (src -> dst), then a commit with one out-of-range entry
    G.copy_pages(tk, tv, [4, 9], [10, 11])
    ek, ev = oracle.copy_pages(ck, cv, [4, 9], [10, 11])
    path, dpg, dsl = [0, 3, 5, 6], [10, 10, 99, 11], [3, 4, 5, 15]
    G.commit(tk, tv, tdk, tdv, path, dpg, dsl, 2)
    ek, ev = oracle.commit(ek, ev, dk, dv, path, dpg, dsl, 2)
    assert np.array_equal(tk.cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(tv.cpu().numpy().view(np.uint16), ev.view(np.uint16))


def _offset_copy(a: np.ndarray, elems: int) -> torch.Tensor:
    """A GPU copy of `a` whose data pointer sits `elems` FP16 elements past a
    16-byte boundary."""
    buf = torch.empty(a.size + 16, device="cuda", dtype=torch.float16)
    view = buf[elems:elems + a.size].view(a.shape)
    view.copy_(torch.from_numpy(a))
    assert view.data_ptr() % 16 != 0
    return view


@pytest.mark.parametrize("elems", [1, 3])
def test_unaligned_commits_and_page_copies_bit_exact(elems, oracle):
    """Cache and draft tensors 2 or 6 bytes off 16-byte alignment (the
    reference accepts any `half*`): bc_copy_pages, bc_commit_path and
    bc_commit_paths take their element-wise paths, bit-exact."""
    rng = np.random.default_rng(22 + elems)
    P, hkv, d, b, n = 12, 8, 64, 3, 7
    ck = rng.standard_normal((P, 16, hkv, d)).astype(np.float16)
    cv = rng.standard_normal((P, 16, hkv, d)).astype(np.float16)
    dk = rng.standard_normal((b, n, hkv, d)).astype(np.float16)
    dv = rng.standard_normal((b, n, hkv, d)).astype(np.float16)
    tk, tv = _offset_copy(ck, elems), _offset_copy(cv, elems)
    tdk, tdv = _offset_copy(dk, elems), _offset_copy(dv, elems)
    G.copy_pages(tk, tv, [4, 9], [10, 11])
    ek, ev = oracle.copy_pages(ck, cv, [4, 9], [10, 11])
    path, dpg, dsl = [0, 3, 5, 6], [10, 10, 99, 11], [3, 4, 5, 15]
    G.commit(tk, tv, tdk, tdv, path, dpg, dsl, 2)
    ek, ev = oracle.commit(ek, ev, dk, dv, path, dpg, dsl, 2)
    G.commit_paths(tk, tv, tdk, tdv, [0, 1], [2, 4], [3, 5], [0, 9])
    for req, node, page, slot in ((0, 2, 3, 0), (1, 4, 5, 9)):
        ek, ev = oracle.commit(ek, ev, dk, dv, [node], [page], [slot], req)
    assert np.array_equal(tk.cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(tv.cpu().numpy().view(np.uint16), ev.view(np.uint16))


def test_driver_commit_sibling_rollback(oracle):
    """src/main.cu:264-313: two requests share a 17-token prefix; clone the
    partial page to P-1, commit path {0,1,3} at slots {1,2,3}, and decode
    node 3's query over the committed cache: equals its tree output."""
    rng = np.random.default_rng(49)
    k, v, pages, lengths, dq, dk, dv, par = oracle_np.tree_fixture(rng, 2, 17, 7, d=128)
    tree_out = G.tree(k, v, pages, lengths, dq, dk, dv, par)
    q = dq[:, 0].copy()  # any query; the sibling check uses request 1
    before = G.decode(q, k, v, pages, lengths, 1)
    tk, tv = G.dev(k), G.dev(v)
    P = k.shape[0]
    new_page, old_page = P - 1, int(pages[0, 1])
    G.copy_pages(tk, tv, [old_page], [new_page])
    G.commit(tk, tv, G.dev(dk), G.dev(dv), [0, 1, 3], [new_page] * 3, [1, 2, 3], 0)
    ck, cv = tk.cpu().numpy(), tv.cpu().numpy()
    ek, ev = oracle.copy_pages(k, v, [old_page], [new_page])
    ek, ev = oracle.commit(ek, ev, dk, dv, [0, 1, 3], [new_page] * 3, [1, 2, 3], 0)
    assert np.array_equal(ck.view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(cv.view(np.uint16), ev.view(np.uint16))
    cpages, clens = pages.copy(), lengths.copy()
    cpages[0, 1] = new_page
    clens[0] += 3
    q2 = q.copy()
    q2[0] = dq[0, 3]
    after = G.decode(q2, ck, cv, cpages, clens, 1)
    G.gate(after[0], tree_out[0, 3], 3e-4, "accepted path replay")
    assert np.array_equal(after[1], before[1]), "sibling changed"
    rolled = G.decode(q, ck, cv, pages, lengths, 1)
    assert np.array_equal(rolled, before), "rollback changed the output"


def test_transaction_shared_partial_page_then_rollback():
    """tests/test_transaction.py:8-29 of the reference."""
    from branchcraft_torch.transaction import PagedTreeCache
    torch.manual_seed(17)
    store = PagedTreeCache(8, 2, 64)
    prefix_k = torch.randn(19, 2, 64, device="cuda", dtype=torch.float16)
    prefix_v = torch.randn_like(prefix_k)
    original = store.new(prefix_k, prefix_v)
    sibling = store.fork(original)
    snapshot = store.checkpoint(original)
    initial_pages = store.pages[original].copy()
    old_bytes = store.k[initial_pages[-1]].clone()
    draft_k = torch.randn(1, 7, 2, 64, device="cuda", dtype=torch.float16)
    draft_v = torch.randn_like(draft_k)
    store.commit(original, [0, 2, 6], draft_k, draft_v)
    torch.cuda.synchronize()
    assert store.pages[original][-1] != store.pages[sibling][-1]
    assert store.lengths[original] == 22
    assert torch.equal(store.k[store.pages[original][-1], 3], draft_k[0, 0])
    assert torch.equal(store.k[store.pages[original][-1], 5], draft_k[0, 6])
    assert torch.equal(store.k[store.pages[sibling][-1]], old_bytes)
    # the clone carried the three prefix tokens of the partial page
    assert torch.equal(store.k[store.pages[original][-1], :3], old_bytes[:3])
    store.rollback(snapshot)
    assert store.pages[original] == initial_pages
    assert store.lengths[original] == 19
    assert torch.equal(store.k[store.pages[original][-1]], old_bytes)


def test_config3_commit_bit_exact(oracle):
    """benchmark config 3: 8 requests share a 2053-token prefix (last page
    holds 5 tokens); each commits a random root-to-leaf path; every request
    clones the shared partial page."""
    from branchcraft_torch.transaction import PagedTreeCache
    rng = np.random.default_rng(33)
    hkv, d, n = 8, 128, 7
    store = PagedTreeCache(129 + 8 * 2 + 4, hkv, d)
    pk = rng.standard_normal((2053, hkv, d)).astype(np.float16)
    pv = rng.standard_normal((2053, hkv, d)).astype(np.float16)
    root = store.new(G.dev(pk), G.dev(pv))
    reqs = [root] + [store.fork(root) for _ in range(7)]
    par = oracle_np.random_parents(rng, 8, n)
    ref_k, ref_v = store.k.cpu().numpy(), store.v.cpu().numpy()
    tables_before = {r: list(store.pages[r]) for r in reqs}
    for i, r in enumerate(reqs):
        snap = store.checkpoint(r)
        leaves = [x for x in range(n) if x not in set(par[i].tolist())]
        leaf = int(rng.choice(leaves))
        path = oracle_np.ancestors(par[i], leaf)[::-1]
        dk = rng.standard_normal((1, n, hkv, d)).astype(np.float16)
        dv = rng.standard_normal((1, n, hkv, d)).astype(np.float16)
        plan = store.commit(r, path, G.dev(dk), G.dev(dv))
        assert plan.cow is not None and plan.cow[0] == tables_before[r][-1]
        ref_k, ref_v = oracle.copy_pages(ref_k, ref_v, [plan.cow[0]], [plan.cow[1]])
        ref_k, ref_v = oracle.commit(ref_k, ref_v, dk, dv, path, plan.dest_pages,
                                     plan.dest_slots, 0)
        store.accept(snap)
        assert store.lengths[r] == 2053 + len(path)
        assert store.pages[r][:-1] == tables_before[r][:-1]
    torch.cuda.synchronize()
    assert np.array_equal(store.k.cpu().numpy().view(np.uint16), ref_k.view(np.uint16))
    assert np.array_equal(store.v.cpu().numpy().view(np.uint16), ref_v.view(np.uint16))
    store.owner.check_invariants()


def test_commit_paths_equals_per_request_commits(oracle):
    """bc_commit_paths (one launch for several requests, with skipped
    out-of-range entries) against the oracle's per-request commits."""
    rng = np.random.default_rng(77)
    P, hkv, d, b, n = 20, 8, 64, 4, 9
    ck = rng.standard_normal((P, 16, hkv, d)).astype(np.float16)
    cv = rng.standard_normal((P, 16, hkv, d)).astype(np.float16)
    dk = rng.standard_normal((b, n, hkv, d)).astype(np.float16)
    dv = rng.standard_normal((b, n, hkv, d)).astype(np.float16)
    reqs = [0, 0, 1, 3, 3, 3, 2, 5, 1]          # request 5 is out of range
    nodes = [0, 4, 2, 8, 1, 0, 7, 0, 9]          # node 9 is out of range
    dpg = [2, 2, 7, 11, 11, 12, 19, 3, 4]
    dsl = [0, 1, 15, 4, 5, 6, 9, 2, 3]
    tk, tv = G.dev(ck), G.dev(cv)
    G.commit_paths(tk, tv, G.dev(dk), G.dev(dv), reqs, nodes, dpg, dsl)
    ek, ev = ck, cv
    for r, x, p, s_ in zip(reqs, nodes, dpg, dsl):
        if r < b:
            ek, ev = oracle.commit(ek, ev, dk, dv, [x], [p], [s_], r)
    assert np.array_equal(tk.cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(tv.cpu().numpy().view(np.uint16), ev.view(np.uint16))


def _shared_store(seed):
    from branchcraft_torch.transaction import PagedTreeCache
    rng = np.random.default_rng(seed)
    hkv, d = 2, 64
    store = PagedTreeCache(40, hkv, d)
    pk = G.dev(rng.standard_normal((37, hkv, d)).astype(np.float16))
    pv = G.dev(rng.standard_normal((37, hkv, d)).astype(np.float16))
    root = store.new(pk, pv)
    reqs = [root, store.fork(root), store.fork(root)]
    other = store.new(pk[:16], pv[:16])  # full last page: no clone
    return store, reqs + [other]


def test_commit_many_matches_sequential_commits():
    """Two launches for all requests leave the same pages, lengths and page
    bytes as one commit per request in the same order (shared partial page
    cloned by the first two requests, written in place by the last sharer,
    appended to a full page for the fourth)."""
    rng = np.random.default_rng(5)
    paths = [[0, 3, 4], [0, 1], [0, 2, 5, 6, 8, 1, 7, 3, 4, 10, 11, 9], [0, 4]]
    dk = G.dev(rng.standard_normal((4, 12, 2, 64)).astype(np.float16))
    dv = G.dev(rng.standard_normal((4, 12, 2, 64)).astype(np.float16))
    seq, reqs = _shared_store(3)
    seq_plans = [seq.commit(r, p, dk[i:i + 1].contiguous(), dv[i:i + 1].contiguous())
                 for i, (r, p) in enumerate(zip(reqs, paths))]
    bat, reqs2 = _shared_store(3)
    plans = bat.commit_many(reqs2, paths, dk, dv)
    torch.cuda.synchronize()
    assert [p.cow for p in plans] == [p.cow for p in seq_plans]
    assert plans[0].cow is not None and plans[2].cow is None  # last sharer writes in place
    assert bat.pages == seq.pages and bat.lengths == seq.lengths
    assert bat.refcount == seq.refcount and bat.free == seq.free
    assert torch.equal(bat.k.view(torch.int16), seq.k.view(torch.int16))
    assert torch.equal(bat.v.view(torch.int16), seq.v.view(torch.int16))


def test_commit_many_runs_planned_work_before_pool_error():
    from branchcraft_torch.transaction import PagedTreeCache
    store = PagedTreeCache(3, 2, 64)
    pk = torch.randn(15, 2, 64, device="cuda", dtype=torch.float16)
    a = store.new(pk, pk)
    b = store.new(pk, pk)
    dk = torch.randn(2, 20, 2, 64, device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError):
        store.commit_many([a, b], [[0], list(range(20))], dk, dk)
    torch.cuda.synchronize()
    assert store.lengths[a] == 16 and store.lengths[b] == 15
    assert torch.equal(store.k[store.pages[a][0], 15], dk[0, 0])
