"""Tree verification (bc_tree_verify[_ws]) against the CPU oracle.

Restates the reference driver's tree cases (src/main.cu:252-262: prefix
{0, 17, 257}, B=2, N=7, binary parents, 3e-4), the reference torch test
(tests/test_torch_ops.py:16-53), benchmark configs 2 and 3, deep/wide trees
over several MFMA row and draft tiles, and the invariant that the tree
output equals paged decode over the expanded-prefix fixture
(src/main.cu:375-423, 457-463).
"""

import numpy as np
import pytest

from oracle import oracle_np
import branchcraft_capi as capi
import gpu_helpers as G

pytestmark = pytest.mark.gpu


def _check(fix, oracle, atol=3e-4, what=""):
    """bc_tree_verify and bc_tree_verify_ws."""
    k, v, pages, lengths, dq, dk, dv, par = fix
    expected = oracle.tree(k, v, pages, lengths, dq, dk, dv, par, threads=16)
    for ws in (False, True):
        out = G.tree(k, v, pages, lengths, dq, dk, dv, par, workspace=ws)
        G.gate(out, expected, atol, f"{what} workspace={ws}")
    return expected


@pytest.mark.parametrize("prefix,dim", [(0, 64), (17, 64), (257, 128)])
def test_reference_tree_cases(prefix, dim, oracle):
    rng = np.random.default_rng(31)
    fix = oracle_np.tree_fixture(rng, 2, prefix, 7, d=dim)
    _check(fix, oracle, what=f"prefix={prefix}")


@pytest.mark.parametrize("dim", [64, 128])
def test_reference_torch_tree_case(dim, oracle):
    rng = np.random.default_rng(7)
    batch, nodes, hq, hkv = 2, 7, 4, 2
    dq = rng.standard_normal((batch, nodes, hq, dim)).astype(np.float16)
    k = rng.standard_normal((7, 16, hkv, dim)).astype(np.float16)
    v = rng.standard_normal((7, 16, hkv, dim)).astype(np.float16)
    pages = np.array([[4, 1], [5, 2]], dtype=np.int32)
    lengths = np.array([23, 0], dtype=np.int32)
    dk = rng.standard_normal((batch, nodes, hkv, dim)).astype(np.float16)
    dv = rng.standard_normal((batch, nodes, hkv, dim)).astype(np.float16)
    par = np.array([[-1, 0, 0, 1, 1, 2, 2]] * batch, dtype=np.int32)
    exp = _check((k, v, pages, lengths, dq, dk, dv, par), oracle, atol=3e-4)
    closed = oracle_np.tree(k, v, pages, lengths, dq, dk, dv, par)
    G.gate(exp, closed, 1e-5, "oracle vs closed form")


def test_config2_single_request_2048(oracle):
    rng = np.random.default_rng(2)
    fix = oracle_np.tree_fixture(rng, 1, 2048, 7, sigma=1.0, parents="random")
    _check(fix, oracle, atol=3e-4, what="config2")


def test_config3_eight_requests_shared_partial_prefix(oracle):
    rng = np.random.default_rng(3)
    fix = oracle_np.tree_fixture(rng, 8, 2053, 7, sigma=1.0, parents="random")
    _check(fix, oracle, atol=3e-4, what="config3")


@pytest.mark.parametrize("nodes,hq,hkv", [(40, 32, 8), (256, 8, 8), (33, 4, 2)])
def test_wide_trees_span_row_and_draft_tiles(nodes, hq, hkv, oracle):
    rng = np.random.default_rng(nodes)
    fix = oracle_np.tree_fixture(rng, 2, 70, nodes, hq=hq, hkv=hkv, d=128,
                                 parents="random")
    _check(fix, oracle, atol=3e-4, what=f"N={nodes}")


@pytest.mark.parametrize("hq,hkv,d,prefix", [(8, 8, 128, 300), (32, 1, 64, 129),
                                             (48, 3, 64, 517), (20, 4, 128, 33)])
def test_head_layouts_beyond_reference(hq, hkv, d, prefix, oracle):
    """Group 1 (7 rows per KV head), group 32 (224 rows: seven row tiles),
    group 16 and group 5 (35 rows: a second, mostly empty row tile)."""
    rng = np.random.default_rng(hq + 13 * hkv + d + prefix)
    fix = oracle_np.tree_fixture(rng, 3, prefix, 7, hq=hq, hkv=hkv, d=d, parents="random")
    _check(fix, oracle, atol=3e-4, what=f"Hq={hq} Hkv={hkv} D={d}")


def test_tree_equals_expanded_decode(oracle):
    rng = np.random.default_rng(91)
    k, v, pages, lengths, dq, dk, dv, par = oracle_np.tree_fixture(rng, 4, 300, 7,
                                                                   parents="random")
    tree = G.tree(k, v, pages, lengths, dq, dk, dv, par)
    el, ep, ek, ev = oracle.expand_tree(k, v, pages, lengths, dk, dv, par)
    b, n, hq, d = dq.shape
    flat = G.decode(dq.reshape(b * n, hq, d), ek, ev, ep, el, 1)
    G.gate(flat.reshape(tree.shape), tree, 3e-4, "tree vs expanded decode")


def test_garbage_past_prefix_is_ignored(oracle):
    rng = np.random.default_rng(12)
    k, v, pages, lengths, dq, dk, dv, par = oracle_np.tree_fixture(rng, 2, 37, 7)
    expected = oracle.tree(k, v, pages, lengths, dq, dk, dv, par)
    last = pages[0, 37 // 16]
    k[last, 37 % 16:] = np.float16(np.nan)
    v[last, 37 % 16:] = np.float16(np.inf)
    for ws in (False, True):
        G.gate(G.tree(k, v, pages, lengths, dq, dk, dv, par, workspace=ws), expected, 3e-4,
               f"garbage slots workspace={ws}")


def test_mid_batch_splits_the_prefix(oracle):
    """Sixteen requests over 1,400 tokens: 128 (request, KV head, row tile)
    units of 45 tiles, so the workspace call splits each unit's tiles over
    several workgroups and merges their partials."""
    rng = np.random.default_rng(16)
    fix = oracle_np.tree_fixture(rng, 16, 1400, 7, parents="random")
    k, v, pages, lengths, dq, dk, dv, par = fix
    b, n, hq, d = dq.shape
    shape = capi.Shape(b, hq, k.shape[2], d, pages.shape[1], k.shape[0])
    assert G.lib().bc_tree_verify_workspace_size(shape, n) > 0
    _check(fix, oracle, atol=3e-4, what="B=16")


@pytest.mark.parametrize("batch,nodes,hq,hkv,d", [(8, 128, 32, 8, 128), (8, 64, 64, 8, 64)])
def test_large_trees_share_tiles_across_row_tiles(batch, nodes, hq, hkv, d, oracle):
    """Trees of 16 row tiles per (request, KV head) whose groups of four row
    tiles fill the CUs (8 requests x 8 KV heads x 4 groups) take
    tree_rows_kernel, which loads each K/V tile once for four row tiles
    (the workspace entry point runs it too: it needs no workspace)."""
    rng = np.random.default_rng(nodes + d)
    fix = oracle_np.tree_fixture(rng, batch, 300, nodes, hq=hq, hkv=hkv, d=d,
                                 parents="random")
    _check(fix, oracle, atol=3e-4, what=f"B={batch} N={nodes} D={d}")


def _group_fixture(rng, lengths, share, nodes=7, hq=32, hkv=8, d=128, cow_last=(),
                   extra_pages=1):
    """Per-request prefixes over one page pool.  Request i reuses request
    share[i]'s page ids (share[i] < i) over the pages both cover and takes
    fresh pages beyond; share[i] = -1 gives it fresh pages throughout.
    Requests in `cow_last` then get a fresh last page, as a copy-on-write
    commit leaves them."""
    lengths = np.asarray(lengths, dtype=np.int32)
    batch = len(lengths)
    npg = [-(-int(x) // 16) for x in lengths]
    max_pages = max(max(npg), 1) + extra_pages
    pool = sum(npg) + len(cow_last) + 8
    _, k, v, _, _ = oracle_np.paged_fixture(rng, 1, hq, hkv, d, [16], pool=pool, sigma=1.0)
    fresh = iter(rng.permutation(pool).astype(np.int32))
    pages = np.full((batch, max_pages), -1, dtype=np.int32)
    for i in range(batch):
        j = share[i]
        for p in range(npg[i]):
            pages[i, p] = pages[j, p] if j >= 0 and p < npg[j] else next(fresh)
        if i in cow_last and npg[i] > 0:
            pages[i, npg[i] - 1] = next(fresh)
    dq = rng.standard_normal((batch, nodes, hq, d)).astype(np.float16)
    dk = rng.standard_normal((batch, nodes, hkv, d)).astype(np.float16)
    dv = rng.standard_normal((batch, nodes, hkv, d)).astype(np.float16)
    par = oracle_np.random_parents(rng, batch, nodes)
    return k, v, pages, lengths, dq, dk, dv, par


@pytest.mark.parametrize("case", [
    # every request on its own pages
    dict(lengths=[611, 95, 870, 402, 333, 777, 128, 640], share=[-1] * 8),
    # requests 1-3 share request 0's pages, request 3 ending early; 5-7
    # share request 4's, request 5 with a copied last page; 8 and 9 share
    # request 0's, 10 has its own (a last group of three)
    dict(lengths=[613, 613, 613, 400, 613, 613, 613, 613, 613, 613, 250],
         share=[-1, 0, 0, 0, -1, 4, 4, 4, 0, 0, -1], cow_last=(5,), extra_pages=42),
    # nine requests on one page table (a last group of one); the spare
    # page-table capacity of this and other short cases keeps them above
    # forty tiles, where the workspace call splits
    dict(lengths=[300] * 9, share=[-1] + [0] * 8, extra_pages=62),
    # empty requests beside sharing ones (their drafts give the output)
    dict(lengths=[300, 0, 300, 300, 300, 300, 0, 300], share=[-1] + [0] * 7, extra_pages=62),
    # page tables far longer than every request (empty prefix chunks)
    dict(lengths=[100] * 8, share=[-1] + [0] * 7, extra_pages=74),
    # D = 64, group 4, eight nodes (32 rows)
    dict(lengths=[517] * 8, share=[-1] + [0] * 7, nodes=8, hq=8, hkv=2, d=64),
    # group 1: 32 nodes fill the row tile and the draft tile
    dict(lengths=[290] * 8, share=[-1] + [0] * 7, nodes=32, hq=8, hkv=8, extra_pages=62),
    # five requests, two page tables
    dict(lengths=[613, 613, 400, 613, 613], share=[-1, 0, 0, -1, 3]),
])
def test_per_request_page_tables(case, oracle):
    """Requests whose page tables share some pages and not others, end at
    different lengths, hold a copied last page or are empty, with and
    without a workspace."""
    rng = np.random.default_rng(len(case["lengths"]) * 7 + sum(case["lengths"]))
    fix = _group_fixture(rng, **case)
    k, v, pages, lengths, dq, dk, dv, par = fix
    b, n, hq, d = dq.shape
    shape = capi.Shape(b, hq, k.shape[2], d, pages.shape[1], k.shape[0])
    assert G.lib().bc_tree_verify_workspace_size(shape, n) > 0
    _check(fix, oracle, atol=3e-4, what=str(case))


@pytest.mark.parametrize("case", [
    # 40 requests on one page table: 320 (request, KV head) units
    dict(lengths=[700] * 40, share=[-1] + [0] * 39),
    # 33 requests (the last workgroup holds one), mixed tables, empty requests
    dict(lengths=[611, 0, 870, 402, 333, 777, 128, 640, 95, 513, 513] * 3,
         share=[j + 11 * (i // 11) if j >= 0 else -1
                for i, j in enumerate([-1, -1, -1, 2, -1, 4, -1, 6, -1, 8, 9] * 3)],
         cow_last=(10, 21)),
    # D = 64 at 8 KV heads
    dict(lengths=[300] * 40, share=[-1] + [0] * 39, hq=32, hkv=8, d=64),
    # 16 nodes: two row tiles per (request, KV head), 1,024 units
    dict(lengths=[300] * 64, share=[-1] + [0] * 63, nodes=16),
])
def test_large_batches_pair_requests(case, oracle):
    """Batches with more (request, KV head) units than CUs run in one pass
    with two requests per workgroup (four waves each, walking the same
    tiles), with and without a workspace; 33 requests leave the last
    workgroup one."""
    rng = np.random.default_rng(len(case["lengths"]) * 11 + sum(case["lengths"]))
    fix = _group_fixture(rng, **case)
    _check(fix, oracle, atol=3e-4, what=f"B={len(case['lengths'])}")


def test_misaligned_workspace_is_ignored():
    """A workspace that is not 16-byte aligned is ignored: the call is
    bc_tree_verify's (whose split scratch is a slot of the library's pool)
    and gives its bits."""
    rng = np.random.default_rng(43)
    fix = oracle_np.tree_fixture(rng, 2, 600, 7, parents="random")
    k, v, pages, lengths, dq, dk, dv, par = fix
    b, n, hq, d = dq.shape
    shape = capi.Shape(b, hq, k.shape[2], d, pages.shape[1], k.shape[0])
    assert G.lib().bc_tree_verify_workspace_size(shape, n) > 0
    plain = G.tree(*fix, workspace=False)
    shifted = G.tree(*fix, workspace=True, ws_offset=4)
    assert np.array_equal(plain, shifted)


def test_malformed_parent_arrays_end_the_walk(oracle):
    """Parent arrays that do not form a tree (the reference walks them
    unbounded, src/tree_attention.cu:50-52): a 2-cycle, a self-loop, parents
    >= N and below -1, a parent after its child, every node its own parent
    and one cycle through all nodes.  Every kernel's walk is bounded by N
    steps and stops outside [0, N), so each row attends to the set of nodes
    its walk reaches, as the oracle's walk (which stops at the first repeat)
    does; both entry points run."""
    rng = np.random.default_rng(61)
    fix = list(oracle_np.tree_fixture(rng, 8, 300, 7, sigma=1.0, parents="random"))
    par = fix[7].copy()
    par[1] = [-1, 0, 3, 2, 1, 4, 5]      # nodes 2 <-> 3 form a cycle
    par[2, 4] = 4                        # self-loop
    par[3, 5], par[3, 6] = 7, 1000       # parents past the last node
    par[4, 1], par[4, 5] = 5, 0          # a parent after its child
    par[5] = np.arange(7)                # every node its own parent
    par[6, 3] = -7                       # negative, not -1
    par[7] = (np.arange(7) + 1) % 7      # one cycle through all nodes
    fix[7] = par.astype(np.int32)
    expected = _check(tuple(fix), oracle, what="malformed parents")
    # the oracle's own sets: node 3 of request 1 sees {3, 2}; request 7 sees all
    closed = oracle_np.tree(*fix)
    G.gate(expected, closed, 1e-5, "oracle vs closed form")


@pytest.mark.parametrize("offset", [2, 6])
def test_unaligned_tensors(offset, oracle):
    """FP16 tensors and the output shifted off 16-byte alignment (the
    reference accepts any `half*`): every entry point takes its element-wise
    path and matches the oracle."""
    import torch

    rng = np.random.default_rng(70 + offset)
    fix = oracle_np.tree_fixture(rng, 2, 300, 7, parents="random")
    k, v, pages, lengths, dq, dk, dv, par = fix
    expected = oracle.tree(*fix)
    b, n, hq, d = dq.shape

    def shifted(a):
        flat = torch.from_numpy(np.ascontiguousarray(a).reshape(-1)).cuda()
        buf = torch.empty(flat.numel() + 16, device="cuda", dtype=flat.dtype)
        view = buf[offset // flat.element_size():][:flat.numel()]
        view.copy_(flat)
        return view

    tk, tv, tq, tdk, tdv = (shifted(a) for a in (k, v, dq, dk, dv))
    assert tk.data_ptr() % 16 != 0
    tp = torch.from_numpy(pages).cuda()
    tl = torch.from_numpy(lengths).cuda()
    tpar = torch.from_numpy(par).cuda()
    obuf = torch.full((b * n * hq * d + 8,), float("nan"), device="cuda")
    out = obuf[1:1 + b * n * hq * d]
    shape = capi.Shape(b, hq, k.shape[2], d, pages.shape[1], k.shape[0])
    prefix = capi.Inputs(None, tk.data_ptr(), tv.data_ptr(), tp.data_ptr(), tl.data_ptr(), None)
    ins = capi.TreeInputs(prefix, tq.data_ptr(), tdk.data_ptr(), tdv.data_ptr(),
                          tpar.data_ptr(), out.data_ptr())
    L = G.lib()
    nbytes = L.bc_tree_verify_workspace_size(shape, n)
    ws = torch.empty(max(1, nbytes), device="cuda", dtype=torch.uint8)
    stream = G.stream()
    for name, call in (("bc_tree_verify", lambda: L.bc_tree_verify(shape, ins, n, stream)),
                       ("bc_tree_verify_ws", lambda: L.bc_tree_verify_ws(
                           shape, ins, n, ws.data_ptr(), nbytes, stream))):
        out.fill_(float("nan"))
        G.check(call(), name)
        torch.cuda.synchronize()
        G.gate(out.cpu().numpy().reshape(b, n, hq, d), expected, 3e-4, f"{name} offset={offset}")
