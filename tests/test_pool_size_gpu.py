"""Calls that do not give the page pool's size, as the reference allows.

The reference's tree_verify and commit_path check no pool size
(src/tree_attention.cu:93-122), and its op passes prefix_k.size(0) and
cache_k.size(0) as physical_pages (bindings/torch_ops.cpp:54,131), which is 0
for an empty pool.  Here physical_pages < 1 means "not given":

- a tree over an empty pool with every length 0 is draft-only attention,
  through both C entry points and the op over a 0-page view of a pool;
- a tree over a real pool whose size is not given trusts the page ids inside
  each length, as the reference does, and reads nothing outside them;
- commits with physical_pages = 0 write the same bytes as with the size;
- kv_heads = 0 copies nothing.

Each result is gated against the oracle (3e-4 for trees, bit-exact for
commits).
"""

import numpy as np
import pytest
import torch

from oracle import oracle_np
import branchcraft_torch  # noqa: F401  (registers the ops)
import gpu_helpers as G

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dim", [64, 128])
def test_empty_pool_gives_draft_only_attention(dim, oracle):
    rng = np.random.default_rng(40 + dim)
    b, n, hq, hkv = 3, 7, 32, 8
    _, _, _, _, dq, dk, dv, par = oracle_np.tree_fixture(rng, b, 0, n, hq=hq, hkv=hkv, d=dim,
                                                         sigma=1.0, parents="random")
    lengths = np.zeros(b, dtype=np.int32)
    pages = np.full((b, 4), 1 << 30, dtype=np.int32)  # never dereferenced
    empty = np.zeros((0, 16, hkv, dim), dtype=np.float16)
    expected = oracle.tree(empty, empty, pages, lengths, dq, dk, dv, par)
    closed = oracle_np.tree(empty, empty, pages, lengths, dq, dk, dv, par)
    G.gate(expected, closed, 1e-5, "oracle vs closed form")
    # C ABI: physical_pages = 0 and a pool buffer of NaN that must not be read
    nan_pool = np.full((1, 16, hkv, dim), np.nan, dtype=np.float16)
    for ws in (False, True):
        out = G.tree(nan_pool, nan_pool, pages, lengths, dq, dk, dv, par, workspace=ws,
                     phys_pages=0)
        G.gate(out, expected, 3e-4, f"empty pool workspace={ws}")
    # The op over a 0-page view of a pool (a non-null data pointer)
    pool = torch.full((2, 16, hkv, dim), float("nan"), device="cuda", dtype=torch.float16)
    out = torch.ops.branchcraft.tree_verify(
        G.dev(dq), pool[:0], pool[:0], G.dev(pages), G.dev(lengths), G.dev(dk), G.dev(dv),
        G.dev(par))
    torch.cuda.synchronize()
    G.gate(out.cpu().numpy(), expected, 3e-4, "op over a 0-page pool view")


def test_op_rejects_a_null_pool_like_the_reference():
    """A freshly allocated 0-page tensor has no storage (a null data
    pointer), which the reference's null check rejects
    (src/tree_attention.cu:97): the op raises."""
    hkv, d = 2, 64
    q = torch.zeros(1, 1, 4, d, device="cuda", dtype=torch.float16)
    empty = torch.empty(0, 16, hkv, d, device="cuda", dtype=torch.float16)
    assert empty.data_ptr() == 0
    dk = torch.zeros(1, 1, hkv, d, device="cuda", dtype=torch.float16)
    with pytest.raises(RuntimeError, match="invalid argument"):
        torch.ops.branchcraft.tree_verify(
            q, empty, empty, torch.zeros(1, 1, device="cuda", dtype=torch.int32),
            torch.zeros(1, device="cuda", dtype=torch.int32), dk, dk,
            torch.full((1, 1), -1, device="cuda", dtype=torch.int32))


@pytest.mark.parametrize("prefix,dim", [(300, 128), (2053, 128), (37, 64)])
def test_tree_without_pool_size_trusts_ids_inside_lengths(prefix, dim, oracle):
    """physical_pages = 0 over a real pool: the result equals the call with
    the size, and page-table entries past each length (set to ids far
    outside the pool) are never read."""
    rng = np.random.default_rng(prefix + dim)
    k, v, pages, lengths, dq, dk, dv, par = oracle_np.tree_fixture(
        rng, 4, prefix, 7, d=dim, sigma=1.0, parents="random")
    used = (prefix + 15) // 16
    pages[:, used:] = 1 << 30
    lengths[1] = max(prefix - 20, 0)  # a shorter request: its tail entries stay valid ids
    expected = oracle.tree(k, v, pages, lengths, dq, dk, dv, par, threads=16)
    for ws in (False, True):
        out = G.tree(k, v, pages, lengths, dq, dk, dv, par, workspace=ws, phys_pages=0)
        G.gate(out, expected, 3e-4, f"pool size not given, workspace={ws}")


def _commit_fixture(rng, P=12, hkv=8, d=128, b=3, n=7):
    ck = rng.standard_normal((P, 16, hkv, d)).astype(np.float16)
    cv = rng.standard_normal((P, 16, hkv, d)).astype(np.float16)
    dk = rng.standard_normal((b, n, hkv, d)).astype(np.float16)
    dv = rng.standard_normal((b, n, hkv, d)).astype(np.float16)
    return ck, cv, dk, dv


def test_commit_without_pool_size_is_bit_exact(oracle):
    rng = np.random.default_rng(23)
    ck, cv, dk, dv = _commit_fixture(rng)
    tk, tv, tdk, tdv = G.dev(ck), G.dev(cv), G.dev(dk), G.dev(dv)
    path, dpg, dsl = [0, 3, 5, 6], [10, 10, -1, 11], [3, 4, 5, 15]
    G.commit(tk, tv, tdk, tdv, path, dpg, dsl, 2, phys_pages=0)
    ek, ev = oracle.commit(ck, cv, dk, dv, path, dpg, dsl, 2)
    assert np.array_equal(tk.cpu().numpy().view(np.uint16), ek.view(np.uint16))
    assert np.array_equal(tv.cpu().numpy().view(np.uint16), ev.view(np.uint16))


def test_commit_of_no_heads_copies_nothing():
    rng = np.random.default_rng(24)
    ck, cv, dk, dv = _commit_fixture(rng)
    tk, tv, tdk, tdv = G.dev(ck), G.dev(cv), G.dev(dk), G.dev(dv)
    G.commit(tk, tv, tdk, tdv, [0, 1], [2, 3], [4, 5], 1, kv_heads=0)
    assert np.array_equal(tk.cpu().numpy().view(np.uint16), ck.view(np.uint16))
    assert np.array_equal(tv.cpu().numpy().view(np.uint16), cv.view(np.uint16))
