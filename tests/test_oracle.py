"""Pins the CPU oracle (oracle/bc_oracle.c) before it is trusted.

Checks, each chosen so that a plausible mistake in the restatement fails:
* FP16 conversion against numpy on all 65536 bit patterns and on rounding
  boundaries (subnormals, ties, overflow to inf);
* decode / packed decode / tree against an independent float64 closed form
  (oracle/oracle_np.py) with brute-force ancestor sets;
* planted mistakes -- a sibling leaking into a node's mask, K and V swapped,
  the wrong softmax scale, a dropped last token -- move the closed form far
  beyond the tolerance the GPU tests use, so those tests can see them;
* invariants: tree == decode over the expanded-prefix fixture
  (src/main.cu:375-423), empty rows give zeros, token order does not matter;
* the reference's known-answer commit (tests/test_torch_ops.py:99-114) and
  its driver commit case (src/main.cu:264-313);
* the committed golden vectors under tests/golden/.
"""

import math
from pathlib import Path

import numpy as np
import pytest

from oracle import oracle_np

GOLDEN = Path(__file__).resolve().parent / "golden"

REF_CASES = [
    (1, 8, 2, 64, [0]), (1, 8, 2, 64, [1]), (1, 8, 2, 64, [16]), (1, 8, 2, 64, [17]),
    (3, 10, 2, 64, [0, 37, 91]), (3, 12, 3, 128, [7, 128, 257]), (2, 32, 8, 128, [513, 3]),
]


def test_f16_conversions_match_numpy(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    got = oracle.h2f(bits)
    want = bits.view(np.float16).astype(np.float32)
    same = (got == want) | (np.isnan(got) & np.isnan(want))
    assert same.all()
    rng = np.random.default_rng(0)
    edge = np.array([65504, 65519.99, 65520, 7e4, -7e4, 2.0 ** -25, 2.0 ** -24,
                     3 * 2.0 ** -26, 2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 0.0, -0.0,
                     1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, np.inf, -np.inf], dtype=np.float32)
    x = np.concatenate([edge, rng.standard_normal(200000).astype(np.float32) * 100,
                        (rng.standard_normal(100000) * 1e-5).astype(np.float32)])
    with np.errstate(over="ignore"):
        want16 = x.astype(np.float16).view(np.uint16)
    assert np.array_equal(oracle.f2h(x), want16)


@pytest.mark.parametrize("case", REF_CASES, ids=str)
def test_decode_matches_closed_form(case, oracle):
    b, hq, hkv, d, lens = case
    rng = np.random.default_rng(17)
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, b, hq, hkv, d, lens)
    got = oracle.decode(q, k, v, pages, lengths)
    want = oracle_np.decode(q, k, v, pages, lengths)
    assert np.max(np.abs(got - want)) < 2e-6
    for bi, n in enumerate(lengths):
        if n == 0:
            assert np.all(got[bi] == 0)


def test_decode_threads_do_not_change_results(oracle):
    rng = np.random.default_rng(2)
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, 3, 12, 3, 128, [7, 128, 257])
    a = oracle.decode(q, k, v, pages, lengths, threads=1)
    b = oracle.decode(q, k, v, pages, lengths, threads=5)
    assert np.array_equal(a, b)


@pytest.mark.parametrize("layout", ["HND", "NHD", "P2SHD"])
def test_packed_matches_closed_form(layout, oracle):
    rng = np.random.default_rng(4)
    P, hkv, d, hq, b = 9, 2, 64, 8, 3
    if layout == "HND":
        cache = rng.standard_normal((P, hkv, 16, 2 * d)).astype(np.float16)
        st = (hkv * 16 * 2 * d, 16 * 2 * d, 2 * d, d)
    elif layout == "NHD":
        cache = rng.standard_normal((P, 16, hkv, 2 * d)).astype(np.float16)
        st = (16 * hkv * 2 * d, 2 * d, hkv * 2 * d, d)
    else:
        cache = rng.standard_normal((P, 2, 16, hkv, d)).astype(np.float16)
        st = (2 * 16 * hkv * d, d, hkv * d, 16 * hkv * d)
    q = rng.standard_normal((b, hq, d)).astype(np.float16)
    pages = np.array([[4, 1], [2, 7], [8, 6]], dtype=np.int32)
    lengths = np.array([23, 9, 0], dtype=np.int32)
    got32, got16 = oracle.packed_decode(q, cache, pages, lengths, st, hkv, 0.1)
    want = oracle_np.packed_decode(q, cache.reshape(-1), st, hkv, P, pages, lengths, 0.1)
    assert np.max(np.abs(got32 - want)) < 2e-6
    assert np.array_equal(got16, got32.astype(np.float16))
    assert np.all(got32[2] == 0)


@pytest.mark.parametrize("prefix,nodes,parents", [(0, 7, "binary"), (17, 7, "binary"),
                                                 (37, 7, "random"), (64, 40, "random")])
def test_tree_matches_closed_form(prefix, nodes, parents, oracle):
    rng = np.random.default_rng(prefix + nodes)
    fix = oracle_np.tree_fixture(rng, 2, prefix, nodes, hq=8, hkv=2, d=64, parents=parents)
    got = oracle.tree(*fix)
    want = oracle_np.tree(*fix)
    assert np.max(np.abs(got - want)) < 2e-6


def test_ancestor_sets_brute_force():
    par = oracle_np.binary_parents(1, 7)[0]
    assert oracle_np.ancestors(par, 0) == [0]
    assert oracle_np.ancestors(par, 6) == [6, 2, 0]
    assert oracle_np.ancestors(par, 4) == [4, 1, 0]
    # a cycle ends at the first repeated node; a parent outside [0, N) ends
    # the chain
    assert oracle_np.ancestors(np.array([1, 0, -1]), 0) == [0, 1]
    assert oracle_np.ancestors(np.array([-1, 5, 1]), 2) == [2, 1]


def test_planted_mistakes_exceed_gpu_tolerance(oracle):
    """If the kernel made any of these mistakes, the 3e-4 gate would fail."""
    rng = np.random.default_rng(8)
    k, v, pages, lengths, dq, dk, dv, par = oracle_np.tree_fixture(
        rng, 1, 20, 7, hq=4, hkv=2, d=64, sigma=1.0)
    good = oracle.tree(k, v, pages, lengths, dq, dk, dv, par)
    # 1. sibling leaks into the mask: node 3 also sees node 4
    bad = par.copy()
    bad[0, 4] = 3
    leak = oracle_np.tree(k, v, pages, lengths, dq, dk, dv, bad)
    assert np.max(np.abs(leak[0, 4] - good[0, 4])) > 1e-2
    # 2. K and V swapped
    swap = oracle.tree(v, k, pages, lengths, dq, dv, dk, par)
    assert np.max(np.abs(swap - good)) > 1e-2
    # 3. wrong scale (1/D instead of 1/sqrt(D)) in decode
    q, kk, vv, pg, ln = oracle_np.paged_fixture(rng, 1, 4, 2, 64, [40], sigma=1.0)
    right = oracle.decode(q, kk, vv, pg, ln)
    wrong = oracle_np.decode(q, kk, vv, pg, ln, scale=1.0 / 64)
    assert np.max(np.abs(right - wrong)) > 1e-2
    # 4. last token dropped
    short = oracle.decode(q, kk, vv, pg, ln - 1)
    assert np.max(np.abs(right - short)) > 1e-3


def test_tree_equals_expanded_decode(oracle):
    rng = np.random.default_rng(91)
    k, v, pages, lengths, dq, dk, dv, par = oracle_np.tree_fixture(
        rng, 2, 45, 7, hq=8, hkv=2, d=64, parents="random")
    tree = oracle.tree(k, v, pages, lengths, dq, dk, dv, par)
    el, ep, ek, ev = oracle.expand_tree(k, v, pages, lengths, dk, dv, par)
    b, n, hq, d = dq.shape
    flat = oracle.decode(dq.reshape(b * n, hq, d), ek, ev, ep, el)
    assert np.max(np.abs(flat.reshape(tree.shape) - tree)) < 1e-6
    # each expanded sequence is prefix + root..node path
    for s in range(b * n):
        bi, node = divmod(s, n)
        assert el[s] == 45 + len(oracle_np.ancestors(par[bi], node))


def test_token_order_invariance(oracle):
    """Relabelling physical pages (and moving their contents) changes nothing."""
    rng = np.random.default_rng(6)
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, 2, 8, 2, 64, [50, 33])
    perm = rng.permutation(k.shape[0])
    inv = np.argsort(perm)
    k2, v2 = k[perm], v[perm]
    pages2 = np.where(pages >= 0, inv[np.maximum(pages, 0)], -1).astype(np.int32)
    a = oracle.decode(q, k, v, pages, lengths)
    b = oracle.decode(q, k2, v2, pages2, lengths)
    assert np.max(np.abs(a - b)) < 1e-6


def test_known_answer_commit(oracle):
    """tests/test_torch_ops.py:99-114 of the reference, on the oracle."""
    ck = np.zeros((4, 16, 2, 64), dtype=np.float16)
    cv = np.zeros_like(ck)
    dk = np.broadcast_to(np.arange(3, dtype=np.float16).reshape(1, 3, 1, 1),
                         (1, 3, 2, 64)).copy()
    dv = dk + np.float16(10)
    nk, nv = oracle.commit(ck, cv, dk, dv, [0, 2], [3, 3], [6, 7], 0)
    assert np.array_equal(nk[3, 6], dk[0, 0]) and np.array_equal(nk[3, 7], dk[0, 2])
    assert np.array_equal(nv[3, 7], dv[0, 2])
    assert np.count_nonzero(nk[:3]) == 0 and np.count_nonzero(nk[3, 8:]) == 0
    # out-of-range entries are skipped
    nk2, _ = oracle.commit(ck, cv, dk, dv, [0, 5, 1], [3, 3, 9], [0, 1, 2], 0)
    assert np.count_nonzero(nk2) == 0  # node 0 is zero-valued, others skipped
    nk3, _ = oracle.commit(ck, cv, dk, dv, [1], [3], [16], 0)
    assert np.count_nonzero(nk3) == 0


def test_driver_commit_case(oracle):
    """src/main.cu:264-313: clone the shared partial page to P-1, commit
    path {0,1,3} at slots {1,2,3}; decoding node 3's query over the committed
    cache equals node 3's tree output, the sibling is untouched."""
    rng = np.random.default_rng(49)
    k, v, pages, lengths, dq, dk, dv, par = oracle_np.tree_fixture(rng, 2, 17, 7, hq=8,
                                                                   hkv=2, d=64)
    tree = oracle.tree(k, v, pages, lengths, dq, dk, dv, par)
    P = k.shape[0]
    ck, cv = oracle.copy_pages(k, v, [int(pages[0, 1])], [P - 1])
    assert np.array_equal(ck[P - 1], k[pages[0, 1]])
    ck, cv = oracle.commit(ck, cv, dk, dv, [0, 1, 3], [P - 1] * 3, [1, 2, 3], 0)
    cp, cl = pages.copy(), lengths.copy()
    cp[0, 1] = P - 1
    cl[0] += 3
    q = dq[:, 3].copy()
    after = oracle.decode(q, ck, cv, cp, cl)
    assert np.max(np.abs(after[0] - tree[0, 3])) < 1e-6
    before = oracle.decode(q, k, v, pages, lengths)
    assert np.array_equal(after[1], before[1])
    assert np.array_equal(ck[pages[0, 1]], k[pages[0, 1]])


@pytest.mark.parametrize("name", sorted(p.stem for p in GOLDEN.glob("*.npz")))
def test_golden_vectors(name, oracle):
    g = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    kind = str(g["kind"])
    if kind == "decode":
        got = oracle.decode(g["q"], g["k"], g["v"], g["pages"], g["lengths"])
        closed = oracle_np.decode(g["q"], g["k"], g["v"], g["pages"], g["lengths"])
    elif kind == "tree":
        args = (g["k"], g["v"], g["pages"], g["lengths"], g["dq"], g["dk"], g["dv"],
                g["parent"])
        got = oracle.tree(*args)
        closed = oracle_np.tree(*args)
    elif kind == "packed":
        st = tuple(int(x) for x in g["strides"])
        got, _ = oracle.packed_decode(g["q"], g["cache"], g["pages"], g["lengths"], st,
                                      int(g["hkv"]), float(g["scale"]))
        closed = oracle_np.packed_decode(g["q"], g["cache"].reshape(-1), st, int(g["hkv"]),
                                         g["cache"].shape[0], g["pages"], g["lengths"],
                                         float(g["scale"]))
    else:
        raise AssertionError(kind)
    assert np.array_equal(got, g["expected"]), "oracle drifted from its golden output"
    assert np.max(np.abs(closed - g["expected"])) < 2e-6
