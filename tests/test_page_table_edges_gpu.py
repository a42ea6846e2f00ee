"""Page tables and lengths that the reference leaves undefined, through every
compute entry point.

The reference reads page-table entries and lengths unchecked
(src/paged_gqa.cu:42-44, src/packed_decode.cu:38, src/tree_attention.cu:34).
Here the kernels' own bounds checks give them a defined result:

- an entry inside a sequence's length that is negative or not below
  physical_pages names no page, and its slots are skipped;
- a length above the table's capacity (max_pages * 16) reads the whole table;
- a negative length is an empty sequence (zeros for decode; the draft tree
  alone for tree verification).

Attention over a prefix is a softmax over a set of tokens, so each expected
output is the oracle's over equivalent valid inputs: the table with the
invalid entries removed and the length cut by their valid slots, the length
clamped to the capacity, or zero.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle_np
import gpu_helpers as G

pytestmark = pytest.mark.gpu

CAP = 48  # page-table columns: 768 tokens


def _case(rng, d, hq=32, hkv=8):
    pool = 4 * CAP + 4
    ids = rng.permutation(pool).astype(np.int32)
    pages = ids[:4 * CAP].reshape(4, CAP).copy()  # every entry names a page
    lengths = np.array([700, 5000, -7, 100], dtype=np.int32)
    pages[0, 5] = -1          # a full page inside the length
    pages[0, 20] = pool + 1000
    pages[3, 6] = pool        # the partial last page (4 of 16 slots)
    # The equivalent valid inputs.
    exp_pages = pages.copy()
    row = np.delete(pages[0], [5, 20])
    exp_pages[0] = np.concatenate([row, row[:2]])
    exp_pages[3, 6] = ids[-1]
    exp_len = np.array([700 - 32, CAP * 16, 0, 96], dtype=np.int32)
    k = (rng.standard_normal((pool, 16, hkv, d)) * 0.5).astype(np.float16)
    v = (rng.standard_normal((pool, 16, hkv, d)) * 0.5).astype(np.float16)
    q = (rng.standard_normal((4, hq, d)) * 0.5).astype(np.float16)
    return q, k, v, pages, lengths, exp_pages, exp_len


@pytest.mark.parametrize("d", [64, 128])
def test_decode_and_packed_skip_invalid_pages_and_clamp_lengths(d, oracle):
    rng = np.random.default_rng(300 + d)
    q, k, v, pages, lengths, exp_pages, exp_len = _case(rng, d)
    expected = oracle.decode(q, k, v, exp_pages, exp_len, threads=8)
    assert np.all(expected[2] == 0)
    for splits in (1, 3, 8):
        G.gate(G.decode(q, k, v, pages, lengths, splits), expected, 3e-4,
               f"bc_decode D={d} splits={splits}")
    # The same pool as a packed [P, 2, 16, Hkv, D] cache.
    cache = torch.from_numpy(np.ascontiguousarray(np.stack([k, v], axis=1))).cuda()
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    for ws in (False, True):
        out = G.packed(q, cache, strides, k.shape[2], k.shape[0], pages, lengths,
                       1 / math.sqrt(d), workspace=ws)
        err = np.abs(out.astype(np.float32) - expected)
        assert np.all(err <= G.f16_tolerance(expected, 3e-4)), \
            f"packed D={d} workspace={ws}: max err {err.max():.3e}"


@pytest.mark.parametrize("d", [64, 128])
def test_tree_skips_invalid_pages_and_clamps_lengths(d, oracle):
    rng = np.random.default_rng(400 + d)
    _, k, v, pages, lengths, exp_pages, exp_len = _case(rng, d)
    nodes = 7
    dq = (rng.standard_normal((4, nodes, 32, d)) * 0.5).astype(np.float16)
    dk = (rng.standard_normal((4, nodes, 8, d)) * 0.5).astype(np.float16)
    dv = (rng.standard_normal((4, nodes, 8, d)) * 0.5).astype(np.float16)
    par = oracle_np.random_parents(rng, 4, nodes)
    expected = oracle.tree(k, v, exp_pages, exp_len, dq, dk, dv, par, threads=8)
    for ws in (False, True):
        out = G.tree(k, v, pages, lengths, dq, dk, dv, par, workspace=ws)
        G.gate(out, expected, 3e-4, f"tree D={d} workspace={ws}")
