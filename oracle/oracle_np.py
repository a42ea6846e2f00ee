"""Independent float64 closed forms and fixture generators (numpy).

TEST INFRASTRUCTURE ONLY.  The closed forms here pin the C oracle: they
compute softmax(q . K^T * scale) . V in float64 with whole-array numpy
operations, without the C oracle's float casts or token loop, and derive
ancestor sets by brute force.  They follow the reference's torch oracles
(tests/test_torch_ops.py:32-52 and :77-88 of Haaziq386/branchcraft-cuda).

Fixture generators produce the benchmark configurations' shapes from a
numpy seed (inputs are stored with the golden files, so generation never
has to be reproduced bit for bit across numpy versions).
"""

from __future__ import annotations

import math

import numpy as np

PAGE = 16


def softmax_attend(q: np.ndarray, keys: np.ndarray, vals: np.ndarray, scale: float):
    """q [D]; keys, vals [T, D]; float64; empty T gives zeros."""
    if keys.shape[0] == 0:
        return np.zeros(q.shape[-1], dtype=np.float64)
    s = keys.astype(np.float64) @ q.astype(np.float64) * scale
    s -= s.max()
    p = np.exp(s)
    return (p @ vals.astype(np.float64)) / p.sum()


def gather_paged(k, pages_row, length, kvh):
    """Rows of token t = k[pages_row[t // 16], t % 16, kvh] for t < length."""
    t = np.arange(length)
    return k[pages_row[t // PAGE], t % PAGE, kvh]


def decode(q, k, v, pages, lengths, scale=None):
    b, hq, d = q.shape
    hkv = k.shape[2]
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    out = np.zeros((b, hq, d), dtype=np.float64)
    for bi in range(b):
        n = int(max(0, min(lengths[bi], pages.shape[1] * PAGE)))
        for h in range(hq):
            kvh = h // (hq // hkv)
            out[bi, h] = softmax_attend(q[bi, h], gather_paged(k, pages[bi], n, kvh),
                                        gather_paged(v, pages[bi], n, kvh), scale)
    return out


def packed_view(cache_flat, strides, shape_pages, hkv, d):
    """Logical [P, Hkv, 16, D] K and V arrays read through element strides."""
    bs, hs, ss, kvs = strides
    p = np.arange(shape_pages)[:, None, None, None]
    h = np.arange(hkv)[None, :, None, None]
    s = np.arange(PAGE)[None, None, :, None]
    e = np.arange(d)[None, None, None, :]
    off = p * bs + h * hs + s * ss + e
    return cache_flat[off], cache_flat[off + kvs]


def packed_decode(q, cache_flat, strides, hkv, phys_pages, pages, lengths, scale):
    """strides = (block, head, slot, kv) in elements of cache_flat."""
    d = q.shape[2]
    kk, vv = packed_view(cache_flat, strides, phys_pages, hkv, d)
    # to paged [P,16,Hkv,D]
    return decode(q, kk.transpose(0, 2, 1, 3), vv.transpose(0, 2, 1, 3), pages, lengths,
                  scale)


def ancestors(parent_row, node):
    """Brute force: the nodes reached from node by following parents, each
    once; the walk ends at a parent outside [0, N) or at a repeated node."""
    n = len(parent_row)
    seen = []
    cur = node
    while 0 <= cur < n and cur not in seen:
        seen.append(cur)
        cur = int(parent_row[cur])
    return seen


def tree(k, v, pages, lengths, dq, dk, dv, parent):
    b, n, hq, d = dq.shape
    hkv = k.shape[2]
    scale = 1.0 / math.sqrt(d)
    out = np.zeros((b, n, hq, d), dtype=np.float64)
    for bi in range(b):
        ln = int(max(0, min(lengths[bi], pages.shape[1] * PAGE)))
        for node in range(n):
            anc = ancestors(parent[bi], node)
            for h in range(hq):
                kvh = h // (hq // hkv)
                keys = np.concatenate([gather_paged(k, pages[bi], ln, kvh), dk[bi, anc, kvh]])
                vals = np.concatenate([gather_paged(v, pages[bi], ln, kvh), dv[bi, anc, kvh]])
                out[bi, node, h] = softmax_attend(dq[bi, node, h], keys, vals, scale)
    return out


# ---- fixtures -------------------------------------------------------------

def paged_fixture(rng, batch, hq, hkv, d, lengths, spare=7, sigma=0.5, pool=None):
    """Reference-style paged fixture (src/main.cu:48-79): shuffled page ids,
    `spare` extra pages, N(0, sigma) FP16 values."""
    lengths = np.asarray(lengths, dtype=np.int32)
    max_pages = max(1, int(-(-lengths.max() // PAGE)) if len(lengths) else 1)
    used = int(sum(-(-int(x) // PAGE) for x in lengths))
    phys = pool if pool is not None else used + spare
    ids = rng.permutation(phys).astype(np.int32)
    pages = np.full((batch, max_pages), -1, dtype=np.int32)
    cur = 0
    for bi in range(batch):
        cnt = -(-int(lengths[bi]) // PAGE)
        pages[bi, :cnt] = ids[cur:cur + cnt]
        cur += cnt
    q = (rng.standard_normal((batch, hq, d)) * sigma).astype(np.float16)
    k = (rng.standard_normal((phys, PAGE, hkv, d)) * sigma).astype(np.float16)
    v = (rng.standard_normal((phys, PAGE, hkv, d)) * sigma).astype(np.float16)
    return q, k, v, pages, lengths


def random_parents(rng, batch, nodes):
    """parent[0] = -1, parent[i] ~ U{0..i-1} (benchmark configs 2-3)."""
    par = np.full((batch, nodes), -1, dtype=np.int32)
    for bi in range(batch):
        for i in range(1, nodes):
            par[bi, i] = rng.integers(0, i)
    return par


def binary_parents(batch, nodes):
    """parent = (n-1)/2 (src/main.cu:177)."""
    par = np.array([-1] + [(i - 1) // 2 for i in range(1, nodes)], dtype=np.int32)
    return np.tile(par, (batch, 1))


def tree_fixture(rng, batch, prefix, nodes, hq=32, hkv=8, d=128, sigma=0.5,
                 parents="binary", shared=True, extra_pages=2):
    """Tree fixture: all requests share one prefix page list (as the
    reference's make_tree_fixture, src/main.cu:145-179)."""
    q0, k, v, pages0, _ = paged_fixture(rng, 1, hq, hkv, d, [prefix], sigma=sigma)
    max_pages = pages0.shape[1] + extra_pages
    phys = k.shape[0] + batch * extra_pages
    kk = np.zeros((phys, PAGE, hkv, d), dtype=np.float16)
    vv = np.zeros_like(kk)
    kk[:k.shape[0]] = k
    vv[:v.shape[0]] = v
    pages = np.full((batch, max_pages), -1, dtype=np.int32)
    pages[:, :pages0.shape[1]] = pages0[0]
    if prefix == 0:
        pages[:, 0] = -1
    lengths = np.full(batch, prefix, dtype=np.int32)
    dq = (rng.standard_normal((batch, nodes, hq, d)) * sigma).astype(np.float16)
    dk = (rng.standard_normal((batch, nodes, hkv, d)) * sigma).astype(np.float16)
    dv = (rng.standard_normal((batch, nodes, hkv, d)) * sigma).astype(np.float16)
    par = binary_parents(batch, nodes) if parents == "binary" else random_parents(rng, batch, nodes)
    return kk, vv, pages, lengths, dq, dk, dv, par
