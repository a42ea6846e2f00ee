"""Seeded random shapes through every compute entry point, against the CPU
oracle.

Each case draws its shape from a fixed seed: batch, per-request lengths
(empty requests included), page sharing between requests, GQA layout
(groups 1 to 8), head dimension 64 or 128, tree size and parent shape, split
count and cache layout.  The host's plan choices -- single pass, four- or
eight-wave parts, two requests per workgroup, the row-sharing tree kernel,
unsplit and flat-range decode, one or four merge waves per row -- are then
crossed at many boundaries instead of the handful the fixed cases pin.
Sizes are bounded so the oracle finishes in about a second per case; the
gate is the reference driver's 3e-4 (src/main.cu:505-509), plus half an FP16
ulp for FP16 outputs.

BC_RANDOM_SEEDS=n runs seeds 1000 .. 1000 + n - 1 in each test instead of
the short default set, for a longer sweep.
"""

import math
import os

import numpy as np
import pytest
import torch

from oracle import oracle_np
import branchcraft_capi as capi
import gpu_helpers as G

pytestmark = pytest.mark.gpu

_WIDE = int(os.environ.get("BC_RANDOM_SEEDS", "0"))


def _seeds(n):
    return range(1000, 1000 + _WIDE) if _WIDE > 0 else range(n)


LAYOUTS = [(32, 8), (8, 8), (16, 2), (8, 1), (64, 8), (12, 3), (4, 4), (24, 8)]


def _parents(rng, batch, nodes, kind):
    """Valid trees (parent[i] < i, parent[0] = -1) of three shapes."""
    if kind == "random":
        return oracle_np.random_parents(rng, batch, nodes)
    row = np.arange(-1, nodes - 1, dtype=np.int32)  # chain: depth nodes - 1
    if kind == "star":
        row = np.where(np.arange(nodes) == 0, -1, 0).astype(np.int32)
    return np.tile(row, (batch, 1))


def _tree_case(seed):
    rng = np.random.default_rng(7000 + seed)
    d = int(rng.choice([64, 128]))
    hq, hkv = LAYOUTS[rng.integers(len(LAYOUTS))]
    nodes = int(rng.choice([1, 2, 5, 7, 16, 31, 32, 33, 64, 100, 200, 256]))
    batch = int(rng.integers(1, 25))
    maxlen = int(rng.choice([0, 40, 300, 700, 1500, 2500]))
    # Bound the oracle's work (rows x attended tokens).
    while batch > 1 and batch * nodes * hq * (maxlen + nodes) > 8e6:
        batch = max(1, batch // 2)
    while maxlen > 16 and batch * nodes * hq * (maxlen + nodes) > 8e6:
        maxlen //= 2
    lengths = rng.integers(0, maxlen + 1, size=batch).astype(np.int32)
    if rng.random() < 0.5:
        lengths[:] = maxlen  # one length for every request, as forked requests have
    share = [-1 if i == 0 or rng.random() < 0.4 else int(rng.integers(0, i))
             for i in range(batch)]
    npg = [-(-int(x) // 16) for x in lengths]
    max_pages = max(max(npg), 1) + int(rng.integers(0, 40))
    cow = {i for i in range(batch) if share[i] >= 0 and rng.random() < 0.3}
    pool = sum(npg) + len(cow) + 8
    sigma = float(rng.choice([0.5, 1.0]))
    k = (rng.standard_normal((pool, 16, hkv, d)) * sigma).astype(np.float16)
    v = (rng.standard_normal((pool, 16, hkv, d)) * sigma).astype(np.float16)
    fresh = iter(rng.permutation(pool).astype(np.int32))
    pages = np.full((batch, max_pages), -1, dtype=np.int32)
    for i in range(batch):
        j = share[i]
        for p in range(npg[i]):
            pages[i, p] = pages[j, p] if j >= 0 and p < npg[j] else next(fresh)
        if i in cow and npg[i] > 0:
            pages[i, npg[i] - 1] = next(fresh)
    dq = (rng.standard_normal((batch, nodes, hq, d)) * sigma).astype(np.float16)
    dk = (rng.standard_normal((batch, nodes, hkv, d)) * sigma).astype(np.float16)
    dv = (rng.standard_normal((batch, nodes, hkv, d)) * sigma).astype(np.float16)
    par = _parents(rng, batch, nodes, str(rng.choice(["random", "chain", "star"])))
    what = (f"seed={seed} B={batch} N={nodes} H={hq}/{hkv} D={d} maxlen={maxlen} "
            f"pages={max_pages}")
    return (k, v, pages, lengths, dq, dk, dv, par), what


@pytest.mark.parametrize("seed", _seeds(24))
def test_random_trees(seed, oracle):
    """bc_tree_verify and bc_tree_verify_ws on a random tree batch, and one
    of them again with every FP16 tensor off 16-byte alignment."""
    fix, what = _tree_case(seed)
    print(what, flush=True)
    k, v, pages, lengths, dq, dk, dv, par = fix
    expected = oracle.tree(k, v, pages, lengths, dq, dk, dv, par, threads=16)
    shift = 2 + 4 * (seed % 3)  # 2, 6 or 10 bytes
    for ws, sh in ((False, 0), (True, 0), (seed % 2 == 0, shift)):
        out = G.tree(k, v, pages, lengths, dq, dk, dv, par, workspace=ws, shift=sh)
        G.gate(out, expected, 3e-4, f"{what} workspace={ws} shift={sh}")


def _decode_case(seed):
    rng = np.random.default_rng(8000 + seed)
    d = int(rng.choice([64, 128]))
    hq, hkv = LAYOUTS[rng.integers(len(LAYOUTS))]
    batch = int(rng.integers(1, 80))
    maxlen = int(rng.choice([1, 17, 300, 1000, 3000, 9000]))
    while batch > 1 and batch * hq * maxlen > 4e6:
        batch = max(1, batch // 2)
    lengths = rng.integers(0, maxlen + 1, size=batch).astype(np.int32)
    lengths[rng.integers(batch)] = maxlen
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, batch, hq, hkv, d, lengths,
                                                      spare=int(rng.integers(1, 9)),
                                                      sigma=float(rng.choice([0.5, 1.0])))
    what = f"seed={seed} B={batch} H={hq}/{hkv} D={d} maxlen={maxlen}"
    return (q, k, v, pages, lengths), rng, what


@pytest.mark.parametrize("seed", _seeds(16))
def test_random_paged_decode(seed, oracle):
    """bc_decode at the auto_splits choice and at two random split counts,
    then at the auto choice with Q, K, V and the output off 16-byte
    alignment."""
    (q, k, v, pages, lengths), rng, what = _decode_case(seed)
    print(what, flush=True)
    expected = oracle.decode(q, k, v, pages, lengths, threads=16)
    b, hq, d = q.shape
    auto = G.lib().bc_auto_splits(capi.Shape(b, hq, k.shape[2], d, pages.shape[1], k.shape[0]),
                                  int(lengths.max()), 256)
    for splits in sorted({int(auto), *(int(x) for x in rng.choice(
            [1, 2, 3, 4, 7, 8, 16, 33, 64, 128], size=2, replace=False))}):
        out = G.decode(q, k, v, pages, lengths, splits)
        G.gate(out, expected, 3e-4, f"{what} splits={splits}")
    shift = 2 + 4 * (seed % 3)
    out = G.decode(q, k, v, pages, lengths, int(auto), shift=shift)
    G.gate(out, expected, 3e-4, f"{what} splits={int(auto)} shift={shift}")


@pytest.mark.parametrize("seed", _seeds(16))
def test_random_packed_decode(seed, oracle):
    """bc_packed_decode and bc_packed_decode_ws over a random cache layout:
    HND, NHD or [P, 2, 16, Hkv, D]; then one of them with the FP16 output
    off 16-byte alignment."""
    (q, k, v, pages, lengths), rng, what = _decode_case(100 + seed)
    P, _, hkv, d = k.shape
    layout = str(rng.choice(["HND", "NHD", "5D"]))
    what += f" layout={layout}"
    print(what, flush=True)
    kv = np.concatenate([k, v], axis=-1)  # [P, 16, Hkv, 2D]: K then V per slot
    if layout == "HND":
        cache = torch.from_numpy(np.ascontiguousarray(kv.transpose(0, 2, 1, 3))).cuda()
        strides = (cache.stride(0), cache.stride(1), cache.stride(2), d)
    elif layout == "NHD":
        cache = torch.from_numpy(np.ascontiguousarray(kv)).cuda()
        strides = (cache.stride(0), cache.stride(2), cache.stride(1), d)
    else:
        five = np.stack([k, v], axis=1)  # [P, 2, 16, Hkv, D]
        cache = torch.from_numpy(np.ascontiguousarray(five)).cuda()
        strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    scale = 1 / math.sqrt(d)
    expected, _ = oracle.packed_decode(q, cache.cpu().numpy(), pages, lengths, strides, hkv,
                                       scale, threads=16)
    shift = 2 + 4 * (seed % 3)
    for ws, sh in ((False, 0), (True, 0), (seed % 2 == 0, shift)):
        out = G.packed(q, cache, strides, hkv, P, pages, lengths, scale, workspace=ws,
                       out_shift=sh)
        err = np.abs(out.astype(np.float32) - expected)
        assert np.all(np.isfinite(out)), f"{what} workspace={ws} shift={sh}: non-finite output"
        assert np.all(err <= G.f16_tolerance(expected, 3e-4)), \
            f"{what} workspace={ws} shift={sh}: max err {err.max():.3e}"


def _large_batch_case(seed):
    """65 to 1500 sequences of short contexts (empty ones included): the
    flat ranges of one wave then cover many sequences each, and the merge
    finds its ranges from the range records; packed batches above the range
    count use two partial slots per range."""
    rng = np.random.default_rng(9000 + seed)
    d = int(rng.choice([64, 128]))
    hq, hkv = LAYOUTS[rng.integers(len(LAYOUTS))]
    maxlen = int(rng.choice([16, 100, 400, 1200]))
    batch = int(rng.integers(65, 1501))
    # Bound the fixture (K and V elements) and the oracle's work.
    while batch > 65 and (batch * maxlen * hkv * d > 1e8 or batch * hq * maxlen > 12e6):
        batch = max(65, batch * 3 // 4)
    lengths = rng.integers(0, maxlen + 1, size=batch).astype(np.int32)
    lengths[rng.random(batch) < 0.1] = 0
    lengths[rng.integers(batch)] = maxlen
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, batch, hq, hkv, d, lengths,
                                                      spare=int(rng.integers(1, 9)))
    what = f"seed={seed} B={batch} H={hq}/{hkv} D={d} maxlen={maxlen}"
    return (q, k, v, pages, lengths), rng, what


@pytest.mark.parametrize("seed", _seeds(8))
def test_random_large_batch_paged_decode(seed, oracle):
    """bc_decode over a large batch at the auto split count, two splits and
    a random count up to 9."""
    (q, k, v, pages, lengths), rng, what = _large_batch_case(seed)
    print(what, flush=True)
    expected = oracle.decode(q, k, v, pages, lengths, threads=16)
    b, hq, d = q.shape
    auto = G.lib().bc_auto_splits(capi.Shape(b, hq, k.shape[2], d, pages.shape[1], k.shape[0]),
                                  int(lengths.max()), 256)
    for splits in sorted({int(auto), 2, int(rng.integers(3, 10))}):
        out = G.decode(q, k, v, pages, lengths, splits)
        G.gate(out, expected, 3e-4, f"{what} splits={splits}")


@pytest.mark.parametrize("seed", _seeds(8))
def test_random_large_batch_packed_decode(seed, oracle):
    """bc_packed_decode_ws and bc_packed_decode ([P, 2, 16, Hkv, D] cache)
    over a large batch: within tolerance of the oracle, and bit-identical to
    each other, since every packed workspace fits a slot of the pool."""
    (q, k, v, pages, lengths), rng, what = _large_batch_case(100 + seed)
    print(what, flush=True)
    P, _, hkv, d = k.shape
    cache = torch.from_numpy(np.ascontiguousarray(np.stack([k, v], axis=1))).cuda()
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    scale = 1 / math.sqrt(d)
    expected, _ = oracle.packed_decode(q, cache.cpu().numpy(), pages, lengths, strides, hkv,
                                       scale, threads=16)
    need = G.lib().bc_packed_decode_workspace_size(
        capi.Shape(q.shape[0], q.shape[1], hkv, d, pages.shape[1], P))
    assert need <= capi.BC_SCRATCH_SLOT_BYTES, need
    outs = [G.packed(q, cache, strides, hkv, P, pages, lengths, scale, workspace=ws)
            for ws in (True, False)]
    for ws, out in zip((True, False), outs):
        err = np.abs(out.astype(np.float32) - expected)
        assert np.all(np.isfinite(out)), f"{what} workspace={ws}: non-finite output"
        assert np.all(err <= G.f16_tolerance(expected, 3e-4)), \
            f"{what} workspace={ws}: max err {err.max():.3e}"
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16)), what
