"""Paged GQA decode (bc_decode) against the CPU oracle.

Cases restate the reference driver's suite (src/main.cu:318-352): empty,
single token, page boundary 16/17, ragged batch, non-power-of-two GQA
(10/2, 12/3), D=64/128 and splits 1..16 at its 3e-4 gate; then splits
beyond the reference's cap, benchmark config 1 and config 4 at full size.
"""

import numpy as np
import pytest
import torch

import branchcraft_capi as capi
from oracle import oracle_np
import gpu_helpers as G

pytestmark = pytest.mark.gpu

REF_CASES = [
    (1, 8, 2, 64, [0]), (1, 8, 2, 64, [1]), (1, 8, 2, 64, [16]), (1, 8, 2, 64, [17]),
    (3, 10, 2, 64, [0, 37, 91]), (3, 12, 3, 128, [7, 128, 257]), (2, 32, 8, 128, [513, 3]),
]


@pytest.mark.parametrize("case", REF_CASES, ids=lambda c: f"B{c[0]}_H{c[1]}x{c[2]}_D{c[3]}")
def test_reference_cases_all_splits(case, oracle):
    b, hq, hkv, d, lens = case
    rng = np.random.default_rng(17)
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, b, hq, hkv, d, lens)
    expected = oracle.decode(q, k, v, pages, lengths)
    for splits in (1, 2, 4, 8, 16, 33, 64):
        out = G.decode(q, k, v, pages, lengths, splits)
        G.gate(out, expected, 3e-4, f"splits={splits}")


def test_config1_b1_l512(oracle):
    """benchmark config 1: B=1, L=512, 32/8 heads, D=128, pool of 64 pages,
    page table = first 32 ids of a seeded permutation, N(0,1)."""
    rng = np.random.default_rng(1)
    perm = rng.permutation(64).astype(np.int32)
    pages = perm[:32].reshape(1, 32)
    lengths = np.array([512], dtype=np.int32)
    q = rng.standard_normal((1, 32, 128)).astype(np.float16)
    k = rng.standard_normal((64, 16, 8, 128)).astype(np.float16)
    v = rng.standard_normal((64, 16, 8, 128)).astype(np.float16)
    expected = oracle.decode(q, k, v, pages, lengths)
    closed = oracle_np.decode(q, k, v, pages, lengths)
    G.gate(expected, closed, 1e-5, "oracle vs float64 closed form")
    for splits in (1, 2, 4, 8):
        G.gate(G.decode(q, k, v, pages, lengths, splits), expected, 3e-4, f"splits={splits}")


def test_config4_split_k_long_context(oracle):
    """benchmark config 4: B=4, L ~ U[16384, 32768], random page map; the
    split count keeps chunks in [256, 2048] tokens."""
    rng = np.random.default_rng(4)
    lens = rng.integers(16384, 32769, size=4)
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, 4, 32, 8, 128, lens, spare=16,
                                                     sigma=1.0)
    expected = oracle.decode(q, k, v, pages, lengths, threads=16)
    # bc_auto_splits' own choice, which bench.py times (33 on 256 CUs), and
    # the reference's cap of 16 that branchcraft::auto_splits returns.
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    shape = capi.Shape(4, 32, 8, 128, pages.shape[1], k.shape[0])
    auto = G.lib().bc_auto_splits(shape, int(lens.max()), cus)
    if cus == 256:
        assert auto == 33
    for splits in sorted({16, auto, 64}):
        out = G.decode(q, k, v, pages, lengths, splits)
        G.gate(out, expected, 2e-3, f"config4 splits={splits}")
        G.gate(out, expected, 3e-4, f"config4 splits={splits} (reference gate)")


def test_garbage_in_unused_slots_is_ignored(oracle):
    """Slots past a sequence's length (in its last page) may hold NaN/inf;
    they must not reach the output."""
    rng = np.random.default_rng(5)
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, 3, 8, 2, 128, [5, 33, 16])
    expected = oracle.decode(q, k, v, pages, lengths)
    k2, v2 = k.copy(), v.copy()
    for bi, n in enumerate(lengths):
        if n % 16:
            last = pages[bi, n // 16]
            k2[last, n % 16:] = np.float16(np.nan)
            v2[last, n % 16:] = np.float16(np.inf)
    for splits in (1, 3):
        G.gate(G.decode(q, k2, v2, pages, lengths, splits), expected, 3e-4, "garbage slots")


def test_split_matches_single_at_scale():
    """Split-K and single-partition results agree (src/main.cu:505-509)."""
    rng = np.random.default_rng(9)
    lens = [8192 - (i % 4) * 1024 for i in range(8)]
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, 8, 32, 8, 128, lens)
    single = G.decode(q, k, v, pages, lengths, 1)
    for splits in (2, 16, 128):
        G.gate(G.decode(q, k, v, pages, lengths, splits), single, 3e-4, f"splits={splits}")


@pytest.mark.parametrize("hq,hkv,d", [(8, 8, 128), (32, 1, 64), (64, 2, 128), (48, 3, 64),
                                      (40, 8, 128), (24, 6, 64)])
def test_head_layouts_beyond_reference(hq, hkv, d, oracle):
    """Multi-head (group 1), one KV head for 32 query heads (two 16-column
    head blocks per KV head), group 32 with two KV heads, and groups that
    leave part of a head block empty (16, 5 and 4 heads), with and without
    splits."""
    rng = np.random.default_rng(hq * 131 + hkv * 7 + d)
    lens = [0, 31, 200, 1029]
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, len(lens), hq, hkv, d, lens)
    expected = oracle.decode(q, k, v, pages, lengths, threads=8)
    for splits in (1, 3, 40):
        out = G.decode(q, k, v, pages, lengths, splits)
        G.gate(out, expected, 3e-4, f"Hq={hq} Hkv={hkv} D={d} splits={splits}")


@pytest.mark.parametrize("batch", [40, 64, 70, 130])
def test_unsplit_ragged_batches(batch, oracle):
    """splits = 1 runs one workgroup per (sequence, head block), and
    workgroup r takes the sequence with the r-th most pages (ties by index)
    for batches of up to 64; larger batches keep index order.  Ragged
    lengths with ties and empty sequences cover both orders; with splits,
    130 sequences make the workgroups' range search cross three blocks of
    64 lengths."""
    rng = np.random.default_rng(batch)
    lens = rng.integers(0, 300, size=batch)
    lens[::7] = 129
    lens[3] = 0
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, batch, 8, 2, 64, list(lens))
    expected = oracle.decode(q, k, v, pages, lengths, threads=8)
    G.gate(G.decode(q, k, v, pages, lengths, 1), expected, 3e-4, f"B={batch} splits=1")
    G.gate(G.decode(q, k, v, pages, lengths, 5), expected, 3e-4, f"B={batch} splits=5")


def test_large_batch_short_contexts_split(oracle):
    """A batch of a wave of flat ranges or more (128 at 32/8 heads) takes two
    splits at contexts below 512 tokens too, so one wave of ranges streams
    many sequences each; ragged lengths with empty sequences.  One split and
    five splits (ranges capped at one wave) give the same result."""
    rng = np.random.default_rng(300)
    lens = rng.integers(0, 401, size=300)
    lens[::11] = 0
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, 300, 32, 8, 128, lens)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    shape = capi.Shape(300, 32, 8, 128, pages.shape[1], k.shape[0])
    assert G.lib().bc_auto_splits(shape, int(lens.max()), cus) == 2
    expected = oracle.decode(q, k, v, pages, lengths, threads=16)
    for splits in (2, 1, 5):
        G.gate(G.decode(q, k, v, pages, lengths, splits), expected, 3e-4, f"splits={splits}")


@pytest.mark.parametrize("out_shift,scratch_shift", [(4, 0), (0, 4), (8, 12)])
def test_element_aligned_output_and_scratch(out_shift, scratch_shift, oracle):
    """The reference takes any `float*` for the output and the split
    partials.  Aligned Q/K/V with an output or caller scratch that is only
    4-byte aligned switch the launch to element-wise stores; unsplit and
    split calls match the oracle."""
    rng = np.random.default_rng(90 + out_shift + scratch_shift)
    lens = [700, 0, 1500, 33]
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, len(lens), 32, 8, 128, lens)
    expected = oracle.decode(q, k, v, pages, lengths, threads=8)
    for splits in (1, 5):
        out = G.decode(q, k, v, pages, lengths, splits, out_shift=out_shift,
                       scratch_shift=scratch_shift)
        G.gate(out, expected, 3e-4,
               f"splits={splits} out_shift={out_shift} scratch_shift={scratch_shift}")
