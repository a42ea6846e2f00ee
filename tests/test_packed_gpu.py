"""Packed-cache decode (bc_packed_decode[_ws]) against the CPU oracle.

Restates the reference's packed test (tests/test_torch_ops.py:62-96: HND and
NHD strides, lengths [23, 9, 0]) and adds the [P,2,16,Hkv,D] layout of
benchmark config 5, unaligned strides, the split/unsplit paths and config 5
at full size.  FP16 outputs are gated at 2e-3 plus half an FP16 ulp.
"""

import math

import numpy as np
import pytest
import torch

from oracle import oracle_np
import branchcraft_capi as capi
import gpu_helpers as G

pytestmark = pytest.mark.gpu


def _run_both(q, cache, strides, hkv, phys, pages, lengths, scale, oracle, atol=2e-3):
    exp32, _ = oracle.packed_decode(q, cache.cpu().numpy(), pages, lengths, strides, hkv,
                                    scale)
    # The same inputs again through a page table of 80 columns: more than 1024
    # tokens of capacity take the split path (flat page ranges and the merge)
    # where a short table runs unsplit.
    wide = np.full((pages.shape[0], max(pages.shape[1], 80)), -1, dtype=np.int32)
    wide[:, :pages.shape[1]] = pages
    b, hq, d = q.shape
    if G.lib().bc_packed_decode_workspace_size(capi.Shape(b, hq, hkv, d, 80, phys)) > 0:
        runs = ((False, pages), (True, pages), (True, wide))
    else:  # batches large enough that the split rule keeps even 1280 tokens unsplit
        runs = ((False, pages), (True, pages))
    for ws, pg in runs:
        out = G.packed(q, cache, strides, hkv, phys, pg, lengths, scale, workspace=ws)
        tol = G.f16_tolerance(exp32, atol)
        err = np.abs(out.astype(np.float32) - exp32)
        assert np.all(np.isfinite(out)), "non-finite output"
        assert np.all(err <= tol), (f"workspace={ws} columns={pg.shape[1]}: "
                                    f"max err {err.max():.3e}")
    return exp32


@pytest.mark.parametrize("layout", ["HND", "NHD"])
@pytest.mark.parametrize("dim", [64, 128])
def test_reference_packed_layouts(layout, dim, oracle):
    rng = np.random.default_rng(11)
    batch, hq, hkv = 3, 8, 2
    if layout == "HND":
        base = torch.from_numpy(rng.standard_normal((9, hkv, 16, 2 * dim)).astype(np.float16))
        cache = base.cuda()
        strides = (cache.stride(0), cache.stride(1), cache.stride(2), dim)
    else:
        base = torch.from_numpy(rng.standard_normal((9, 16, hkv, 2 * dim)).astype(np.float16))
        cache = base.cuda()  # physical NHD; logical HND view = transpose(1, 2)
        view = cache.transpose(1, 2)
        strides = (view.stride(0), view.stride(1), view.stride(2), dim)
    q = rng.standard_normal((batch, hq, dim)).astype(np.float16)
    pages = np.array([[4, 1], [2, 7], [8, 6]], dtype=np.int32)
    lengths = np.array([23, 9, 0], dtype=np.int32)
    exp32 = _run_both(q, cache, strides, hkv, 9, pages, lengths, 1 / math.sqrt(dim), oracle)
    # Closed-form pin of the oracle on the same inputs.
    closed = oracle_np.packed_decode(q, cache.cpu().numpy().reshape(-1), strides, hkv, 9,
                                     pages, lengths, 1 / math.sqrt(dim))
    G.gate(exp32, closed, 1e-5, "oracle vs closed form")
    assert np.all(exp32[2] == 0), "empty sequence must give zeros"


def test_five_dim_layout_small(oracle):
    """[P, 2, 16, Hkv, D]: K at block*16*2*Hkv*D + slot*Hkv*D + head*D, V at
    +16*Hkv*D (benchmark config 5's layout) at a small size."""
    rng = np.random.default_rng(3)
    P, hkv, d, hq, b = 40, 8, 128, 32, 5
    cache = torch.from_numpy(rng.standard_normal((P, 2, 16, hkv, d)).astype(np.float16)).cuda()
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    lengths = np.array([1, 16, 17, 200, 0], dtype=np.int32)
    perm = rng.permutation(P).astype(np.int32)
    pages = np.full((b, 13), -1, dtype=np.int32)
    cur = 0
    for i, n in enumerate(lengths):
        c = -(-int(n) // 16)
        pages[i, :c] = perm[cur:cur + c]
        cur += c
    q = rng.standard_normal((b, hq, d)).astype(np.float16)
    _run_both(q, cache, strides, hkv, P, pages, lengths, 0.07, oracle)


def test_unaligned_strides_take_the_scalar_path(oracle):
    """Strides that are not multiples of 8 elements still decode correctly."""
    rng = np.random.default_rng(13)
    P, hkv, d, hq, b = 6, 2, 64, 4, 2
    ss, hs = 2 * d + 1, 16 * (2 * d + 1) + 3
    bs = hkv * hs + 5
    flat = torch.from_numpy(rng.standard_normal(P * bs + 16).astype(np.float16)).cuda()
    strides = (bs, hs, ss, d)
    pages = np.array([[3, 0], [5, 1]], dtype=np.int32)
    lengths = np.array([20, 31], dtype=np.int32)
    q = rng.standard_normal((b, hq, d)).astype(np.float16)
    _run_both(q, flat, strides, hkv, P, pages, lengths, 0.125, oracle)


def test_config5_full_size(oracle):
    """benchmark config 5: B=64, contexts U[128, 4096], cache [20000,2,16,8,128],
    block-table rows = consecutive slices of a seeded permutation."""
    rng = np.random.default_rng(5)
    B, hq, hkv, d, NB, maxp = 64, 32, 8, 128, 20000, 256
    g = torch.Generator(device="cuda").manual_seed(5)
    cache = torch.randn((NB, 2, 16, hkv, d), generator=g, device="cuda", dtype=torch.float16)
    lengths = rng.integers(128, 4097, size=B).astype(np.int32)
    perm = rng.permutation(NB).astype(np.int32)
    pages = np.full((B, maxp), -1, dtype=np.int32)
    cur = 0
    for i, n in enumerate(lengths):
        c = -(-int(n) // 16)
        pages[i, :c] = perm[cur:cur + c]
        cur += c
    q = rng.standard_normal((B, hq, d)).astype(np.float16)
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    scale = 1 / math.sqrt(d)
    exp32, _ = oracle.packed_decode(q, cache.cpu().numpy(), pages, lengths, strides, hkv,
                                    scale, threads=16)
    for ws in (True, False):
        out = G.packed(q, cache, strides, hkv, NB, pages, lengths, scale, workspace=ws)
        err = np.abs(out.astype(np.float32) - exp32)
        assert np.all(err <= G.f16_tolerance(exp32, 2e-3)), f"ws={ws} max err {err.max():.3e}"


@pytest.mark.parametrize("lens", [[32768], [30000, 700]], ids=["one-32k", "long-and-short"])
def test_long_sequences_many_partials(lens, oracle):
    """A few long sequences cut by most of the 256 flat ranges: each output row
    has up to 256 partials, combined by four waves (a quarter each) and then
    through LDS."""
    torch.manual_seed(len(lens))
    rng = np.random.default_rng(len(lens))
    B, hq, hkv, d = len(lens), 32, 8, 128
    maxp = -(-max(lens) // 16)
    NB = sum(-(-n // 16) for n in lens) + 8
    cache = torch.randn((NB, 2, 16, hkv, d), device="cuda", dtype=torch.float16)
    lengths = np.array(lens, dtype=np.int32)
    perm = rng.permutation(NB).astype(np.int32)
    pages = np.full((B, maxp), -1, dtype=np.int32)
    cur = 0
    for i, n in enumerate(lens):
        c = -(-n // 16)
        pages[i, :c] = perm[cur:cur + c]
        cur += c
    q = rng.standard_normal((B, hq, d)).astype(np.float16)
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    scale = 1 / math.sqrt(d)
    assert G.lib().bc_packed_decode_workspace_size(capi.Shape(B, hq, hkv, d, maxp, NB)) > 0
    exp32, _ = oracle.packed_decode(q, cache.cpu().numpy(), pages, lengths, strides, hkv,
                                    scale, threads=16)
    out = G.packed(q, cache, strides, hkv, NB, pages, lengths, scale, workspace=True)
    err = np.abs(out.astype(np.float32) - exp32)
    assert np.all(err <= G.f16_tolerance(exp32, 2e-3)), f"max err {err.max():.3e}"


def test_large_batch_takes_split_path(oracle):
    """128 sequences (one wave of flat ranges at 8 KV heads) run split with a
    workspace; ragged lengths include empty sequences."""
    torch.manual_seed(128)
    rng = np.random.default_rng(128)
    B, hq, hkv, d = 128, 32, 8, 128
    lens = rng.integers(0, 801, size=B)
    lens[::9] = 0
    maxp = -(-int(lens.max()) // 16)
    NB = sum(-(-int(n) // 16) for n in lens) + 8
    cache = torch.randn((NB, 2, 16, hkv, d), device="cuda", dtype=torch.float16)
    lengths = lens.astype(np.int32)
    perm = rng.permutation(NB).astype(np.int32)
    pages = np.full((B, maxp), -1, dtype=np.int32)
    cur = 0
    for i, n in enumerate(lens):
        c = -(-int(n) // 16)
        pages[i, :c] = perm[cur:cur + c]
        cur += c
    q = rng.standard_normal((B, hq, d)).astype(np.float16)
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    scale = 1 / math.sqrt(d)
    assert G.lib().bc_packed_decode_workspace_size(capi.Shape(B, hq, hkv, d, maxp, NB)) > 0
    exp32, _ = oracle.packed_decode(q, cache.cpu().numpy(), pages, lengths, strides, hkv,
                                    scale, threads=16)
    for ws in (True, False):
        out = G.packed(q, cache, strides, hkv, NB, pages, lengths, scale, workspace=ws)
        err = np.abs(out.astype(np.float32) - exp32)
        assert np.all(err <= G.f16_tolerance(exp32, 2e-3)), f"ws={ws} max err {err.max():.3e}"


def _packed_fixture(rng, lens, hq, hkv, d, min_pages=1):
    lens = np.asarray(lens, dtype=np.int32)
    B = len(lens)
    maxp = max(min_pages, -(-int(lens.max()) // 16))
    NB = sum(-(-int(n) // 16) for n in lens) + 8
    cache = torch.randn((NB, 2, 16, hkv, d), device="cuda", dtype=torch.float16)
    perm = rng.permutation(NB).astype(np.int32)
    pages = np.full((B, maxp), -1, dtype=np.int32)
    cur = 0
    for i, n in enumerate(lens):
        c = -(-int(n) // 16)
        pages[i, :c] = perm[cur:cur + c]
        cur += c
    q = rng.standard_normal((B, hq, d)).astype(np.float16)
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    return q, cache, strides, NB, pages, lens


PAIR_CASES = {
    # 200 sequences of 3 pages over 128 ranges of 5 pages: ranges start on a
    # sequence's first page (its partial in slot 2r) and inside one (2r + 1)
    "3-page-sequences": (32, 8, 128, lambda rng: np.full(200, 48)),
    "ragged-with-empties": (32, 8, 128, lambda rng: np.where(np.arange(300) % 7 == 0, 0,
                                                             rng.integers(1, 601, size=300))),
    # three head blocks: 341 ranges; four: 256; 32 (no grouping): 32, or 64
    # at D = 64 (twice the ranges)
    "three-head-blocks": (48, 3, 128, lambda rng: rng.integers(0, 201, size=500)),
    "four-head-blocks": (32, 4, 128, lambda rng: rng.integers(1, 301, size=400)),
    "32-head-blocks": (32, 32, 64, lambda rng: rng.integers(0, 501, size=100)),
    # at most 64 sequences: range + sequence slots, the merge finds the
    # ranges from the lengths
    "32-head-blocks-60": (32, 32, 128, lambda rng: rng.integers(0, 301, size=60)),
}


@pytest.mark.parametrize("case", list(PAIR_CASES))
def test_batches_above_the_ranges_use_pair_slots(case, oracle):
    """Batches of more sequences than flat ranges (4 * CUs / head blocks,
    twice that at D = 64) split at any context length.  Above 64 sequences
    they keep two partial slots per range, a workspace of 2 * ranges slots
    whatever the batch; up to 64, ranges + batch slots.  The workspace call
    and the reference-signature call (its scratch a slot of the library's
    pool, where the workspace fits one) give the same bits, within the
    packed tolerance of the oracle."""
    hq, hkv, d, make = PAIR_CASES[case]
    rng = np.random.default_rng(len(case))
    torch.manual_seed(len(case))
    q, cache, strides, NB, pages, lens = _packed_fixture(rng, make(rng), hq, hkv, d)
    B = len(lens)
    zdim = hkv * -(-(hq // hkv) // 16)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    ranges = 4 * cus * (2 if d == 64 else 1) // zdim
    assert B > ranges
    need = G.lib().bc_packed_decode_workspace_size(capi.Shape(B, hq, hkv, d, pages.shape[1], NB))
    slots = 2 * ranges if B > 64 else ranges + B
    assert need == slots * hq * (d + 2) * 4 + ranges * 4, need
    scale = 1 / math.sqrt(d)
    exp32, _ = oracle.packed_decode(q, cache.cpu().numpy(), pages, lens, strides, hkv, scale,
                                    threads=16)
    outs = [G.packed(q, cache, strides, hkv, NB, pages, lens, scale, workspace=ws)
            for ws in (True, False)]
    for ws, out in zip((True, False), outs):
        err = np.abs(out.astype(np.float32) - exp32)
        assert np.all(err <= G.f16_tolerance(exp32, 2e-3)), f"ws={ws} max err {err.max():.3e}"
    if need <= capi.BC_SCRATCH_SLOT_BYTES:  # fits a pool slot: the same split
        assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))
    assert np.all(exp32[lens == 0] == 0) and np.all(outs[0][lens == 0] == 0)


def _one_long(rng):
    lens = rng.integers(0, 49, size=100)
    lens[37] = 6000  # 375 pages of about 575: more than 64 of the 128 ranges
    return lens


MID_CASES = {
    # 1-4 ranges per sequence (ranges of about 50 pages)
    "100-uniform": (lambda rng: rng.integers(16, 2049, size=100), 1),
    # one sequence cut by over 64 boundaries among short and empty ones
    "100-one-long": (_one_long, 1),
    # 128 sequences of 4 pages over 128 ranges of 4 pages: no range cuts a
    # sequence, every boundary row leaves at its record
    "128-aligned": (lambda rng: np.full(128, 64), 32),
    "72-ragged-empties": (lambda rng: np.where(np.arange(72) % 5 == 0, 0,
                                               rng.integers(1, 1500, size=72)), 1),
}


@pytest.mark.parametrize("case", list(MID_CASES))
def test_batches_above_64_merge_per_range_boundary(case, oracle):
    """Above 64 sequences, while the ranges number under four per sequence,
    packed decode keeps two partial slots per range and its merge takes one
    wave per range boundary, loading the range records, every part's (max,
    sum) and the first parts' accumulators in one round.  Rows whose
    sequence spans more parts than that round holds (over 64 here) load the
    rest after it.  Both entry points give the same bits, within the packed
    tolerance of the oracle; empty sequences give zeros."""
    hq, hkv, d = 32, 8, 128
    make, min_pages = MID_CASES[case]
    rng = np.random.default_rng(len(case) + 100)
    torch.manual_seed(len(case) + 100)
    q, cache, strides, NB, pages, lens = _packed_fixture(rng, make(rng), hq, hkv, d,
                                                          min_pages=min_pages)
    B = len(lens)
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    ranges = 4 * cus // 8
    assert 64 < B <= ranges < 4 * B
    need = G.lib().bc_packed_decode_workspace_size(capi.Shape(B, hq, hkv, d, pages.shape[1], NB))
    assert need == 2 * ranges * hq * (d + 2) * 4 + ranges * 4, need
    scale = 1 / math.sqrt(d)
    exp32, _ = oracle.packed_decode(q, cache.cpu().numpy(), pages, lens, strides, hkv, scale,
                                    threads=16)
    outs = [G.packed(q, cache, strides, hkv, NB, pages, lens, scale, workspace=ws)
            for ws in (True, False)]
    for ws, out in zip((True, False), outs):
        err = np.abs(out.astype(np.float32) - exp32)
        assert np.all(err <= G.f16_tolerance(exp32, 2e-3)), f"ws={ws} max err {err.max():.3e}"
    assert np.array_equal(outs[0].view(np.uint16), outs[1].view(np.uint16))
    assert np.all(outs[0][lens == 0] == 0)


def test_misaligned_workspace_is_ignored():
    """A workspace that is not 16-byte aligned is ignored: the call is
    bc_packed_decode's (whose split scratch is a slot of the library's pool)
    and gives its bits."""
    torch.manual_seed(41)
    rng = np.random.default_rng(41)
    B, hq, hkv, d, NB = 4, 8, 2, 64, 300
    cache = torch.randn((NB, 2, 16, hkv, d), device="cuda", dtype=torch.float16)
    lengths = rng.integers(900, 1281, size=B).astype(np.int32)
    pages = np.stack([rng.permutation(NB)[:80] for _ in range(B)]).astype(np.int32)
    q = rng.standard_normal((B, hq, d)).astype(np.float16)
    strides = (cache.stride(0), cache.stride(3), cache.stride(2), cache.stride(1))
    assert G.lib().bc_packed_decode_workspace_size(capi.Shape(B, hq, hkv, d, 80, NB)) > 0
    plain = G.packed(q, cache, strides, hkv, NB, pages, lengths, 0.125, workspace=False)
    shifted = G.packed(q, cache, strides, hkv, NB, pages, lengths, 0.125, workspace=True,
                       ws_offset=4)
    assert np.array_equal(plain, shifted)
