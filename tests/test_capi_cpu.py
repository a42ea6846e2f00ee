"""The C ABI loads without a GPU, exports every declared entry point and
rejects bad arguments with hipErrorInvalidValue before touching the device.

Rejection rules restate the reference's checks: src/paged_gqa.cu:124-129,
src/tree_attention.cu:94-99 and 111-114, src/packed_decode.cu:69-73 and the
driver's API test (src/main.cu:343-349).  No call here reaches a launch.
"""

import ctypes
import re
from pathlib import Path

import pytest

import branchcraft_capi as capi

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "branchcraft.h"
INVALID = capi.BC_ERROR_INVALID_VALUE
FAKE = 0x1000  # a non-null address; never dereferenced on the rejection path


def declared_symbols():
    text = HEADER.read_text()
    return sorted(set(re.findall(r"\b(bc_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = capi.load()
    names = declared_symbols()
    assert len(names) >= 11
    for name in names:
        assert hasattr(lib, name), f"{name} missing from {capi.LIB_PATH}"
    assert set(names) == set(capi.EXPORTED)
    assert b"gfx950" in lib.bc_version()


def _shape(**kw):
    base = dict(batch=2, query_heads=32, kv_heads=8, dim=128, max_pages=4, physical_pages=16)
    base.update(kw)
    return capi.Shape(**base)


def _inputs(**kw):
    base = dict(q=FAKE, k=FAKE, v=FAKE, pages=FAKE, lengths=FAKE, output=FAKE)
    base.update(kw)
    return capi.Inputs(**base)


BAD_DECODE = [
    ("dim96", dict(shape=dict(dim=96))),
    ("batch0", dict(shape=dict(batch=0))),
    ("hq_not_multiple", dict(shape=dict(query_heads=30))),
    ("kv0", dict(shape=dict(kv_heads=0))),
    ("max_pages0", dict(shape=dict(max_pages=0))),
    ("phys0", dict(shape=dict(physical_pages=0))),
    ("splits0", dict(splits=0)),
    ("splits_over_cap", dict(splits=capi.BC_MAX_SPLITS + 1)),
    ("null_q", dict(inputs=dict(q=None))),
    ("null_pages", dict(inputs=dict(pages=None))),
    ("null_out", dict(inputs=dict(output=None))),
    ("null_scratch_split2", dict(splits=2, scratch=(None, None))),
    ("half_scratch_split2", dict(splits=2, scratch=(FAKE, None))),
]


@pytest.mark.parametrize("name,case", BAD_DECODE, ids=[c[0] for c in BAD_DECODE])
def test_decode_rejects(name, case):
    lib = capi.load()
    shape = _shape(**case.get("shape", {}))
    ins = _inputs(**case.get("inputs", {}))
    scr = capi.Scratch(*case.get("scratch", (FAKE, FAKE)))
    assert lib.bc_decode(shape, ins, scr, case.get("splits", 1), None) == INVALID


def _tree_inputs(**kw):
    prefix = capi.Inputs(None, FAKE, FAKE, FAKE, FAKE, None)
    base = dict(draft_q=FAKE, draft_k=FAKE, draft_v=FAKE, parent=FAKE, output=FAKE)
    base.update(kw)
    return capi.TreeInputs(prefix, **base)


@pytest.mark.parametrize("nodes", [0, capi.BC_MAX_TREE_NODES + 1])
def test_tree_rejects_node_count(nodes):
    lib = capi.load()
    assert lib.bc_tree_verify(_shape(), _tree_inputs(), nodes, None) == INVALID
    assert lib.bc_tree_verify_ws(_shape(), _tree_inputs(), nodes, None, 0, None) == INVALID
    assert lib.bc_tree_verify_workspace_size(_shape(), nodes) == 0


@pytest.mark.parametrize("field", ["draft_q", "draft_k", "draft_v", "parent", "output"])
def test_tree_rejects_null(field):
    lib = capi.load()
    assert lib.bc_tree_verify(_shape(), _tree_inputs(**{field: None}), 7, None) == INVALID


def test_tree_rejects_bad_shape_and_null_prefix():
    lib = capi.load()
    assert lib.bc_tree_verify(_shape(dim=80), _tree_inputs(), 7, None) == INVALID
    for field in ("k", "v", "pages", "lengths"):
        ins = _tree_inputs()
        setattr(ins.prefix, field, None)
        assert lib.bc_tree_verify(_shape(), ins, 7, None) == INVALID, field
        assert lib.bc_tree_verify_ws(_shape(), ins, 7, None, 0, None) == INVALID, field
    for bad in (dict(batch=0), dict(kv_heads=0), dict(query_heads=30), dict(max_pages=0)):
        assert lib.bc_tree_verify(_shape(**bad), _tree_inputs(), 7, None) == INVALID, bad


def test_tree_accepts_any_pool_size():
    """The reference checks no pool size (src/tree_attention.cu:94-99):
    physical_pages < 1 is not rejected; it means the size is not given, and
    such calls need no workspace (they run the single pass)."""
    lib = capi.load()
    c3 = dict(batch=8, max_pages=129)
    assert lib.bc_tree_verify_workspace_size(_shape(**c3), 7) > 0
    for phys in (0, -1):
        assert lib.bc_tree_verify_workspace_size(_shape(physical_pages=phys, **c3), 7) == 0


@pytest.mark.parametrize("request_,nodes,accepted", [(-1, 7, 1), (2, 7, 1), (0, 0, 1),
                                                     (0, 7, 0), (0, 7, 8)])
def test_commit_rejects(request_, nodes, accepted):
    lib = capi.load()
    s = capi.Shape(2, 8, 8, 128, 1, 16)
    assert lib.bc_commit_path(s, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, request_, nodes,
                              accepted, None) == INVALID
    assert lib.bc_commit_path(capi.Shape(2, 8, 8, 96, 1, 16), FAKE, FAKE, FAKE, FAKE, FAKE,
                              FAKE, FAKE, 0, 7, 1, None) == INVALID


def test_commit_checks_are_the_reference_s():
    """bc_commit_path rejects what src/tree_attention.cu:111-114 rejects (a
    null pointer, a request outside [0, batch), nodes < 1, accepted outside
    [1, nodes], dim not 64/128) and nothing else: kv_heads < 1 is an empty
    copy (success, nothing launched), and physical_pages < 1 means the pool
    size is not given (covered on the GPU)."""
    lib = capi.load()
    args = [FAKE] * 7
    for i in range(7):
        bad = list(args)
        bad[i] = None
        assert lib.bc_commit_path(capi.Shape(2, 8, 8, 128, 1, 16), *bad, 0, 7, 1,
                                  None) == INVALID
    for kvh in (0, -3):
        for phys in (16, 0):
            s = capi.Shape(2, kvh, kvh, 128, 1, phys)
            assert lib.bc_commit_path(s, *args, 1, 7, 3, None) == capi.BC_SUCCESS
            assert lib.bc_commit_paths(s, *args[:4], FAKE, *args[4:], 7, 2,
                                       None) == capi.BC_SUCCESS
            assert lib.bc_copy_pages(capi.Shape(1, kvh, kvh, 64, 1, phys), FAKE, FAKE, FAKE,
                                     FAKE, 2, None) == capi.BC_SUCCESS


def test_commit_paths_rejects():
    lib = capi.load()
    s = capi.Shape(2, 8, 8, 128, 1, 16)
    args = [FAKE] * 8
    for i in range(8):  # every pointer is required
        bad = list(args)
        bad[i] = None
        assert lib.bc_commit_paths(s, *bad, 7, 1, None) == INVALID
    assert lib.bc_commit_paths(s, *args, 0, 1, None) == INVALID       # nodes < 1
    assert lib.bc_commit_paths(s, *args, 7, -1, None) == INVALID      # count < 0
    assert lib.bc_commit_paths(capi.Shape(0, 8, 8, 128, 1, 16), *args, 7, 1, None) == INVALID
    assert lib.bc_commit_paths(capi.Shape(2, 8, 8, 96, 1, 16), *args, 7, 1, None) == INVALID
    assert lib.bc_commit_paths(s, *args, 7, 0, None) == capi.BC_SUCCESS


def test_copy_pages_rejects():
    lib = capi.load()
    s = capi.Shape(1, 8, 8, 128, 1, 16)
    assert lib.bc_copy_pages(s, None, FAKE, FAKE, FAKE, 1, None) == INVALID
    assert lib.bc_copy_pages(s, FAKE, FAKE, FAKE, FAKE, -1, None) == INVALID
    assert lib.bc_copy_pages(s, FAKE, FAKE, FAKE, FAKE, 0, None) == capi.BC_SUCCESS


@pytest.mark.parametrize("strides,scale", [((0, 1, 1, 1), 0.1), ((1, 0, 1, 1), 0.1),
                                           ((1, 1, 0, 1), 0.1), ((1, 1, 1, 0), 0.1),
                                           ((8, 8, 8, 8), 0.0), ((8, 8, 8, 8), -1.0),
                                           ((8, 8, 8, 8), float("nan"))])
def test_packed_rejects(strides, scale):
    lib = capi.load()
    s = _shape()
    assert lib.bc_packed_decode(s, FAKE, FAKE, FAKE, FAKE, FAKE, *strides, scale,
                                None) == INVALID
    assert lib.bc_packed_decode_ws(s, FAKE, FAKE, FAKE, FAKE, FAKE, *strides, scale, None, 0,
                                   None) == INVALID


def test_noalloc_rejects_before_launch():
    """bc_packed_decode_noalloc checks its arguments, then rejects a shape
    whose split workspace exceeds the static scratch with
    hipErrorOutOfMemory -- all before touching a pointer or the GPU."""
    lib = capi.load()
    strides = (2 * 16 * 8 * 128, 128, 8 * 128, 16 * 8 * 128)
    ok = capi.Shape(64, 32, 8, 128, 256, 20000)
    assert lib.bc_packed_decode_workspace_size(ok) <= capi.BC_STATIC_SCRATCH_BYTES
    bad = capi.Shape(0, 32, 8, 128, 256, 20000)
    assert lib.bc_packed_decode_noalloc(bad, FAKE, FAKE, FAKE, FAKE, FAKE, *strides, 0.1,
                                        None) == INVALID
    # 200 sequences of 128 query heads split, and their partials (two slots
    # per range of 128: 17.0 MB) exceed the 16 MiB scratch
    big = capi.Shape(200, 128, 8, 128, 256, 20000)
    assert lib.bc_packed_decode_workspace_size(big) > capi.BC_STATIC_SCRATCH_BYTES
    assert lib.bc_packed_decode_noalloc(big, FAKE, FAKE, FAKE, FAKE, FAKE, *strides, 0.1,
                                        None) == capi.BC_ERROR_OUT_OF_MEMORY


def test_packed_workspace_fits_a_pool_slot():
    """Every packed decode workspace up to D = 128 on 256 CUs fits a slot of
    the scratch pool, so the reference-signature call splits wherever the
    workspace call does: 2R slots of Hq (D + 2) floats with R = 1024 / head
    blocks and head blocks >= Hq / 16 stay within 128 * 256 * 130 * 4 bytes
    plus the range records, whatever the batch and heads."""
    lib = capi.load()
    worst = 0
    for hq, hkv in ((128, 1), (128, 8), (64, 1), (32, 1), (16, 1), (8, 1), (32, 8), (48, 3),
                    (64, 64), (1, 1)):
        for batch in (1, 64, 1000, 100000):
            for d in (64, 128):  # D = 64 runs twice the ranges at half the slot size
                need = lib.bc_packed_decode_workspace_size(capi.Shape(batch, hq, hkv, d, 4096, 10**6))
                worst = max(worst, need)
                assert need <= capi.BC_SCRATCH_SLOT_BYTES, (hq, hkv, batch, d, need)
    assert worst >= 128 * 256 * 130 * 4  # the D = 128 bound is reached


def test_auto_splits_policy():
    """Split decode runs min((splits - 1) * batch + 1, R) flat page ranges,
    R = 4 * CUs / head blocks (one wave of workgroups at four waves per CU).
    Batches of R or more take two splits at any context length; smaller
    ones keep contexts below 512 tokens whole, stay whole while their
    (sequence, head block) workgroups fit the CUs at up to 768 tokens, and
    otherwise take the fewest splits whose ranges fill the wave."""
    lib = capi.load()
    assert lib.bc_auto_splits(_shape(batch=1), 63, 256) == 1  # tiny contexts stay whole
    # below 512 tokens small batches stay whole (src/paged_gqa.cu:135) ...
    for batch in (1, 64, 127):
        assert lib.bc_auto_splits(_shape(batch=batch), 511, 256) == 1
    # ... and batches of a wave of ranges or more split at any length
    for batch in (128, 512, 4096):
        assert lib.bc_auto_splits(_shape(batch=batch), 16, 256) == 2
    # short contexts whose (sequence, head block) workgroups fit the CUs run
    # unsplit: eight waves share each sequence's pages, no merge kernel
    assert lib.bc_auto_splits(_shape(batch=1), 512, 256) == 1
    assert lib.bc_auto_splits(_shape(batch=1), 768, 256) == 1
    assert lib.bc_auto_splits(_shape(batch=1), 769, 256) > 1
    assert lib.bc_auto_splits(_shape(batch=12), 1024, 256) > 1
    assert lib.bc_auto_splits(_shape(batch=16), 1024, 256) == 1
    assert lib.bc_auto_splits(_shape(batch=32), 1024, 256) == 1
    assert lib.bc_auto_splits(_shape(batch=33), 1024, 256) > 1
    assert lib.bc_auto_splits(_shape(batch=1), 1025, 256) > 1
    ranges = 4 * 256 // 8  # 8 KV heads of 4 query heads: 8 head blocks
    for batch in (1, 2, 4, 16, 64, 100, 127):
        s = lib.bc_auto_splits(_shape(batch=batch), 32768, 256)
        assert 1 <= s <= capi.BC_MAX_SPLITS
        assert (s - 1) * batch + 1 >= ranges  # a full wave of workgroups
        assert (s - 2) * batch + 1 < ranges  # one split fewer would leave CUs idle
    assert lib.bc_auto_splits(_shape(batch=1), 32768, 256) == 128
    assert lib.bc_auto_splits(_shape(batch=4), 32768, 256) == 33
    assert lib.bc_auto_splits(_shape(batch=64), 4096, 256) == 3
    for batch in (128, 200, 256, 257, 512, 1024):
        assert lib.bc_auto_splits(_shape(batch=batch), 4096, 256) == 2, batch
    # sixteen KV heads: 16 head blocks, 64 ranges
    assert lib.bc_auto_splits(_shape(batch=1, query_heads=16, kv_heads=16), 4096, 256) == 64
    # one KV head of 8 query heads: one head block, 1024 ranges; whole from
    # 256 sequences on (their workgroups fill the CUs)
    one = dict(query_heads=8, kv_heads=1)
    assert lib.bc_auto_splits(_shape(batch=1, **one), 32768, 256) == capi.BC_MAX_SPLITS
    assert lib.bc_auto_splits(_shape(batch=8, **one), 32768, 256) == 129
    assert lib.bc_auto_splits(_shape(batch=255, **one), 4096, 256) == 6
    for batch in (256, 600, 1024, 4096):
        assert lib.bc_auto_splits(_shape(batch=batch, **one), 4096, 256) == 1, batch
    # 32 query heads on one KV head: two head blocks, whole from 128 sequences
    two = dict(query_heads=32, kv_heads=1)
    assert lib.bc_auto_splits(_shape(batch=127, **two), 4096, 256) == 6
    assert lib.bc_auto_splits(_shape(batch=128, **two), 4096, 256) == 1
    # 32 query heads on 4 KV heads: four head blocks, 256 ranges
    assert lib.bc_auto_splits(_shape(batch=256, query_heads=32, kv_heads=4), 100, 256) == 2
    assert lib.bc_auto_splits(_shape(batch=255, query_heads=32, kv_heads=4), 100, 256) == 1


def test_workspace_sizes():
    lib = capi.load()
    c5 = capi.Shape(64, 32, 8, 128, 256, 20000)
    assert lib.bc_packed_decode_workspace_size(c5) > 0
    # Page tables of at most 768 tokens (1024 for batches whose (sequence,
    # head block) workgroups fill half the CUs or more) whose workgroups fit
    # the CUs run unsplit: no workspace.
    assert lib.bc_packed_decode_workspace_size(capi.Shape(4, 32, 8, 128, 8, 64)) == 0
    assert lib.bc_packed_decode_workspace_size(capi.Shape(4, 32, 8, 128, 48, 64)) == 0
    assert lib.bc_packed_decode_workspace_size(capi.Shape(4, 32, 8, 128, 49, 64)) > 0
    assert lib.bc_packed_decode_workspace_size(capi.Shape(32, 32, 8, 128, 64, 64)) == 0
    assert lib.bc_packed_decode_workspace_size(capi.Shape(32, 32, 8, 128, 65, 64)) > 0
    # Tables below 512 tokens split only for batches of a wave of ranges (128
    # at 32/8 heads) or more; from 512 on, batches whose workgroups
    # outnumber the CUs split too.
    assert lib.bc_packed_decode_workspace_size(capi.Shape(64, 32, 8, 128, 8, 64)) == 0
    assert lib.bc_packed_decode_workspace_size(capi.Shape(128, 32, 8, 128, 8, 64)) > 0
    assert lib.bc_packed_decode_workspace_size(capi.Shape(64, 32, 8, 128, 32, 64)) > 0
    # Partial slots per head: ranges + batch (C5: 128 + 64), or two per range
    # above 64 sequences while the ranges number under four per sequence,
    # whatever the batch; then one int per range for the merge kernel.
    row = 32 * (128 + 2) * 4  # one slot of every head: acc and (max, sum)
    assert lib.bc_packed_decode_workspace_size(c5) == (128 + 64) * row + 128 * 4
    for batch in (65, 100, 128):
        mid = capi.Shape(batch, 32, 8, 128, 64, 70000)
        assert lib.bc_packed_decode_workspace_size(mid) == 2 * 128 * row + 128 * 4, batch
    for batch in (129, 1024, 65536):
        big = capi.Shape(batch, 32, 8, 128, 64, 70000)
        assert lib.bc_packed_decode_workspace_size(big) == 2 * 128 * row + 128 * 4, batch
    assert lib.bc_packed_decode_workspace_size(capi.Shape(4, 32, 8, 96, 80, 64)) == 0
    c3 = capi.Shape(8, 32, 8, 128, 129, 160)
    assert lib.bc_tree_verify_workspace_size(c3, 7) > 0
    assert lib.bc_tree_verify_workspace_size(c3, 0) == 0
    # Trees split the prefix while splitting gives more waves a tile (eight
    # wave slots per CU): 17 requests (136 units) take three four-wave parts,
    # 24 and 32 requests one eight-wave pass.
    for batch, split in ((12, True), (16, True), (17, True), (20, True), (24, False),
                         (32, False)):
        size = lib.bc_tree_verify_workspace_size(capi.Shape(batch, 32, 8, 128, 129, 160), 7)
        assert (size > 0) == split, batch
    # Prefixes short enough that a single pass gives each of its eight waves
    # two tiles or fewer (16 tiles, drafts included) do not split.
    for batch in (1, 2, 4, 8):
        short = capi.Shape(batch, 32, 8, 128, 30, 160)  # 480 tokens + 1 draft tile
        assert lib.bc_tree_verify_workspace_size(short, 7) == 0
    # Three to five tiles per wave: a single pass once the (request, KV head)
    # units fill (tiles per wave - 1) eighths of the 256 CUs.
    for batch, pages, split in ((4, 31, True), (8, 31, False), (8, 47, True), (12, 47, False),
                                (12, 63, True), (16, 63, False), (16, 78, False), (16, 79, True),
                                (16, 81, True), (8, 81, True)):
        size = lib.bc_tree_verify_workspace_size(capi.Shape(batch, 32, 8, 128, pages, 160), 7)
        assert (size > 0) == split, (batch, pages)


def test_torch_ops_register_reference_schemas():
    """The op library loads on a GPU-less host and registers the reference's
    schemas verbatim (bindings/torch_ops.cpp:144-148)."""
    import torch
    import branchcraft_torch  # noqa: F401

    want = {
        "tree_verify": "branchcraft::tree_verify(Tensor q, Tensor prefix_k, Tensor prefix_v, "
                       "Tensor pages, Tensor lengths, Tensor draft_k, Tensor draft_v, "
                       "Tensor parent) -> Tensor",
        "packed_decode_out": "branchcraft::packed_decode_out(Tensor q, Tensor packed_kv, "
                             "Tensor pages, Tensor lengths, Tensor(a!) output, float scale) "
                             "-> Tensor(a!)",
        "commit_path_": "branchcraft::commit_path_(Tensor(a!) cache_k, Tensor(b!) cache_v, "
                        "Tensor draft_k, Tensor draft_v, Tensor path_nodes, "
                        "Tensor dest_pages, Tensor dest_slots, int request) -> ()",
    }
    for name, schema in want.items():
        assert str(getattr(torch.ops.branchcraft, name).default._schema) == schema
    # added ops: the page clone and the batched commit
    assert "commit_paths_(Tensor(a!) cache_k, Tensor(b!) cache_v" in str(
        torch.ops.branchcraft.commit_paths_.default._schema)
    assert "copy_pages_(Tensor(a!) cache_k" in str(torch.ops.branchcraft.copy_pages_.default._schema)
    # the reference's C++ decode as an op
    assert str(torch.ops.branchcraft.paged_decode.default._schema) == (
        "branchcraft::paged_decode(Tensor q, Tensor k, Tensor v, Tensor pages, "
        "Tensor lengths, int splits=0) -> Tensor")


def test_ops_have_no_cpu_fallback():
    import torch
    import branchcraft_torch as bc

    q = torch.zeros(1, 1, 4, 64, dtype=torch.float16)
    k = torch.zeros(1, 16, 2, 64, dtype=torch.float16)
    pages = torch.zeros(1, 1, dtype=torch.int32)
    with pytest.raises((NotImplementedError, RuntimeError)):
        bc.tree_verify(q, k, k, pages, torch.zeros(1, dtype=torch.int32),
                       torch.zeros(1, 1, 2, 64, dtype=torch.float16),
                       torch.zeros(1, 1, 2, 64, dtype=torch.float16),
                       torch.full((1, 1), -1, dtype=torch.int32))
