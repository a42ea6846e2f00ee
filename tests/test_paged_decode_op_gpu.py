"""torch.ops.branchcraft.paged_decode: the reference's C++ paged GQA decode
(branchcraft::decode / auto_splits, include/branchcraft.hpp:39-41,
src/paged_gqa.cu:122-142) as a dispatcher op with FP32 output.

* benchmark configs 1 and 4 against the CPU oracle, with the op's own
  shape-only split choice (splits=0) and explicit split counts;
* the reference driver's empty and ragged cases (src/main.cu:320-326);
* opcheck schema/FakeTensor, torch.compile(inductor) equality and HIP-graph
  capture replayed several times with eager work in between;
* argument errors raise RuntimeError.
"""

import numpy as np
import pytest
import torch

import branchcraft_torch as bc
from oracle import oracle_np
import gpu_helpers as G

pytestmark = pytest.mark.gpu


def _dev(*arrays):
    return [torch.from_numpy(np.ascontiguousarray(a)).cuda() for a in arrays]


def test_config1_op_matches_oracle(oracle):
    rng = np.random.default_rng(1)
    perm = rng.permutation(64).astype(np.int32)
    pages = perm[:32].reshape(1, 32)
    lengths = np.array([512], dtype=np.int32)
    q = rng.standard_normal((1, 32, 128)).astype(np.float16)
    k = rng.standard_normal((64, 16, 8, 128)).astype(np.float16)
    v = rng.standard_normal((64, 16, 8, 128)).astype(np.float16)
    expected = oracle.decode(q, k, v, pages, lengths)
    args = _dev(q, k, v, pages, lengths)
    for splits in (0, 1, 2, 8):
        out = bc.paged_decode(*args, splits=splits)
        assert out.dtype == torch.float32 and out.shape == (1, 32, 128)
        G.gate(out.cpu().numpy(), expected, 3e-4, f"paged_decode C1 splits={splits}")


def test_config4_op_auto_splits_matches_oracle(oracle):
    rng = np.random.default_rng(4)
    lens = rng.integers(16384, 32769, size=4)
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, 4, 32, 8, 128, lens, spare=16,
                                                     sigma=1.0)
    expected = oracle.decode(q, k, v, pages, lengths, threads=16)
    args = _dev(q, k, v, pages, lengths)
    for splits in (0, 16):
        out = bc.paged_decode(*args, splits=splits).cpu().numpy()
        G.gate(out, expected, 2e-3, f"paged_decode C4 splits={splits}")
        G.gate(out, expected, 3e-4, f"paged_decode C4 splits={splits} (reference gate)")


@pytest.mark.parametrize("lens", [[0], [1], [17], [0, 37, 91], [513, 3]])
def test_reference_lengths(lens, oracle):
    rng = np.random.default_rng(17)
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, len(lens), 8, 2, 64, lens)
    expected = oracle.decode(q, k, v, pages, lengths)
    args = _dev(q, k, v, pages, lengths)
    for splits in (0, 1, 4):
        out = bc.paged_decode(*args, splits=splits).cpu().numpy()
        G.gate(out, expected, 3e-4, f"lengths={lens} splits={splits}")
        for b, n in enumerate(lens):
            if n == 0:
                assert not np.any(out[b])


def _small_case():
    rng = np.random.default_rng(29)
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, 3, 8, 2, 128, [40, 1100, 0])
    return _dev(q, k, v, pages, lengths), (q, k, v, pages, lengths)


def test_opcheck_compile_and_graph_replay(oracle):
    args, host = _small_case()
    expected = oracle.decode(*host)
    # A 69-column page table: the shape-only rule splits it, so the graph
    # holds the attention kernel, the merge and a scratch allocation.
    for splits in (0, 3):
        torch.library.opcheck(torch.ops.branchcraft.paged_decode, (*args, splits),
                              test_utils=("test_schema", "test_faketensor"))
    eager = bc.paged_decode(*args)
    G.gate(eager.cpu().numpy(), expected, 3e-4, "eager")
    compiled = torch.compile(bc.paged_decode, backend="inductor")
    torch.testing.assert_close(compiled(*args), eager)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = bc.paged_decode(*args)
    for i in range(4):
        out.fill_(float("nan"))
        junk = torch.randn(1024, 1024, device="cuda").sum()  # unrelated eager work
        graph.replay()
        torch.cuda.synchronize()
        G.gate(out.cpu().numpy(), expected, 3e-4, f"replay {i}")
        del junk


def test_argument_errors_raise():
    (q, k, v, pages, lengths), _ = _small_case()
    with pytest.raises(RuntimeError):
        bc.paged_decode(q, k, v, pages, lengths, splits=-1)
    with pytest.raises(RuntimeError):
        bc.paged_decode(q, k, v, pages, lengths, splits=257)
    with pytest.raises(RuntimeError):
        bc.paged_decode(q.float(), k, v, pages, lengths)
    with pytest.raises(RuntimeError):
        bc.paged_decode(q, k, v[:-1], pages, lengths)
    with pytest.raises(RuntimeError):
        bc.paged_decode(q, k, v, pages.long(), lengths)
