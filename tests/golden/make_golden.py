"""Writes the golden vectors under tests/golden/ from the C oracle.

The reference ships no numeric golden files (its CSVs record only
max_abs_diff), so these vectors are the oracle's outputs on small seeded
inputs, each cross-checked against the float64 closed form when written and
again by tests/test_oracle.py.  Run: python tests/golden/make_golden.py
"""

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parent.parent))
from oracle import oracle_c, oracle_np  # noqa: E402


def main():
    rng = np.random.default_rng(2026)
    # decode: ragged batch with an empty row, non-power-of-two GQA
    q, k, v, pages, lengths = oracle_np.paged_fixture(rng, 3, 10, 2, 64, [0, 37, 91])
    exp = oracle_c.decode(q, k, v, pages, lengths)
    assert np.max(np.abs(exp - oracle_np.decode(q, k, v, pages, lengths))) < 2e-6
    np.savez(HERE / "decode_ragged_d64.npz", kind="decode", q=q, k=k, v=v, pages=pages,
             lengths=lengths, expected=exp)
    # tree: partial prefix page, random parents
    fix = oracle_np.tree_fixture(rng, 2, 17, 7, hq=8, hkv=2, d=64, parents="random")
    exp = oracle_c.tree(*fix)
    assert np.max(np.abs(exp - oracle_np.tree(*fix))) < 2e-6
    kk, vv, pg, ln, dq, dk, dv, par = fix
    np.savez(HERE / "tree_prefix17_d64.npz", kind="tree", k=kk, v=vv, pages=pg, lengths=ln,
             dq=dq, dk=dk, dv=dv, parent=par, expected=exp)
    # packed: NHD physical layout read as logical HND
    P, hkv, d = 9, 2, 64
    cache = rng.standard_normal((P, 16, hkv, 2 * d)).astype(np.float16)
    st = np.array([16 * hkv * 2 * d, 2 * d, hkv * 2 * d, d], dtype=np.int64)
    q = rng.standard_normal((3, 8, d)).astype(np.float16)
    pages = np.array([[4, 1], [2, 7], [8, 6]], dtype=np.int32)
    lengths = np.array([23, 9, 0], dtype=np.int32)
    exp, _ = oracle_c.packed_decode(q, cache, pages, lengths, st, hkv, 0.125)
    np.savez(HERE / "packed_nhd_d64.npz", kind="packed", q=q, cache=cache, pages=pages,
             lengths=lengths, strides=st, hkv=np.int32(hkv), scale=np.float64(0.125),
             expected=exp)


if __name__ == "__main__":
    main()
