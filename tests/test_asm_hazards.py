"""The shipped MFMA kernels keep a margin between every MFMA and the VALU
instructions that touch its registers.

Twelve builds of an earlier decode loop (the same page-processing body, the
last pages of a range peeled off the loop in nine of them) were compared on
an MI355X at benchmark config 5.  The nine peeled builds gave wrong outputs
(max error 0.17; three passing builds matched the oracle to 2.4e-4).  In
their gfx950 assembly, and in none of the passing ones, a VALU instruction
overwrites a register that a `v_mfma_f32_16x16x16_f16` issued 3 wait states
earlier reads as its accumulator input:

    v_mfma_f32_16x16x16_f16 v[4:7], v[0:1], v[8:9], v[50:53]
    ds_read_b64_tr_b16 ...   (x3)
    v_sub_f32_e32 v50, v44, v54

In those builds the register allocator ping-ponged the P.V accumulation
through a temporary (tmp = mfma(V, P_hi, acc); acc = mfma(V, P_lo, tmp))
and reused a freed accumulator register for a softmax temporary; the
compiler's hazard model accepts 3 wait states for that write-after-read,
the hardware evidently reads the accumulator later.  Every passing build,
and every kernel shipped now, keeps at least 10 wait states there, which is
what this test holds the compiled kernels to (the source builds them with
in-place accumulations).  The checker itself is pinned by planted assembly:
the failing sequence above must read as 3 wait states, padded sequences as
their padding.
"""

import pytest

import asm_hazards as H

MARGIN = 10  # fewest wait states any passing build had (the failing ones: 3)


def _scan_text(text: str, window: int = 12) -> dict:
    insts, labels = H.parse(text.strip().split("\n"))
    return H.scan(insts, labels, window)


def test_checker_reads_the_failing_sequence():
    bad = """
\tv_mfma_f32_16x16x16_f16 v[4:7], v[0:1], v[8:9], v[50:53]
\tds_read_b64_tr_b16 v[10:11], v146 offset:32
\tds_read_b64_tr_b16 v[12:13], v146 offset:64
\tds_read_b64_tr_b16 v[30:31], v146 offset:96
\tv_sub_f32_e32 v50, v44, v54
\ts_endpgm
"""
    assert _scan_text(bad)["WARC"] == 3


def test_checker_counts_nops_branches_and_kills():
    padded = """
\tv_mfma_f32_16x16x16_f16 v[4:7], v[0:1], v[8:9], v[4:7]
\ts_nop 7
\ts_cbranch_execz .LBB0_2
\tv_add_f32_e32 v9, v8, v8
.LBB0_2:
\tv_mov_b32_e32 v4, 0
\tv_add_f32_e32 v1, v5, v2
\ts_endpgm
"""
    best = _scan_text(padded)
    # taken branch: s_nop 7 (8) + s_cbranch (1) -> v_mov at 9 wait states;
    # fall-through adds the v_add: 10
    assert best["WAW"] == 9 and best["WARC"] == 9
    assert best["RAW"] == 10  # v5 read after the v_mov (which killed only v4)
    killed = """
\tv_mfma_f32_16x16x16_f16 v[4:7], v[0:1], v[8:9], v[12:15]
\tglobal_load_dword v12, v[2:3], off
\tv_mov_b32_e32 v12, 0
\ts_endpgm
"""
    assert "WARC" not in _scan_text(killed)  # v12 was reloaded before the write


@pytest.mark.parametrize("src", ["decode.hip", "tree_verify.hip"])
def test_shipped_kernels_keep_the_margin(compiled_kernels, src):
    found_mfma = 0
    for name, lines in compiled_kernels[src].items():
        insts, labels = H.parse(lines)
        if not any(op.startswith("v_mfma") for op, _ in insts):
            continue
        found_mfma += 1
        best = H.scan(insts, labels, window=MARGIN)
        for kind in ("WARC", "WAW"):
            assert best.get(kind, MARGIN) >= MARGIN, (name, kind, best)
    assert found_mfma >= 8, f"{src}: expected the MFMA kernels, found {found_mfma}"
