"""The standalone `branchcraft` driver (tests/driver): the reference's
`branchcraft test | bench | tree-bench` command line (src/main.cu:504-525)
with its CSV schemas (src/main.cu:451-453, 495-496).

CPU tests check the command-line contract without touching a GPU; GPU tests
run the driver's own oracle-gated test mode and the quick sweeps.
"""

import csv
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
DRIVER = ROOT / "tests" / "driver" / "_build" / "branchcraft"

DECODE_COLUMNS = ("gpu,sm,cuda_runtime,batch,query_heads,kv_heads,head_dim,context,page_size,"
                  "splits,single_us,split_us,speedup,max_abs_diff,kv_mib").split(",")
TREE_COLUMNS = ("gpu,sm,cuda_runtime,requests,tree_nodes,prefix_tokens,query_heads,kv_heads,"
                "head_dim,page_size,tree_us,expanded_us,latency_ratio,max_abs_diff,"
                "shared_kv_mib,expanded_kv_mib,memory_saving_pct").split(",")


def _driver():
    if not DRIVER.exists():
        pytest.fail(f"{DRIVER} is not built; run __graft_entry__.build()")
    return str(DRIVER)


def run(*args, timeout=240):
    return subprocess.run([_driver(), *args], capture_output=True, text=True, timeout=timeout)


def test_usage_and_argument_errors():
    r = run()
    assert r.returncode == 2 and "Usage: branchcraft test | bench | tree-bench" in r.stderr
    r = run("frobnicate")
    assert r.returncode == 1 and "unknown mode" in r.stderr


@pytest.mark.gpu
def test_driver_test_mode_passes():
    r = run("test")
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    assert "PASS 42 CPU-oracle checks" in r.stdout
    assert "tree CPU-oracle cases plus shared-page commit" in r.stdout


@pytest.mark.gpu
def test_driver_quick_benches_write_reference_csv(tmp_path):
    decode_csv, tree_csv = tmp_path / "decode.csv", tmp_path / "tree.csv"
    r = run("bench", "--quick", "--output", str(decode_csv))
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    r = run("tree-bench", "--quick", "--output", str(tree_csv))
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    with decode_csv.open() as f:
        rows = list(csv.DictReader(f))
        assert list(rows[0].keys()) == DECODE_COLUMNS
    assert len(rows) == 4
    for row in rows:
        assert float(row["max_abs_diff"]) <= 3e-4
        assert float(row["split_us"]) > 0 and row["sm"] == "gfx950"
    with tree_csv.open() as f:
        rows = list(csv.DictReader(f))
        assert list(rows[0].keys()) == TREE_COLUMNS
    assert len(rows) == 4
    for row in rows:
        assert float(row["max_abs_diff"]) <= 3e-4
        assert float(row["memory_saving_pct"]) > 0


@pytest.mark.gpu
@pytest.mark.parametrize("n", [1, 2, 3, 4, 5])
def test_driver_configs_pass_parity(n):
    r = run("config", str(n), timeout=600)
    print(r.stdout, r.stderr)
    assert r.returncode == 0, r.stderr
    assert f"config {n}" in r.stdout and "GB/s" in r.stdout
