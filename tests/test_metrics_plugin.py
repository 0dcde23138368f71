"""The metrics plugin (iron_amd/common/test_metrics.py) on the CPU: a throwaway test file run in
a child pytest with ``--iterations`` and ``--csv-output``, then the CSV's rows, columns and
statistics checked (reference behaviour: conftest.py:60-166, :204-211)."""

import csv
import os
import subprocess
import sys
from pathlib import Path

from iron_amd.common.test_metrics import MetricsTable, split_nodeid

REPO = Path(__file__).resolve().parent.parent

SAMPLE = '''
import pytest

RUNS = {}

@pytest.mark.metrics(Latency=r"Latency \\(us\\): (?P<value>[\\d\\.]+)",
                     Bandwidth=r"Effective Bandwidth: (?P<value>[\\d\\.e\\+-]+) GB/s")
@pytest.mark.parametrize("n", [1, 2])
def test_timed(n, request):
    k = RUNS[n] = RUNS.get(n, 0) + 1
    print(f"Latency (us): {10 * n + k}")
    print(f"Effective Bandwidth: {1.5e2 * n:.6e} GB/s")
    assert not (n == 2 and k == 3), "third run of n=2 fails"

def test_unmarked():
    print("Latency (us): 99")
'''


def _run(tmp_path, *args):
    (tmp_path / "test_sample.py").write_text(SAMPLE)
    env = dict(os.environ, PYTHONPATH=str(REPO))
    return subprocess.run([sys.executable, "-m", "pytest", "-q", "-p", "no:cacheprovider",
                           "-p", "iron_amd.common.test_metrics", *args, "test_sample.py"],
                          cwd=tmp_path, env=env, capture_output=True, text=True, timeout=120)


def test_csv_rows_and_statistics(tmp_path):
    out = tmp_path / "m.csv"
    r = _run(tmp_path, "--iterations", "3", "--csv-output", str(out))
    assert r.returncode == 1, r.stdout + r.stderr      # the planted failure
    # every test runs three times (the unmarked one too); one run of n=2 fails
    assert "8 passed" in r.stdout and "1 failed" in r.stdout, r.stdout
    rows = list(csv.DictReader(open(out)))
    assert [(x["Test Path"], x["Test"]) for x in rows] == [
        ("test_sample.py::test_timed", "1"), ("test_sample.py::test_timed", "2")]
    one, two = rows
    assert one["Checks"] == "3/3" and two["Checks"] == "2/3"
    # n=1 printed 11, 12, 13; n=2 printed 21, 22, 23 (the failing run's output still counts)
    assert float(one["Latency (mean)"]) == 12.0 and float(one["Latency (median)"]) == 12.0
    assert float(one["Latency (min)"]) == 11.0 and float(one["Latency (max)"]) == 13.0
    assert float(one["Latency (stddev)"]) == 1.0
    assert float(two["Latency (mean)"]) == 22.0
    assert float(two["Bandwidth (mean)"]) == 300.0 and float(two["Bandwidth (stddev)"]) == 0.0
    assert len(one["Commit"]) >= 7 and one["Date"]


def test_no_csv_without_metric_tests(tmp_path):
    out = tmp_path / "none.csv"
    r = _run(tmp_path, "--csv-output", str(out), "-k", "unmarked")
    assert r.returncode == 0, r.stdout + r.stderr
    assert not out.exists()


def test_nodeid_split_and_table():
    assert split_nodeid("a.py::t[iter2-4096-1024]") == ("a.py::t", "4096-1024")
    assert split_nodeid("a.py::t[4096-iter0]") == ("a.py::t", "4096")
    assert split_nodeid("a.py::t") == ("a.py::t", "t")
    t = MetricsTable()
    t.add("p", "x", True, "Latency (us): 5\n", {"Latency": r"Latency \(us\): (?P<value>[\d.]+)"})
    t.add("p", "x", False, "no number", {"Latency": r"Latency \(us\): (?P<value>[\d.]+)"})
    (row,) = t.rows("c", "d")
    assert row["Checks"] == "1/2" and row["Latency (mean)"] == 5.0 and row["Latency (stddev)"] == 0.0
