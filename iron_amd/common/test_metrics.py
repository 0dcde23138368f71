"""pytest plugin: per-test metrics parsed from captured output, aggregated into one CSV.

Mirrors the reference harness's metrics collection (conftest.py:28-45 options, :60-166 the
reporter and its hooks, :204-211 repeated iterations):

* ``@pytest.mark.metrics(Name=regex, ...)`` on a test names the metrics it prints; each regex has
  a ``value`` group, e.g. ``Latency=r"Latency \\(us\\): (?P<value>[\\d\\.]+)"``;
* ``--iterations N`` runs every test N times (ids ``iter0``..``iterN-1``) so each metric gets
  N samples;
* ``--csv-output PATH`` is where the CSV goes: one row per test (its parametrisation without the
  iteration id) with the commit, date, ``Checks`` = passed/runs, and mean, median, min, max and
  stddev of every metric. Nothing is written when no test carried a ``metrics`` marker.

Defaults differ from the reference on purpose: one iteration (its default of five would run the
GPU parity suite five times) and the CSV only for runs with metric tests.
"""

from __future__ import annotations

import csv
import re
import statistics
import subprocess
from datetime import datetime
from pathlib import Path

import pytest

_NODEID = re.compile(r"^(?P<path>.+?::[^\[]+)(?:\[(?P<params>.*)\])?$")
_ITER = re.compile(r"(?:^|-)iter\d+(?=-|$)")
_PROP = "iron_metrics"


def _commit() -> str:
    try:
        out = subprocess.run(["git", "rev-parse", "HEAD"], capture_output=True, text=True,
                             check=True)
        return out.stdout.strip()
    except (OSError, subprocess.CalledProcessError):
        return "unknown"


def split_nodeid(nodeid: str) -> tuple[str, str]:
    """``path::test[iterK-params]`` -> (``path::test``, ``params``); an unparametrised test keeps
    its function name as the test name."""
    m = _NODEID.match(nodeid)
    if not m:
        return nodeid, nodeid.rsplit("::", 1)[-1]
    params = _ITER.sub("", m.group("params") or "").strip("-")
    return m.group("path"), params if params else m.group("path").rsplit("::", 1)[-1]


class MetricsTable:
    """Samples per (test path, test name): pass flags and every metric value found."""

    def __init__(self):
        self.samples: dict[tuple[str, str], dict[str, list]] = {}

    def add(self, path: str, name: str, passed: bool, output: str, patterns: dict) -> None:
        entry = self.samples.setdefault((path, name), {"passed": []})
        entry["passed"].append(bool(passed))
        for metric, pattern in patterns.items():
            found = re.search(pattern, output)
            if found:
                entry.setdefault(metric, []).append(float(found.group("value")))

    def rows(self, commit: str, date: str) -> list[dict]:
        out = []
        for (path, name), entry in sorted(self.samples.items()):
            runs = entry["passed"]
            row = {"Commit": commit, "Date": date, "Test Path": path, "Test": name,
                   "Checks": f"{sum(runs)}/{len(runs)}"}
            for metric, values in entry.items():
                if metric == "passed" or not values:
                    continue
                row[f"{metric} (mean)"] = statistics.mean(values)
                row[f"{metric} (median)"] = statistics.median(values)
                row[f"{metric} (min)"] = min(values)
                row[f"{metric} (max)"] = max(values)
                row[f"{metric} (stddev)"] = statistics.stdev(values) if len(values) > 1 else 0.0
            out.append(row)
        return out

    def write(self, path: Path, commit: str, date: str) -> int:
        rows = self.rows(commit, date)
        columns: dict[str, None] = {}
        for row in rows:
            columns.update(dict.fromkeys(row))
        path.parent.mkdir(parents=True, exist_ok=True)
        with open(path, "w", newline="") as f:
            w = csv.DictWriter(f, list(columns))
            w.writeheader()
            w.writerows(rows)
        return len(rows)


def pytest_addoption(parser):
    group = parser.getgroup("iron metrics")
    group.addoption("--csv-output", default="tests_latest.csv",
                    help="CSV file for the metrics of tests marked with @pytest.mark.metrics")
    group.addoption("--iterations", type=int, default=1,
                    help="run every test this many times (metric statistics over the runs)")


def pytest_configure(config):
    config.addinivalue_line("markers", "metrics(**patterns): metric regexes (group 'value') "
                                       "searched in the test's captured stdout")
    config.pluginmanager.register(_Collector(config), "iron-metrics-collector")


def pytest_generate_tests(metafunc):
    n = metafunc.config.getoption("--iterations")
    if n > 1:
        metafunc.fixturenames.append("_iteration")
        metafunc.parametrize("_iteration", range(n), ids=lambda i: f"iter{i}")


@pytest.hookimpl(hookwrapper=True)
def pytest_runtest_makereport(item, call):
    # the patterns travel with the report (user_properties survive pytest-xdist's transport),
    # so the process that logs reports -- the controller under xdist -- does the collection
    outcome = yield
    report = outcome.get_result()
    marker = item.get_closest_marker("metrics")
    if report.when == "call" and marker is not None:
        report.user_properties.append((_PROP, dict(marker.kwargs)))


class _Collector:
    def __init__(self, config):
        self.config = config
        self.table = MetricsTable()

    def pytest_runtest_logreport(self, report):
        if report.when != "call":
            return
        patterns = next((v for k, v in report.user_properties if k == _PROP), None)
        if patterns is not None:
            path, name = split_nodeid(report.nodeid)
            self.table.add(path, name, report.passed, report.capstdout, patterns)

    def pytest_sessionfinish(self, session):
        if not self.table.samples or hasattr(self.config, "workerinput"):
            return
        target = Path(self.config.getoption("--csv-output"))
        n = self.table.write(target, _commit(), datetime.now().strftime("%Y-%m-%d %H:%M:%S"))
        reporter = self.config.pluginmanager.get_plugin("terminalreporter")
        if reporter is not None:
            reporter.ensure_newline()
            reporter.write_line(f"metrics of {n} test(s) written to {target}")
