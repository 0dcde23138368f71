"""Operator tests in the reference harness's form: ``run_test`` (device copies of the inputs,
timed calls, ``verify_buffer`` on the outputs) under ``@pytest.mark.metrics``, printing the
Latency / Throughput / Effective Bandwidth lines whose values the metrics plugin collects into
the ``--csv-output`` CSV (reference: iron/operators/gemv_int8/test.py:40-110 and
iron/operators/rms_norm/test.py for the pattern; conftest.py:60-166 for the collection)."""

import pytest
import torch

from iron_amd.common.test_utils import run_test
from iron_amd.operators import RMSNorm, GEMVInt8
from iron_amd.operators.wire import pack_wire
from oracle import gemv as ogemv
from oracle import norms as onorm

pytestmark = pytest.mark.gpu

PATTERNS = dict(
    Latency=r"Latency \(us\): (?P<value>[\d\.]+)",
    Bandwidth=r"Effective Bandwidth: (?P<value>[\d\.e\+-]+) GB/s",
    Throughput=r"Throughput: (?P<value>[\d\.e\+-]+) GFLOP/s",
)


@pytest.mark.metrics(**PATTERNS)
@pytest.mark.parametrize("M,K,tile_m", [(4096, 1024, 16), (2048, 6144, 4)])
@pytest.mark.parametrize("domain", ["biased", "signed"])
def test_gemv_int8_run_test(M, K, tile_m, domain):
    print(f"[case] gemv run_test M={M} K={K} {domain}", flush=True)
    G = 32
    gen = torch.Generator().manual_seed(M + K)
    q = torch.randint(-127, 128, (M, K), generator=gen, dtype=torch.int16)
    s = (torch.randn(M, K // G, generator=gen) * 0.02).abs().to(torch.bfloat16)
    x = torch.randn(K, generator=gen).to(torch.bfloat16)
    op = GEMVInt8(M=M, K=K, tile_size_input=tile_m, group_size=G,
                  kernel_source=None if domain == "biased" else "mv_int8_signed.cc")
    wire = pack_wire(q, s, tile_m, domain).view(torch.bfloat16)
    want = ogemv.gemv_exact(q, s, x).float().to(torch.bfloat16)
    errors, latency_us, bandwidth_gbps = run_test(
        op, {"weights": wire, "vector": x}, {"output": want}, rel_tol=0.04, abs_tol=1e-2,
        warmup_iters=3, timed_iters=20)
    print(f"\nLatency (us): {latency_us:.2f}")
    print(f"Throughput: {2 * M * K / (latency_us * 1e-6) / 1e9:.6e} GFLOP/s")
    print(f"Effective Bandwidth: {bandwidth_gbps:.6e} GB/s\n")
    assert not errors, f"Test failed with errors: {errors}"


@pytest.mark.metrics(**PATTERNS)
@pytest.mark.parametrize("rows,cols", [(1, 1024), (16, 4096)])
def test_rmsnorm_run_test(rows, cols):
    print(f"[case] rmsnorm run_test rows={rows} cols={cols}", flush=True)
    gen = torch.Generator().manual_seed(rows + cols)
    x = (torch.randn(rows, cols, generator=gen) * 3).to(torch.bfloat16)
    w = (torch.rand(cols, generator=gen) + 0.5).to(torch.bfloat16)
    op = RMSNorm(size=rows * cols, num_aie_columns=1, num_channels=1, tile_size=cols,
                 weighted=True, epsilon=1e-6)
    errors, latency_us, bandwidth_gbps = run_test(
        op, {"input": x, "weight": w}, {"output": onorm.rms_norm(x, w, 1e-6)},
        rel_tol=0.0, abs_tol=0.0, warmup_iters=3, timed_iters=20)
    print(f"\nLatency (us): {latency_us:.2f}")
    print(f"Throughput: {4 * rows * cols / (latency_us * 1e-6) / 1e9:.6e} GFLOP/s")
    print(f"Effective Bandwidth: {bandwidth_gbps:.6e} GB/s\n")
    assert not errors, f"Test failed with errors: {errors}"
