"""test_abi.py's validation cases under AddressSanitizer (CPU only).

tests/asan/Makefile builds the C-ABI library's host code with -fsanitize=address (host-only,
relocatable device code: the device link emits no kernels) and a Python interpreter linked with
the sanitizer, so that its runtime comes first in the process. That interpreter runs
tests/test_abi.py against the instrumented library (IRON_HIP_LIB): every null, shape, alignment
and workspace check of every entry point, with out-of-bounds reads and writes, use-after-free and
double frees in the host code reported as errors. Nothing is launched on a GPU.
"""

import os
import subprocess
from pathlib import Path

REPO = Path(__file__).resolve().parent.parent
ASAN = REPO / "tests" / "asan"


def test_abi_validation_under_address_sanitizer():
    r = subprocess.run(["make", "-s", "-j8"], cwd=ASAN, capture_output=True, text=True,
                       timeout=600)
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-4000:]
    env = dict(os.environ, IRON_HIP_LIB=str(ASAN / "_build" / "libiron_hip_asan.so"),
               ASAN_OPTIONS="detect_leaks=0:halt_on_error=1")
    r = subprocess.run([str(ASAN / "_build" / "pyasan"), "-m", "pytest", "-q", "-p",
                        "no:cacheprovider", str(REPO / "tests" / "test_abi.py")],
                       cwd=REPO, env=env, capture_output=True, text=True, timeout=600)
    out = r.stdout + r.stderr
    assert "AddressSanitizer" not in out, out[-6000:]
    assert r.returncode == 0 and " passed" in r.stdout, out[-4000:]
