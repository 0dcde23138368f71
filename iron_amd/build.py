"""Build ``libiron_hip.so`` (the C-ABI library of the HIP kernels) in-tree for gfx950.

The library is built with plain ``hipcc`` (no torch extension machinery): every ``*.hip`` file
under ``iron_amd/csrc`` is compiled to an object in ``iron_amd/_build`` and linked into
``iron_amd/libiron_hip.so``. Objects are rebuilt when their source or any header is newer.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
REPO_DIR = PKG_DIR.parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libiron_hip.so"
ARCH = os.environ.get("IRON_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Packed fp32 VALU forms are kept out of every kernel (v_pk_{add,mul,fma}_f32).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-Wno-unused-command-line-argument",
    f"-I{REPO_DIR / 'include'}",
]


def _hipcc() -> str:
    exe = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(exe).exists():
        raise RuntimeError("hipcc not found; the MI355X build needs ROCm's hipcc")
    return exe


def _headers() -> list[Path]:
    return sorted(CSRC.glob("*.h")) + [REPO_DIR / "include" / "iron_hip.h"]


def _compile(src: Path, force: bool) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    newest_dep = max([src.stat().st_mtime] + [h.stat().st_mtime for h in _headers()])
    if force or not obj.exists() or obj.stat().st_mtime < newest_dep:
        cmd = [_hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stderr}")
    return obj


def build(force: bool = True, verbose: bool = False) -> Path:
    """Compile every HIP source and link ``libiron_hip.so``; returns the library path."""
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources in {CSRC}")
    workers = min(len(sources), int(os.environ.get("MAX_JOBS", "8")))
    with ThreadPoolExecutor(max_workers=workers) as ex:
        objs = list(ex.map(lambda s: _compile(s, force), sources))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    cmd = [_hipcc(), "-shared", f"--offload-arch={ARCH}", "-fPIC", *map(str, objs), "-o", str(tmp)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stderr}")
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"built {LIB_PATH} from {len(sources)} sources")
    return LIB_PATH


if __name__ == "__main__":
    build(force="--force" in sys.argv, verbose=True)
