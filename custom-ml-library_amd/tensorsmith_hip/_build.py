"""Build ``libtsattn.so`` from ``custom-ml-library_amd/csrc/*.hip`` for gfx950.

Every translation unit is compiled with hipcc for gfx950 only, with packed
fp32 instructions disabled (``-Xclang -target-feature -Xclang
-packed-fp32-ops``), then linked into one shared library placed inside the
package (``tensorsmith_hip/_native/libtsattn.so``) so it ships with the tree.

    python -m tensorsmith_hip._build            # from custom-ml-library_amd/
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
CSRC = PKG.parent / "csrc"
INCLUDE = PKG.parents[1] / "include"
NATIVE = PKG / "_native"
LIB = NATIVE / "libtsattn.so"
ARCH = "gfx950"

FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-result",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
    f"-I{CSRC}",
]


# Per-source extra hipcc flags (none needed at present).
EXTRA_FLAGS: dict[str, list[str]] = {}


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found; the HIP toolchain is required to build libtsattn.so")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        msg = "\n".join(line for line in proc.stderr.splitlines()
                        if "packed-fp32-ops" not in line)
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{msg}")


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every csrc/*.hip and link libtsattn.so; returns the library path."""
    cc = hipcc()
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objdir = NATIVE / "obj"
    objdir.mkdir(parents=True, exist_ok=True)
    objects = [objdir / (s.stem + ".o") for s in sources]

    def compile_one(pair):
        src, obj = pair
        cmd = [cc, *FLAGS, *EXTRA_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
        if verbose:
            print(" ".join(cmd), flush=True)
        _run(cmd)

    workers = jobs or min(len(sources), max(1, (os.cpu_count() or 2) // 2), 8)
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(compile_one, zip(sources, objects)))
    tmp = LIB.with_suffix(".so.tmp")
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)])
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB}", flush=True)
    return LIB


if __name__ == "__main__":
    build(verbose="-v" in sys.argv)
