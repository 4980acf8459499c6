"""Build libqutai_amd.so (HIP, gfx950) in-tree with hipcc.

Each ``csrc/*.hip`` file is compiled to an object under ``qutai_amd/_build``
in parallel, then linked into ``qutai_amd/libqutai_amd.so`` next to this file.
The GPU code is compiled ahead of time for gfx950 only; there is no run-time
compilation and no other target.

Usage: ``python -m qutai_amd.build`` (or ``__graft_entry__.build()``).
"""
from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
SOURCES = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libqutai_amd.so"
ARCH = "gfx950"


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    path = Path(rocm) / "bin" / "hipcc"
    return str(path) if path.exists() else "hipcc"


def flags() -> list[str]:
    return [
        f"--offload-arch={ARCH}",
        "-O3",
        "-std=c++17",
        "-fPIC",
        # packed fp32 VALU forms are kept out of the generated code
        "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
        "-Wno-unused-command-line-argument",
        f"-I{ROOT / 'include'}",
        f"-I{SOURCES}",
    ]


def _compile(source: Path) -> Path:
    target = BUILD / (source.stem + ".o")
    command = [hipcc(), *flags(), "-c", str(source), "-o", str(target)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError(f"hipcc failed for {source.name}:\n{result.stderr}")
    return target


def build(verbose: bool = False) -> Path:
    """Compile every HIP source and link the shared library; returns its path."""
    BUILD.mkdir(exist_ok=True)
    sources = sorted(SOURCES.glob("*.hip"))
    workers = min(len(sources), max(1, min(8, os.cpu_count() or 1)))
    with ThreadPoolExecutor(workers) as pool:
        objects = list(pool.map(_compile, sources))
    temporary = LIBRARY.with_suffix(".so.tmp")
    command = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(temporary)]
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(temporary, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}", file=sys.stderr)
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
