"""Builds the gfx950 decode worker library and the ``tile_runtime`` command in-tree.

``python -m tiles_amd.build`` (or ``__graft_entry__.build()``) compiles every source with
hipcc for gfx950 and links ``tiles_amd/libtileinfer_amd.so`` and ``tiles_amd/tile_runtime``.
"""

from __future__ import annotations

import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
BUILD = PACKAGE / "_build"
LIBRARY = PACKAGE / "libtileinfer_amd.so"
CLI = PACKAGE / "tile_runtime"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")

SOURCES = ["worker_bf16.hip", "worker_f32.hip", "launch.hip", "static_exchange.hip", "prefill.hip", "lm_head.hip", "plan.cpp",
           "runtime.cpp", "json.cpp", "sha256.cpp"]
# Packed-FP32 instructions are kept out of every GPU code object (a known-bad form on this pool).
FLAGS = ["--offload-arch=gfx950", "-O3", "-std=c++20", "-fPIC", f"-I{ROOT / 'include'}", f"-I{CSRC}",
         "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wno-unused-command-line-argument"]


def _run(command: list[str]) -> None:
    result = subprocess.run(command, capture_output=True, text=True)
    if result.returncode:
        sys.stderr.write(result.stdout + result.stderr)
        raise RuntimeError(f"build step failed: {' '.join(command)}")


def _object(source: str) -> Path:
    out = BUILD / (source.replace(".", "_") + ".o")
    language = ["-x", "hip"] if source.endswith(".cpp") else []
    _run([HIPCC, *FLAGS, *language, "-c", str(CSRC / source), "-o", str(out)])
    return out


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    with ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as pool:
        objects = list(pool.map(_object, SOURCES))
    temporary = LIBRARY.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(temporary), *map(str, objects)])
    os.replace(temporary, LIBRARY)
    cli_object = _object("main.cpp")
    _run([HIPCC, "--offload-arch=gfx950", "-o", str(CLI), str(cli_object), f"-L{PACKAGE}", "-ltileinfer_amd",
          f"-Wl,-rpath,$ORIGIN"])
    if verbose:
        print(f"built {LIBRARY} and {CLI}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
