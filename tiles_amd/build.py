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
# The stress build: the same library with the worker compiled with TILES_DELAY_INJECTION (random
# sleeps before every exchange publish and poll), for tests/test_gpu_delay_injection.py.
DELAY_LIBRARY = PACKAGE / "libtileinfer_amd_delay.so"
WORKER_SOURCES = ("worker_bf16.hip", "worker_f32.hip")
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


def _object(source: str, delay: bool = False) -> Path:
    out = BUILD / (source.replace(".", "_") + ("_delay" if delay else "") + ".o")
    language = ["-x", "hip"] if source.endswith(".cpp") else []
    defines = ["-DTILES_DELAY_INJECTION=1"] if delay else []
    _run([HIPCC, *FLAGS, *defines, *language, "-c", str(CSRC / source), "-o", str(out)])
    return out


def _link(library: Path, objects: list[Path]) -> None:
    temporary = library.with_suffix(".so.tmp")
    _run([HIPCC, "--offload-arch=gfx950", "-shared", "-fPIC", "-o", str(temporary), *map(str, objects)])
    os.replace(temporary, library)


def build(verbose: bool = False) -> Path:
    BUILD.mkdir(exist_ok=True)
    jobs = [(source, False) for source in SOURCES] + [(source, True) for source in WORKER_SOURCES]
    with ThreadPoolExecutor(max_workers=8) as pool:
        built = list(pool.map(lambda job: _object(*job), jobs))
    objects, delayed = built[: len(SOURCES)], dict(zip(WORKER_SOURCES, built[len(SOURCES):]))
    _link(LIBRARY, objects)
    _link(DELAY_LIBRARY, [delayed.get(source, obj) for source, obj in zip(SOURCES, objects)])
    cli_object = _object("main.cpp")
    _run([HIPCC, "--offload-arch=gfx950", "-o", str(CLI), str(cli_object), f"-L{PACKAGE}", "-ltileinfer_amd",
          f"-Wl,-rpath,$ORIGIN"])
    if verbose:
        print(f"built {LIBRARY}, {DELAY_LIBRARY} and {CLI}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
