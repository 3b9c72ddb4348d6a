"""Target description: normalizes the worker's ``--describe-target-json`` into ``target.json``
(schema 3), as the reference's tileplan/src/tileplan/probe.py:23-97 does."""

from __future__ import annotations

import json
import subprocess
from pathlib import Path

from .plan import ABI, OPCODES

# The compiled gfx950 worker's constants (tiles_amd/csrc/worker_config.hpp).
FINGERPRINT = "decoder-gfx950-wave64-exchange-v4-b512"
THREADS = 512
ATTENTION_SHARED_BYTES = 8448


def normalize(raw: dict) -> dict:
    """probe.py:23-68: validate the executor's description; worker_count = CU count."""
    try:
        device, executor = raw["device"], raw["executor"]
        sm, active, block = device["sm_count"], executor["active_blocks_per_sm"], executor["threads_per_block"]
        capability = device["compute_capability"]
        if type(sm) is not int or sm < 1 or type(active) is not int or active < 1 or type(block) is not int or block < 1:
            raise ValueError("invalid residency or block size")
        if not isinstance(capability, list) or len(capability) != 2 or any(type(n) is not int or n < 0 for n in capability):
            raise ValueError("invalid compute capability")
        if device["cooperative_launch"] is not True or executor["abi"] != ABI or not OPCODES.issubset(set(executor["opcodes"])):
            raise ValueError("executor lacks required decoder capabilities")
        if not isinstance(executor["fingerprint"], str) or not executor["fingerprint"]:
            raise ValueError("missing compiled-kernel fingerprint")
        shared = executor["attention_shared_bytes"]
        if type(shared) is not int or shared < 1:
            raise ValueError("invalid attention shared-memory capacity")
    except (KeyError, TypeError) as exc:
        raise ValueError(f"incomplete target description: {exc}") from exc
    return {"schema_version": 3, "device": device, "executor": executor,
            "launch": {"worker_count": sm, "grid_blocks": sm, "threads_per_block": block,
                       "cooperative_grid_limit": sm * active}}


def mi355x_target(sm_count: int = 256) -> dict:
    """The normalized target of this worker on an MI355X, for planning without a device
    (the reference's tests use a fixture target the same way, test_decoder_planning.py:20-38)."""
    return normalize({
        "device": {"name": "AMD Instinct MI355X", "compute_capability": [9, 5], "sm_count": sm_count,
                   "cooperative_launch": True},
        "executor": {"abi": ABI, "opcodes": sorted(OPCODES), "active_blocks_per_sm": 1, "threads_per_block": THREADS,
                     "fingerprint": FINGERPRINT, "attention_shared_bytes": ATTENTION_SHARED_BYTES},
    })


def probe_library() -> dict:
    """Describe the live device through the C ABI (ti_describe_target)."""
    from ..runtime import describe_target, library

    t = describe_target()
    return normalize({
        "device": {"name": t.name.decode(), "compute_capability": [t.major, t.minor], "sm_count": t.sm_count,
                   "cooperative_launch": bool(t.cooperative_launch), "global_memory_bytes": t.global_memory_bytes},
        "executor": {"abi": library().ti_abi().decode(), "opcodes": sorted(OPCODES),
                     "active_blocks_per_sm": t.active_blocks_per_sm, "threads_per_block": t.threads_per_block,
                     "fingerprint": library().ti_fingerprint().decode(),
                     "attention_shared_bytes": t.attention_shared_bytes},
    })


def probe(executable: Path, out: Path) -> dict:
    """Run ``tile_runtime --describe-target-json`` and write target.json (probe.py:71-88)."""
    completed = subprocess.run([str(executable), "--describe-target-json"], text=True, capture_output=True, check=False)
    if completed.returncode:
        raise RuntimeError(f"target probe failed: {completed.stderr.strip() or completed.stdout.strip()}")
    target = normalize(json.loads(completed.stdout))
    out.parent.mkdir(parents=True, exist_ok=True)
    out.write_text(json.dumps(target, sort_keys=True, indent=2) + "\n")
    return target


def read_target(path: Path) -> dict:
    target = json.loads(Path(path).read_text())
    if target.get("schema_version") != 3 or target != normalize({"device": target["device"], "executor": target["executor"]}):
        raise ValueError("target.json is invalid or has an inconsistent launch")
    return target
