"""HBM traffic of the decode worker from rocprofv3 counter passes.

Four ``rocprofv3 --pmc`` passes, one counter each (the commands are in
``profiles/decoder_worker_llama1b_bf16_hbm_counters.md``):

* FETCH_SIZE and WRITE_SIZE over ``tile_runtime bench`` on a package (one round, no warmup);
* the same two counters over ``tile_runtime --measure-stream-read MIB 1``, whose fill and read
  dispatches move a known number of bytes and so calibrate each counter (FETCH_SIZE of a
  nontemporal read counts half of the bytes on this part: scale 2).

``summarize`` turns the four ``run_counter_collection.csv`` files into bytes per decoded token for
the generate launches, beside the algorithmic bytes, and stamps the summary with the SHA-256 of
the worker's sources, so that ``bench.py`` reports the figure as ``roofline.traffic`` only while
the kernel it was measured on is the one being benchmarked.

    python -m tiles_amd.counters --config ctx1 --first-position 1 --tokens-per-launch 64 \\
        --fetch DIR --write DIR --fetch-ref DIR --write-ref DIR --ref-mib 256 [--prefill-dispatches N] \\
        --out SUMMARY.json
"""

from __future__ import annotations

import argparse
import csv
import hashlib
import json
import statistics
from pathlib import Path

ROOT = Path(__file__).resolve().parent
KERNEL_SOURCES = ("csrc/worker_kernel.hpp", "csrc/worker_config.hpp", "csrc/device_common.hpp", "csrc/worker_bf16.hip")
WORKER = "decoder_worker"
WEIGHT_BYTES = 2_471_628_800      # Llama-3.2-1B bf16: every weight byte once per token
KV_BYTES_PER_POSITION = 32_768    # 16 layers x (K + V) x 8 heads x 64 x 2 bytes


def kernel_source_sha256() -> str:
    h = hashlib.sha256()
    for name in KERNEL_SOURCES:
        h.update(name.encode())
        h.update((ROOT / name).read_bytes())
    return h.hexdigest()


def algorithmic_bytes(position: int) -> int:
    """Bytes a token at `position` must move: the weights and the K/V of positions 0..position."""
    return WEIGHT_BYTES + (position + 1) * KV_BYTES_PER_POSITION


def dispatches(directory: Path, counter: str) -> list[tuple[str, float]]:
    """(kernel name, counter value in KiB) per dispatch, in dispatch order."""
    path = next(Path(directory).rglob("*counter_collection.csv"))
    rows = []
    with open(path, newline="") as f:
        for row in csv.DictReader(f):
            if row["Counter_Name"] == counter:
                rows.append((int(row["Dispatch_Id"]), row["Kernel_Name"], float(row["Counter_Value"])))
    rows.sort()
    return [(name, value) for _, name, value in rows]


def scale(directory: Path, counter: str, kernel: str, mib: int) -> float:
    """Bytes per counted KiB, from dispatches of `kernel` that move exactly `mib` MiB."""
    values = [v for name, v in dispatches(directory, counter) if kernel in name]
    if not values:
        raise ValueError(f"no {kernel} dispatch in {directory}")
    return mib * 1024.0 / statistics.median(values) * 1024.0


def summarize(config: str, first_position: int, tokens_per_launch: int, fetch: Path, write: Path, fetch_ref: Path,
              write_ref: Path, ref_mib: int, prefill_dispatches: int = 1) -> dict:
    fetch_scale = scale(fetch_ref, "FETCH_SIZE", "stream_read", ref_mib)
    write_scale = scale(write_ref, "WRITE_SIZE", "fillBuffer", ref_mib)
    fetched = [v for name, v in dispatches(fetch, "FETCH_SIZE") if WORKER in name]
    written = [v for name, v in dispatches(write, "WRITE_SIZE") if WORKER in name]
    if len(fetched) != len(written) or len(fetched) <= prefill_dispatches:
        raise ValueError("the two passes must record the same worker dispatches (prefill, then generate launches)")
    # A bench round's first worker dispatches are its prefill; the rest are generate launches.
    launches = []
    for k, (f, w) in enumerate(zip(fetched[prefill_dispatches:], written[prefill_dispatches:])):
        first = first_position + k * tokens_per_launch
        algorithmic = sum(algorithmic_bytes(p) for p in range(first, first + tokens_per_launch))
        launches.append({"fetch_bytes": f * fetch_scale, "write_bytes": w * write_scale, "algorithmic_bytes": algorithmic})
    traffic = sum(x["fetch_bytes"] + x["write_bytes"] for x in launches) / len(launches)
    algorithmic = sum(x["algorithmic_bytes"] for x in launches) / len(launches)
    return {"config": config, "source_sha256": kernel_source_sha256(),
            "calibration": {"fetch_bytes_per_kib": fetch_scale, "write_bytes_per_kib": write_scale, "reference_mib": ref_mib},
            "tokens_per_launch": tokens_per_launch, "launches": launches,
            "traffic_bytes_per_launch": traffic, "algorithmic_bytes_per_launch": algorithmic,
            "traffic_bytes_per_token": traffic / tokens_per_launch, "ratio": traffic / algorithmic}


def load(path: Path, config: str) -> dict | None:
    """The summary of `config` in a file written by ``--out``, if it was measured on the current
    worker sources; None otherwise."""
    try:
        data = json.loads(Path(path).read_text())
    except (OSError, ValueError):
        return None
    entry = data.get(config)
    if not entry or entry.get("source_sha256") != kernel_source_sha256():
        return None
    return entry


def main() -> int:
    parser = argparse.ArgumentParser()
    parser.add_argument("--config", required=True)
    parser.add_argument("--first-position", type=int, required=True, help="position of the first generated token")
    parser.add_argument("--tokens-per-launch", type=int, default=64)
    for name in ("fetch", "write", "fetch-ref", "write-ref"):
        parser.add_argument(f"--{name}", type=Path, required=True)
    parser.add_argument("--ref-mib", type=int, default=256)
    parser.add_argument("--prefill-dispatches", type=int, default=1, help="worker dispatches of the prefill (64 steps each)")
    parser.add_argument("--out", type=Path, required=True, help="JSON file of summaries keyed by config (updated in place)")
    a = parser.parse_args()
    entry = summarize(a.config, a.first_position, a.tokens_per_launch, a.fetch, a.write, a.fetch_ref, a.write_ref, a.ref_mib,
                      a.prefill_dispatches)
    data = json.loads(a.out.read_text()) if a.out.exists() else {}
    data[a.config] = entry
    a.out.write_text(json.dumps(data, indent=1) + "\n")
    print(json.dumps({k: v for k, v in entry.items() if k != "launches"}))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
