"""Controlled decode timing: interleaved arms in resident processes, paired bootstrap, amd-smi
telemetry (the reference's tileinfer/tests/controlled_decode.py:1-26, for this runtime).

An arm is a package, optionally with another build of this library:
``NAME=PACKAGE`` or ``NAME=PACKAGE:LIBRARY_ROOT`` (a directory holding a built ``tiles_amd``
package that includes this module; the arm's server runs from there).  Each arm runs in a
resident server process (``python -m tiles_amd.controlled --serve``) that loads its package
once.  A round resets the context, prefills the context's
prompt and times one generation launch of ``--tokens`` tokens: microseconds per token from the
launch's HIP events, the unit bench.py reports.  For every context the arms run ``--blocks``
blocks of ``--rounds`` rounds (after one untimed round), in alternating order (forward, then
reversed), so drift reaches every arm alike.  A background ``amd-smi metric`` sampler records
power, clocks and temperatures, joined to every block by time.

Every arm is compared with the first through paired block differences: block i of two arms ran
next to each other in time, and a bootstrap over the pairs gives the 95% interval of the mean
difference.  Two arms of one package (an A/A run) measure the protocol's own resolution.  Rounds
further than OUTLIER_FRACTION from their arm's median at one context are excluded and counted
(a block none of whose rounds lies inside keeps them all).

Server placement biases a comparison: in an A/A run on MI355X the server started first was
0.4-0.8% faster than the second, steadily (each process uploads its own weights and buffers).
So halfway through each context's blocks every server is restarted in the reverse order; the
paired mean over both halves cancels a symmetric placement effect, and half the difference
between the halves' means is reported as that effect (``--no-swap`` keeps one spawn order).

    python -m tiles_amd.controlled --arm A=/tmp/llama4k --arm B=/tmp/llama4k --contexts 1 4096 \\
        --blocks 6 --rounds 5 --out report.json
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import statistics
import subprocess
import sys
import tempfile
import threading
import time
from pathlib import Path

import numpy as np

BOOTSTRAP = 10_000
OUTLIER_FRACTION = 0.01
ROOT = Path(__file__).resolve().parent.parent


def sha256(path: Path) -> str:
    return hashlib.sha256(Path(path).read_bytes()).hexdigest()


def prompt_for(context: int, vocab: int = 128256) -> list[int]:
    """The benchmark's prompts: Llama's BOS alone at context 1, else `context` seeded uniform
    tokens; for a model whose vocabulary lacks BOS, token 1 alone."""
    from . import synthetic as S

    if context == 1:
        return [S.BOS if S.BOS < vocab else 1]
    return S.prompt(context, seed=context, vocab=vocab)


# ---------------------------------------------------------------- the resident server

def serve(package: str) -> int:
    """Loads `package` once, then answers one JSON line per request line
    {"context": n, "rounds": r, "tokens": t, "warmup": w} with {"us_per_token": [...]}."""
    from . import runtime as R

    model = R.DecoderModel(R.load_plan(package, verify_weights=False))
    ctx = model.create_context()
    library = Path(R.library()._name)
    print(json.dumps({"ready": True, "library": str(library), "library_sha256": sha256(library),
                      "plan_sha256": sha256(Path(package) / "plan.json")}), flush=True)
    prompts: dict[int, list[int]] = {}
    vocab = json.loads((Path(package) / "plan.json").read_text())["model"].get("vocab_size", 128256)
    for line in sys.stdin:
        request = json.loads(line)
        n = int(request["context"])
        prompt = prompts.setdefault(n, prompt_for(n, vocab))
        times = []
        for k in range(int(request.get("warmup", 1)) + int(request["rounds"])):
            ctx.wait(ctx.enqueue_reset())
            ctx.wait(ctx.enqueue_prefill(prompt))
            result = ctx.wait(ctx.enqueue_generate(int(request["tokens"])))
            if k >= int(request.get("warmup", 1)):
                times.append(result.compute_us / int(request["tokens"]))
        print(json.dumps({"us_per_token": times}), flush=True)
    return 0


class Arm:
    def __init__(self, spec: str):
        name, _, rest = spec.partition("=")
        package, _, library_root = rest.partition(":")
        if not name or not package:
            raise SystemExit(f"arm {spec!r}: expected NAME=PACKAGE[:LIBRARY_ROOT]")
        self.name, self.package = name, package
        self.library_root = library_root or str(ROOT)
        env = dict(os.environ, PYTHONPATH=self.library_root)
        self.errors = tempfile.TemporaryFile(mode="w+")
        self.process = subprocess.Popen([sys.executable, "-m", "tiles_amd.controlled", "--serve", package],
                                        stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=self.errors, text=True,
                                        env=env, cwd=self.library_root)
        self.ready = json.loads(self._line())

    def _line(self) -> str:
        line = self.process.stdout.readline()
        if not line:
            status = self.process.wait(timeout=60)
            self.errors.seek(0)
            raise RuntimeError(f"{self.name}: server exited with status {status}: {self.errors.read()[-2000:]}")
        return line

    def measure(self, context: int, rounds: int, tokens: int) -> list[float]:
        self.process.stdin.write(json.dumps({"context": context, "rounds": rounds, "tokens": tokens}) + "\n")
        self.process.stdin.flush()
        return json.loads(self._line())["us_per_token"]

    def describe(self) -> dict:
        return {"package": self.package, "library_root": self.library_root, **self.ready}

    def close(self) -> None:
        if self.process.poll() is None:
            self.process.stdin.close()
        status = self.process.wait(timeout=120)
        if status != 0:
            self.errors.seek(0)
            raise RuntimeError(f"{self.name}: server failed with status {status}: {self.errors.read()[-2000:]}")


# ---------------------------------------------------------------- telemetry

def flatten(value, prefix: str = "") -> dict[str, float]:
    """Numeric leaves of an amd-smi JSON record, keyed by their path ("value" levels dropped)."""
    out: dict[str, float] = {}
    if isinstance(value, dict):
        if "value" in value and isinstance(value["value"], (int, float)):
            out[prefix] = float(value["value"])
        else:
            for k, v in value.items():
                out.update(flatten(v, f"{prefix}.{k}" if prefix else k))
    elif isinstance(value, list):
        for i, v in enumerate(value):
            out.update(flatten(v, f"{prefix}.{i}"))
    elif isinstance(value, (int, float)) and not isinstance(value, bool):
        out[prefix] = float(value)
    return out


class Telemetry:
    """Samples `amd-smi metric -g 0 -p -c -t --json` in a background thread."""

    def __init__(self, interval_s: float = 0.5):
        self.samples: list[tuple[float, dict]] = []
        self.available = True
        self._stop = threading.Event()
        self._interval = interval_s
        self._thread = threading.Thread(target=self._run, daemon=True)
        self._thread.start()

    def _run(self) -> None:
        while not self._stop.is_set():
            try:
                out = subprocess.run(["amd-smi", "metric", "-g", "0", "-p", "-c", "-t", "--json"], capture_output=True,
                                     text=True, timeout=10)
                data = json.loads(out.stdout)
                record = data["gpu_data"][0] if isinstance(data, dict) and "gpu_data" in data else data
                self.samples.append((time.time(), flatten(record)))
            except (OSError, ValueError, KeyError, IndexError, subprocess.TimeoutExpired):
                self.available = False
                return
            self._stop.wait(self._interval)

    def stop(self) -> None:
        self._stop.set()
        self._thread.join(timeout=15)

    def window(self, start: float, end: float) -> dict:
        """Mean of every telemetry value sampled in [start, end] (power, clocks, temperatures)."""
        inside = [s for t, s in self.samples if start <= t <= end]
        keys = [k for k in (inside[0] if inside else {}) if any(w in k for w in ("power", "clk", "clock", "temperature"))]
        return {"samples": len(inside), **{k: float(np.mean([s[k] for s in inside if k in s])) for k in keys}}


# ---------------------------------------------------------------- statistics

def paired(reference: list[float], other: list[float], seed: int) -> dict:
    """Mean of block-pair differences (other - reference), in us and in % of the reference, with
    a bootstrap 95% interval over the pairs."""
    d = np.asarray(other) - np.asarray(reference)
    rng = np.random.default_rng(seed)
    means = d[rng.integers(0, len(d), size=(BOOTSTRAP, len(d)))].mean(axis=1)
    low, high = np.percentile(means, [2.5, 97.5])
    base = float(np.mean(reference))
    return {"mean_us": float(d.mean()), "ci95_us": [float(low), float(high)], "mean_percent": 100 * float(d.mean()) / base,
            "ci95_percent": [100 * float(low) / base, 100 * float(high) / base], "pairs": len(d)}


def kept_rounds(blocks: list[list[float]], median: float) -> list[list[float]]:
    """Each block's rounds within OUTLIER_FRACTION of the arm's median at the context; a block
    with none inside keeps all of its rounds, so that every block has a median to pair."""
    kept = [[t for t in block if abs(t - median) <= OUTLIER_FRACTION * median] for block in blocks]
    return [k if k else list(block) for k, block in zip(kept, blocks)]


def spawn_order_effect(reference: list[float], other: list[float], half: int) -> dict:
    """The paired means of the blocks before and after the servers were restarted in the reverse
    order (block `half` on), and half their difference: the placement effect that the mean over
    both halves cancels when it is the same size either way round."""
    first = float(np.mean(np.subtract(other[:half], reference[:half])))
    second = float(np.mean(np.subtract(other[half:], reference[half:])))
    return {"first_half_mean_us": first, "second_half_mean_us": second, "spawn_order_effect_us": (first - second) / 2}


def main() -> int:
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--serve", help=argparse.SUPPRESS)
    parser.add_argument("--arm", action="append", default=[], help="NAME=PACKAGE[:LIBRARY_ROOT]; the first is the reference")
    parser.add_argument("--contexts", type=int, nargs="+", default=[1])
    parser.add_argument("--blocks", type=int, default=6)
    parser.add_argument("--rounds", type=int, default=5)
    parser.add_argument("--tokens", type=int, default=64)
    parser.add_argument("--no-swap", action="store_true", help="keep the first spawn order for every block")
    parser.add_argument("--out", type=Path)
    a = parser.parse_args()
    if a.serve:
        return serve(a.serve)
    if len(a.arm) < 2:
        parser.error("at least two --arm")
    spawn_order = list(a.arm)
    arms = [Arm(spec) for spec in spawn_order]
    names = [arm.name for arm in arms]
    telemetry = Telemetry()
    report = {"protocol": {"blocks": a.blocks, "rounds": a.rounds, "tokens": a.tokens, "warmup_rounds_per_block": 1,
                           "outlier_fraction": OUTLIER_FRACTION, "bootstrap": BOOTSTRAP, "order": "alternating",
                           "spawn_order_swapped_halfway": not a.no_swap},
              "arms": {arm.name: arm.describe() for arm in arms}, "contexts": {}}
    try:
        for n in a.contexts:
            raw = {name: [] for name in names}
            blocks = []
            spawned = {}
            for b in range(a.blocks):
                if not a.no_swap and a.blocks >= 2 and b == a.blocks // 2:
                    for arm in arms:
                        arm.close()
                    spawn_order = spawn_order[::-1]
                    arms = [Arm(spec) for spec in spawn_order]
                by_name = {arm.name: arm for arm in arms}
                spawned[b] = [arm.name for arm in arms]
                order = [by_name[name] for name in (names if b % 2 == 0 else names[::-1])]
                for arm in order:
                    start = time.time()
                    times = arm.measure(n, a.rounds, a.tokens)
                    end = time.time()
                    raw[arm.name].append(times)
                    blocks.append({"block": b, "arm": arm.name, "start": start, "end": end, "us_per_token": times,
                                   "telemetry": telemetry.window(start, end)})
                print(f"ctx {n} block {b} (spawned {', '.join(spawned[b])}): " +
                      "  ".join(f"{name} {statistics.median(raw[name][-1]):.1f}" for name in names), flush=True)
            summary = {}
            for name in names:
                every = [t for block in raw[name] for t in block]
                median = statistics.median(every)
                kept = kept_rounds(raw[name], median)
                summary[name] = {"median_us": median, "excluded_rounds": sum(len(x) for x in raw[name]) - sum(len(k) for k in kept),
                                 "block_medians_us": [statistics.median(k) for k in kept]}
            reference = names[0]
            half = a.blocks // 2
            for name in names[1:]:
                ref_blocks, blocks_of = summary[reference]["block_medians_us"], summary[name]["block_medians_us"]
                comparison = paired(ref_blocks, blocks_of, seed=n)
                if not a.no_swap and half >= 1:
                    comparison.update(spawn_order_effect(ref_blocks, blocks_of, half))
                summary[name]["vs_" + reference] = comparison
            report["contexts"][str(n)] = {"summary": summary, "blocks": blocks, "spawn_order_by_block": spawned}
            for name in names:
                s = summary[name]
                extra = ""
                if "vs_" + reference in s:
                    p = s["vs_" + reference]
                    extra = (f"  vs {reference}: {p['mean_us']:+.2f} us [{p['ci95_us'][0]:+.2f}, {p['ci95_us'][1]:+.2f}] "
                             f"({p['mean_percent']:+.3f}%)")
                    if "spawn_order_effect_us" in p:
                        extra += f"; spawn-order effect {p['spawn_order_effect_us']:+.2f} us"
                print(f"ctx {n} {name}: median {s['median_us']:.2f} us/token, {s['excluded_rounds']} rounds excluded{extra}",
                      flush=True)
    finally:
        telemetry.stop()
        for arm in arms:
            arm.close()
    report["telemetry_available"] = telemetry.available
    if a.out:
        a.out.write_text(json.dumps(report, indent=1) + "\n")
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
