"""Timeline and loss budget of one decoded token (the reference's
tileplan/src/tileplan/timeline.py:1-286, for this worker's clock and synchronization).

With the timeline on (``SequenceContext.set_timeline``), every instruction of a launch's last
step records four 100 MHz device-clock values (``s_memrealtime``, one clock for the whole GPU,
so no per-CU fit is needed as for the reference's per-SM cycle counters): its start, when its
first exchange read returned, when its last exchange wait ended ("ready"), and its end.

The loss budget partitions the traced step into waves.  The reference delimits waves by grid
barriers; this worker has none, so wave w's interval runs from E(w-1) to E(w), where E(w) is
the latest end of any task of waves 0..w (E(-1) is the step's first start).  The intervals
tile the traced time exactly.  Each interval splits into four signed columns:

* sync: E(w-1) until the first task of wave w sees its inputs (exchange latency: the last
  producer's publish reaching a consumer, the counterpart of the reference's barrier release);
* ideal: the wave's algorithmic bytes at the measured streaming bandwidth;
* work: the mean worker's finish (idle workers and early finishers count at the first ready)
  after the first ready, less ideal -- negative when weight loads issued before the wait
  already streamed part of the wave;
* tail: E(w) less that mean finish, the time the slowest worker adds.

By phase, sync + ideal + work + tail is the phase's share of the step, and over the step
ideal + barrier_sync + streaming_excess + attention_excess + small_phases equals the traced
time, as in the reference's budget (timeline.py:184-286).
"""

from __future__ import annotations

from collections import defaultdict
from dataclasses import asdict, dataclass
from html import escape

import numpy as np

TICK_NS = 10.0  # s_memrealtime runs at 100 MHz

PHASES = ("embedding", "qkv", "attention", "wo", "ffn", "ffn_reduce", "final_norm", "lm_head")
# Phases whose time is set by streaming weights or the K/V cache; the FFN reduction streams
# nothing but completes the down projection, so its excess counts here (timeline.py:49-53).
STREAMING = ("qkv", "wo", "ffn", "ffn_reduce", "lm_head")
COLORS = {"embedding": "#94a3b8", "qkv": "#22c55e", "attention": "#f472b6", "wo": "#16a34a", "ffn": "#15803d",
          "ffn_reduce": "#166534", "final_norm": "#1d4ed8", "lm_head": "#0f766e", "wait": "#e2e8f0"}


@dataclass(frozen=True)
class Event:
    """One executed task on a nanosecond axis whose 0 is the traced step's first start."""

    worker: int
    task: int
    start: float
    read: float | None   # first exchange read returned (None: the task read no exchange word)
    ready: float | None  # last exchange wait ended
    end: float


@dataclass(frozen=True)
class Wave:
    """One wave's interval, split as described in the module docstring."""

    wave: int
    phase: str
    bytes: int
    duration_ns: float
    ideal_ns: float
    work_ns: float
    tail_ns: float
    sync_ns: float
    busy_workers: int


def phase(task: dict) -> str:
    """The decoder phase of a plan task (timeline.py:79-94)."""
    return {"embedding": "embedding", "qkv": "qkv", "attention_scores": "attention", "attention_values": "attention",
            "output_projection": "wo", "ffn": "ffn", "ffn_reduce": "ffn_reduce", "final_rms_norm": "final_norm",
            "logits": "lm_head"}[task["opcode"].rsplit("_", 1)[0]]


def active_chunks(model: dict, position: int) -> int:
    """Attention chunks with work at `position` (ops.cuh active_chunks; timeline.py:97-102)."""
    length = position + 1
    if length <= model["attention_fused_steps"]:
        return 1
    return max(2, -(-length // model["attention_chunk_steps"]))


def streamed_bytes(task: dict, model: dict, position: int) -> int:
    """Weight and K/V bytes a task must read at `position`; activations are not counted
    (timeline.py:113-132).  This worker's scores task of a chunk reads the chunk's K and V rows
    of its K/V head (the values task only names the chunk)."""
    element = 2 if model["weight_dtype"] == "bfloat16" else 4
    op = task["opcode"].rsplit("_", 1)[0]
    d = model["hidden_size"]
    if op == "attention_values":
        return 0
    if op == "attention_scores":
        length, chunks = position + 1, active_chunks(model, position)
        chunk = task["operands"]["chunk"]
        if chunk >= chunks:
            return 0
        steps = length * (chunk + 1) // chunks - length * chunk // chunks
        return 2 * steps * model["head_dim"] * element
    if op == "final_rms_norm":
        return 0
    begin, end = task["operands"]["rows"]
    # This worker's FFN chunk streams its gate and up rows; the reduction wave streams the Wdown
    # rows of its outputs (the down projection, re-laid out row-major at upload).
    width = {"embedding": 1, "ffn": 2 * d, "ffn_reduce": model["intermediate_size"]}.get(op, d)
    return (end - begin) * width * element


def instruction_map(plan: dict) -> list[tuple[int, int, int]]:
    """(worker, wave, task id or -1 for a barrier) per encoded instruction, in the loader's order
    (worker streams concatenated; each wave's tasks, then a barrier except after the last wave)."""
    waves = plan["waves"]
    workers = plan["target"]["worker_count"]
    out = []
    for worker in range(workers):
        for index, wave in enumerate(waves):
            out += [(worker, index, task) for task in wave["workers"][worker]]
            if index + 1 < len(waves):
                out.append((worker, index, -1))
    return out


def events(plan: dict, stamps: np.ndarray) -> list[Event]:
    """The traced step's tasks on a common nanosecond axis.  Barrier records and instructions
    that did not run (start 0) are dropped."""
    stamps = np.asarray(stamps, dtype=np.uint64).reshape(-1, 4)
    imap = instruction_map(plan)
    if len(imap) != len(stamps):
        raise ValueError("timeline does not match the plan's instruction count")
    kept = [(worker, task, row) for (worker, _, task), row in zip(imap, stamps) if task >= 0 and row[0] != 0]
    if not kept:
        raise ValueError("the timeline holds no executed task")
    origin = min(int(row[0]) for _, _, row in kept)

    def ns(tick) -> float:
        return (int(tick) - origin) * TICK_NS

    out = []
    for worker, task, (start, read, ready, end) in kept:
        if int(end) < int(start):
            raise ValueError(f"task {task} on worker {worker} ends before it starts")
        out.append(Event(worker, task, ns(start), ns(read) if read else None, ns(ready) if ready else None, ns(end)))
    return out


def budget(plan: dict, stamps: np.ndarray, position: int, bandwidth_gbps: float) -> dict:
    """Decompose the traced step into ideal streaming and named losses (timeline.py:184-286)."""
    tasks = plan["tasks"]
    model = plan["model"]
    workers = plan["target"]["worker_count"]
    evs = events(plan, stamps)
    by_wave: dict[int, list[Event]] = defaultdict(list)
    for e in evs:
        by_wave[tasks[e.task]["wave"]].append(e)
    order = sorted(by_wave)
    previous = 0.0
    waves, rows = [], []
    for w in order:
        members = by_wave[w]
        end = max(previous, max(e.end for e in members))
        readies = [e.ready for e in members if e.ready is not None]
        first_ready = min(max(min(readies), previous), end) if readies else previous
        finish = {worker: first_ready for worker in range(workers)}
        for e in members:
            finish[e.worker] = max(finish[e.worker], min(max(e.end, first_ready), end))
        mean = sum(finish.values()) / workers
        unique = sum(streamed_bytes(tasks[e.task], model, position) for e in members)
        ideal = unique / bandwidth_gbps  # bytes / (GB/s) = ns
        names = [phase(tasks[e.task]) for e in members]
        wave = Wave(wave=w, phase=max(set(names), key=names.count), bytes=unique, duration_ns=end - previous,
                    ideal_ns=ideal, work_ns=mean - first_ready - ideal, tail_ns=end - mean,
                    sync_ns=first_ready - previous, busy_workers=len({e.worker for e in members}))
        waves.append(wave)
        # The wave's last-finishing task: start, first read and ready after its own start.
        last = max(members, key=lambda e: e.end)
        rows.append({**asdict(wave), "opcode": tasks[last.task]["opcode"].rsplit("_", 1)[0],
                     "us": wave.duration_ns / 1e3, "ideal_us": ideal / 1e3,
                     "span_us": (max(e.end for e in members) - min(e.start for e in members)) / 1e3,
                     "last_task_us": [(last.read - last.start) / 1e3 if last.read is not None else None,
                                      (last.ready - last.start) / 1e3 if last.ready is not None else None,
                                      (last.end - last.start) / 1e3],
                     "last_start_after_previous_us": (last.start - previous) / 1e3})
        previous = end

    phases = {}
    for name in PHASES:
        group = [w for w in waves if w.phase == name]
        if not group:
            continue
        duration = sum(w.duration_ns for w in group) / 1e3
        values = {"waves": len(group), "bytes": sum(w.bytes for w in group), "duration_us": duration,
                  "ideal_us": sum(w.ideal_ns for w in group) / 1e3, "work_us": sum(w.work_ns for w in group) / 1e3,
                  "tail_us": sum(w.tail_ns for w in group) / 1e3, "sync_us": sum(w.sync_ns for w in group) / 1e3,
                  "achieved_gbps": sum(w.bytes for w in group) / duration / 1e3 if duration else 0.0}
        values["excess_us"] = values["duration_us"] - values["ideal_us"] - values["sync_us"]
        phases[name] = values
    total = previous / 1e3
    ideal = sum(w.ideal_ns for w in waves) / 1e3
    by_opcode: dict[str, dict[str, float]] = defaultdict(lambda: {"us": 0.0, "ideal_us": 0.0, "waves": 0})
    for r in rows:
        by_opcode[r["opcode"]]["us"] += r["us"]
        by_opcode[r["opcode"]]["ideal_us"] += r["ideal_us"]
        by_opcode[r["opcode"]]["waves"] += 1
    waits = sum(e.ready - e.start for e in evs if e.ready is not None and e.ready > e.start)
    return {
        "bandwidth_gbps": bandwidth_gbps,
        "position": position,
        "traced_kernel_us": total,
        "ideal_stream_us": ideal,
        "bubble_us": total - ideal,
        "components_us": {
            "barrier_sync": sum(w.sync_ns for w in waves) / 1e3,
            "streaming_excess": sum(phases[p]["excess_us"] for p in STREAMING if p in phases),
            "attention_excess": phases["attention"]["excess_us"] if "attention" in phases else 0.0,
            "small_phases": sum(v["excess_us"] for n, v in phases.items() if n not in STREAMING and n != "attention"),
        },
        # Mean time per worker between a task's start and the end of its exchange waits.
        "mean_barrier_wait_us": waits / workers / 1e3,
        "phases": phases,
        "waves": rows,
        "token_us": total,
        "excess_us": total - ideal,
        "by_opcode": dict(by_opcode),
    }


def layer_window(plan: dict, evs: list[Event], layer: int) -> tuple[float, float]:
    """Time span of one layer's tasks (timeline.py:357-361)."""
    tasks = plan["tasks"]
    selected = [e for e in evs if tasks[e.task].get("layer") == layer]
    return min(e.start for e in selected), max(e.end for e in selected)


def render_timeline_svg(plan: dict, evs: list[Event], *, title: str,
                        window: tuple[float, float] | None = None) -> str:
    """One row per worker; each task a bar colored by phase, its exchange wait (start to ready)
    drawn lighter (timeline.py:289-354)."""
    tasks = plan["tasks"]
    workers = plan["target"]["worker_count"]
    begin, end = window or (0.0, max(e.end for e in evs))
    span = max(end - begin, 1.0)
    left, top, row, width = 80, 80, 6, 1500
    plot = width - left - 20
    height = top + workers * row + 40

    def x(t: float) -> float:
        return left + (min(max(t, begin), end) - begin) / span * plot

    out = [f'<svg xmlns="http://www.w3.org/2000/svg" viewBox="0 0 {width} {height}" width="{width}" '
           f'height="{height}" role="img">', f"<title>{escape(title)}</title>",
           '<rect width="100%" height="100%" fill="#ffffff"/>',
           f'<text x="{left}" y="30" font-family="sans-serif" font-size="18" fill="#0f172a">{escape(title)}</text>']
    for i, name in enumerate((*PHASES, "wait")):
        lx = left + i * 120
        out.append(f'<rect x="{lx}" y="44" width="12" height="12" fill="{COLORS[name]}"/>'
                   f'<text x="{lx + 16}" y="55" font-family="sans-serif" font-size="11" fill="#334155">{name}</text>')
    for e in evs:
        if e.end < begin or e.start > end:
            continue
        y = top + e.worker * row
        if e.ready is not None and e.ready > e.start:
            out.append(f'<rect x="{x(e.start):.2f}" y="{y}" width="{max(x(e.ready) - x(e.start), 0.2):.2f}" '
                       f'height="{row - 1}" fill="{COLORS["wait"]}"/>')
        first = e.ready if e.ready is not None and e.ready > e.start else e.start
        out.append(f'<rect x="{x(first):.2f}" y="{y}" width="{max(x(e.end) - x(first), 0.2):.2f}" '
                   f'height="{row - 1}" fill="{COLORS[phase(tasks[e.task])]}"/>')
    step = 10.0 ** int(np.floor(np.log10(span)))
    while span / step < 4:
        step /= 2
    tick = (begin // step + 1) * step
    axis = top + workers * row + 16
    while tick < end:
        out.append(f'<line x1="{x(tick):.1f}" y1="{top}" x2="{x(tick):.1f}" y2="{axis - 10}" stroke="#cbd5e1" '
                   f'stroke-width="0.5"/><text x="{x(tick):.1f}" y="{axis}" text-anchor="middle" '
                   f'font-family="sans-serif" font-size="10" fill="#475569">{tick / 1e3:.1f} µs</text>')
        tick += step
    out.append("</svg>")
    return "\n".join(out) + "\n"


def per_layer(report: dict) -> dict[str, dict[str, float]]:
    """Median per-layer interval of each opcode that runs once per layer: duration and its
    sync / ideal / work / tail columns, in microseconds."""
    groups: dict[str, list[dict]] = defaultdict(list)
    for row in report["waves"]:
        groups[row["opcode"]].append(row)
    layers = max(len(rows) for rows in groups.values())
    out = {}
    for opcode, rows in groups.items():
        if len(rows) == layers and layers > 1:
            out[opcode] = {k: float(np.median([r[f"{k}_ns"] for r in rows])) / 1e3
                           for k in ("duration", "sync", "ideal", "work", "tail")}
    return out


def markdown(report: dict, measured_us: float, title: str) -> str:
    """The budget as tables: components, phases and per-layer medians."""
    c = report["components_us"]
    lines = [f"### {title}", "",
             f"Traced step {report['traced_kernel_us']:.1f} us (launch average {measured_us:.1f} us/token), "
             f"ideal stream {report['ideal_stream_us']:.1f} us at {report['bandwidth_gbps']:.0f} GB/s, "
             f"bubble {report['bubble_us']:.1f} us; mean exchange wait per worker "
             f"{report['mean_barrier_wait_us']:.1f} us.", "",
             "| component | us |", "|---|---:|", f"| ideal stream | {report['ideal_stream_us']:.1f} |"]
    lines += [f"| {name} | {value:.1f} |" for name, value in c.items()]
    lines += [f"| **traced step** | **{report['traced_kernel_us']:.1f}** |", "",
              "| phase | waves | MB | duration | ideal | sync | work | tail | GB/s |",
              "|---|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for name, p in report["phases"].items():
        lines.append(f"| {name} | {p['waves']} | {p['bytes'] / 1e6:.1f} | {p['duration_us']:.1f} | {p['ideal_us']:.1f} | "
                     f"{p['sync_us']:.1f} | {p['work_us']:.1f} | {p['tail_us']:.1f} | {p['achieved_gbps']:.0f} |")
    lines += ["", "Per layer (median over layers, us):", "",
              "| opcode | duration | sync | ideal | work | tail |", "|---|---:|---:|---:|---:|---:|"]
    for opcode, v in per_layer(report).items():
        lines.append(f"| {opcode} | {v['duration']:.2f} | {v['sync']:.2f} | {v['ideal']:.2f} | {v['work']:.2f} | "
                     f"{v['tail']:.2f} |")
    return "\n".join(lines) + "\n"


def main() -> int:
    """Loss budget of the synthetic Llama-3.2-1B bf16 worker at the given prompt lengths: a
    64-token generate launch after the prompt, its last step traced."""
    import argparse
    import json
    import statistics

    from . import runtime as R
    from . import synthetic as S
    from .tileplan import probe

    parser = argparse.ArgumentParser(description=main.__doc__)
    parser.add_argument("--context", type=int, action="append", help="prompt length (1 = the BOS prompt)")
    parser.add_argument("--chunk-steps", type=int, default=130, help="attention chunk steps of contexts above 1")
    parser.add_argument("--out", help="markdown file to write")
    parser.add_argument("--svg", help="SVG of layer 8's tasks at the first context")
    a = parser.parse_args()
    contexts = a.context or [1]
    target = probe.probe_library()
    gbps = R.measure_stream_read(2 << 30, 3)
    print(f"streaming read {gbps:.0f} GB/s", flush=True)
    work = S.scratch_dir()
    weights = None
    sections = []
    for n in contexts:
        path = work / f"ctx{n}"
        _, weights = S.llama_package(path, n + 64, "bfloat16", seed=0, chunk_steps=None if n == 1 else a.chunk_steps,
                                     target=target, weights=weights)
        plan = json.loads((path / "plan.json").read_text())
        prompt = [S.BOS] if n == 1 else S.prompt(n, seed=n)
        ctx = R.DecoderModel(R.load_plan(path, verify_weights=False)).create_context()
        times = []
        for _ in range(3):
            ctx.wait(ctx.enqueue_reset())
            ctx.wait(ctx.enqueue_prefill(prompt))
            times.append(ctx.wait(ctx.enqueue_generate(64)).compute_us / 64)
        ctx.set_timeline(True)
        ctx.wait(ctx.enqueue_reset())
        ctx.wait(ctx.enqueue_prefill(prompt))
        ctx.wait(ctx.enqueue_generate(64))
        stamps = ctx.timeline().reshape(-1, 4)
        report = budget(plan, stamps, len(prompt) + 63, gbps)
        measured = statistics.median(times)
        text = markdown(report, measured, f"ctx {n}: position {len(prompt) + 63}, last step of a 64-token launch")
        print(text, flush=True)
        sections.append(text)
        if a.svg and n == contexts[0]:
            evs = events(plan, stamps)
            with open(a.svg, "w") as f:
                f.write(render_timeline_svg(plan, evs, title=f"layer 8, ctx {n}", window=layer_window(plan, evs, 8)))
        del ctx
    if a.out:
        with open(a.out, "w") as f:
            f.write("\n".join(sections))
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
