"""Per-wave timeline and loss budget of one decoded token (the reference's
tileplan/src/tileplan/timeline.py:135-286 idea, for this worker's 100 MHz device clock).

Every instruction of the last step of a launch carries device-clock stamps at start and end
(``SequenceContext.timeline()``).  A wave's critical-path share is the time from the previous
wave's last end to its own last end; each share is set against the time its bytes would take
at the measured streaming bandwidth, giving the "ideal stream" and "excess" columns of the
reference's loss budget.
"""

from __future__ import annotations

from collections import defaultdict

import numpy as np

TICK_NS = 10.0  # s_memrealtime runs at 100 MHz


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


def wave_bytes(plan: dict, position: int) -> dict[int, int]:
    """Algorithmic HBM bytes each wave must stream at `position` (weights and visible K/V)."""
    model = plan["model"]
    elem = 2 if model["weight_dtype"] == "bfloat16" else 4
    d, f = model["hidden_size"], model["intermediate_size"]
    kvw = model["num_key_value_heads"] * model["head_dim"]
    vocab = model.get("vocab_size", 0)
    out: dict[int, int] = defaultdict(int)
    for task in plan["tasks"]:
        op = task["opcode"].rsplit("_", 1)[0]
        rows = task["operands"].get("rows", [0, 0])
        n = rows[1] - rows[0]
        if op == "qkv":
            out[task["wave"]] += n * d * elem
        elif op == "output_projection":
            out[task["wave"]] += n * d * elem
        elif op == "ffn":
            out[task["wave"]] += 3 * n * d * elem
        elif op == "logits":
            out[task["wave"]] += n * d * elem
        elif op == "attention_scores" and task["operands"]["chunk"] == 0:
            out[task["wave"]] += 2 * (position + 1) * (model["head_dim"]) * elem
    del vocab, f, kvw
    return out


def budget(plan: dict, stamps: np.ndarray, position: int, stream_gbps: float) -> dict:
    """Per-wave critical path and the token's loss budget by opcode."""
    imap = instruction_map(plan)
    if len(imap) != len(stamps):
        raise ValueError("timeline does not match the plan's instruction count")
    opcode_of_wave = {}
    for task in plan["tasks"]:
        opcode_of_wave[task["wave"]] = task["opcode"].rsplit("_", 1)[0]
    starts: dict[int, list[int]] = defaultdict(list)
    ends: dict[int, list[int]] = defaultdict(list)
    last: dict[int, tuple] = {}
    for (worker, wave, task), (start, read, ready, end) in zip(imap, stamps):
        if task < 0 or start == 0:
            continue
        starts[wave].append(int(start))
        ends[wave].append(int(end))
        if wave not in last or end > last[wave][3]:
            last[wave] = (int(start), int(read), int(ready), int(end))
    waves = sorted(ends)
    origin = min(min(starts[w]) for w in waves)
    bytes_ = wave_bytes(plan, position)
    rows = []
    previous = origin
    by_opcode: dict[str, dict[str, float]] = defaultdict(lambda: {"us": 0.0, "ideal_us": 0.0, "waves": 0})
    for w in waves:
        end = max(ends[w])
        share = (end - previous) * TICK_NS / 1e3
        ideal = bytes_.get(w, 0) / (stream_gbps * 1e9) * 1e6
        op = opcode_of_wave[w]
        s0, r0, q0, e0 = last[w]
        rows.append({"wave": w, "opcode": op, "us": share, "ideal_us": ideal,
                     "span_us": (end - min(starts[w])) * TICK_NS / 1e3,
                     # the wave's last-finishing task: start→first read, →inputs ready, →end
                     "last_task_us": [(r0 - s0) * TICK_NS / 1e3 if r0 else None,
                                      (q0 - s0) * TICK_NS / 1e3 if q0 else None, (e0 - s0) * TICK_NS / 1e3],
                     "last_start_after_previous_us": (s0 - previous) * TICK_NS / 1e3})
        by_opcode[op]["us"] += share
        by_opcode[op]["ideal_us"] += ideal
        by_opcode[op]["waves"] += 1
        previous = end
    total = (previous - origin) * TICK_NS / 1e3
    ideal = sum(r["ideal_us"] for r in rows)
    return {"token_us": total, "ideal_stream_us": ideal, "excess_us": total - ideal,
            "by_opcode": dict(by_opcode), "waves": rows}
