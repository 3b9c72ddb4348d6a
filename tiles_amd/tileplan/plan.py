"""Offline tile plan: package format v10 (plan.json + weights.bin) for the decode worker.

The package is the drop-in boundary between the planner and the runtime, so its
fields, task graph, wave schedule and weight layout follow the reference planner's
format exactly (tileplan/src/tileplan/plan_core.py, decoder_stack.py).  The code is
this project's own; each rule cites the reference lines whose behaviour it keeps.
"""

from __future__ import annotations

import heapq
import json
import math
from dataclasses import asdict, dataclass

import numpy as np

FORMAT = 10                                   # plan_core.py:26
GENERATOR = "tileplan-decoder-0.10"           # plan_core.py:27
ABI = "tileinfer-decoder-v10"                 # probe.py:7
MODEL_KIND_STACK = "llama_decoder_stack"      # decoder_stack.py:47
MODEL_KIND_BLOCK = "llama_decoder_block"
WEIGHT_DTYPES = {"float32": 4, "bfloat16": 2}
# Tensor IDs and the order of a layer's weights (plan_core.py:29-51, plan.hpp:76-98).
TENSOR_NAMES = ("x", "attn_norm", "Wq", "Wk", "Wv", "q", "k", "q_rot", "K", "V", "attention",
                "Wo", "r", "ffn_norm", "Wgate", "Wup", "product", "Wdown", "y")
TID = {name: index for index, name in enumerate(TENSOR_NAMES)}
WEIGHTS = ("attn_norm", "Wq", "Wk", "Wv", "Wo", "ffn_norm", "Wgate", "Wup", "Wdown")
SCRATCH = tuple(n for n in TENSOR_NAMES if n not in (*WEIGHTS, "x", "y", "K", "V"))
OPCODE_NAMES = ("qkv", "attention_scores", "attention_values", "output_projection", "ffn",
                "ffn_reduce", "embedding", "final_rms_norm", "logits")
OPCODES = {name + suffix for name in OPCODE_NAMES for suffix in ("_f32", "_bf16")}
FUSED_STEPS = 384                             # plan_core.py:102
CANDIDATE_BYTES = 8                           # plan_core.py:285


def require(condition: bool, message: str) -> None:
    if not condition:
        raise ValueError(message)


def json_bytes(value: dict) -> bytes:
    """Canonical JSON: sorted keys, indent 2, no NaN, trailing newline (plan_core.py:64-67)."""
    return (json.dumps(value, sort_keys=True, indent=2, allow_nan=False) + "\n").encode()


@dataclass(frozen=True)
class BlockSpec:
    """One decoder block's shape and numerics (decoder_reference.py:18-37)."""

    hidden_size: int = 32
    intermediate_size: int = 64
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    head_dim: int = 8
    max_context: int = 6
    rms_norm_eps: float = 1e-5
    rope_type: str = "llama3"
    rope_pairing: str = "split_half"
    rope_theta: float = 500000.0
    rope_factor: float = 32.0
    rope_low_freq_factor: float = 1.0
    rope_high_freq_factor: float = 4.0
    rope_original_max_position_embeddings: int = 8192
    kv_cache_layout: str = "[layers,max_context,kv_heads,head_dim]"
    dtype: str = "float32"
    atol: float = 2e-5
    rtol: float = 2e-5

    def __post_init__(self) -> None:
        require(self.hidden_size == self.num_attention_heads * self.head_dim
                and self.num_attention_heads % self.num_key_value_heads == 0
                and self.head_dim % 2 == 0
                and min(self.hidden_size, self.intermediate_size, self.num_attention_heads,
                        self.num_key_value_heads, self.head_dim, self.max_context) > 0
                and 0 < self.rope_low_freq_factor < self.rope_high_freq_factor,
                "unsupported decoder specification")

    @property
    def head_to_kv(self) -> list[int]:
        group = self.num_attention_heads // self.num_key_value_heads
        return [h // group for h in range(self.num_attention_heads)]

    def as_dict(self) -> dict:
        return {**asdict(self), "head_to_kv": self.head_to_kv}


@dataclass(frozen=True)
class StackSpec:
    block: BlockSpec = BlockSpec()
    layers: int = 3
    vocab_size: int = 48
    tie_word_embeddings: bool = True

    def as_dict(self) -> dict:
        return {**self.block.as_dict(), "layers": self.layers, "vocab_size": self.vocab_size,
                "tie_word_embeddings": self.tie_word_embeddings}


def llama32_1b(max_context: int) -> StackSpec:
    """The Llama-3.2-1B architecture (llama32_import.py:35-90); the context cap is lifted
    above the reference's 8192 so the 32K configuration fits (positions up to 32,831)."""
    require(type(max_context) is int and 1 <= max_context <= 131072, "invalid max_context")
    return StackSpec(BlockSpec(hidden_size=2048, intermediate_size=8192, num_attention_heads=32,
                               num_key_value_heads=8, head_dim=64, max_context=max_context),
                     layers=16, vocab_size=128256, tie_word_embeddings=True)


def weight_size(dtype: str) -> int:
    require(dtype in WEIGHT_DTYPES, "unsupported weight dtype")
    return WEIGHT_DTYPES[dtype]


def numeric_policy(dtype: str) -> dict:
    """plan_core.py:76-88."""
    weight_size(dtype)
    return {"numeric_policy": "hf-llama-eager-bf16-v1" if dtype == "bfloat16" else "decoder-f32-v1",
            "weight_dtype": dtype, "activation_dtype": dtype, "kv_dtype": dtype,
            "accumulation_dtype": "float32", "logits_compute_dtype": dtype,
            "api_output_dtype": "float32"}


def attention_chunking(spec: BlockSpec, dtype: str, target: dict, steps: int | None = None,
                       fused: int | None = None) -> dict:
    """Chunk count per K/V head, chunk length and fused length (plan_core.py:91-137)."""
    group = spec.num_attention_heads // spec.num_key_value_heads
    capacity = target["attention_shared_bytes"] // (group * weight_size(dtype))
    steps = capacity if steps is None else steps
    require(type(steps) is int and 0 < steps <= capacity,
            f"attention chunk steps must be in [1, {capacity}]")
    fused = min(FUSED_STEPS, steps) if fused is None else fused
    require(type(fused) is int and 0 < fused <= steps,
            "attention fused steps must be in [1, attention chunk steps]")
    longest = spec.max_context
    return {"attention_chunks": 1 if longest <= fused else max(2, -(-longest // steps)),
            "attention_chunk_steps": steps, "attention_fused_steps": fused}


def tensor_shape(spec: BlockSpec, name: str) -> tuple[int, ...]:
    """Package shapes; Wdown is stored transposed [f, d] (plan_core.py:160-177)."""
    d, f, dh = spec.hidden_size, spec.intermediate_size, spec.head_dim
    kv = spec.num_key_value_heads * dh
    shapes = {"attn_norm": (d,), "ffn_norm": (d,), "Wq": (d, d), "Wo": (d, d), "Wk": (kv, d),
              "Wv": (kv, d), "Wgate": (f, d), "Wup": (f, d), "Wdown": (f, d), "k": (kv,),
              "product": (f,), "K": (1, spec.max_context, spec.num_key_value_heads, dh),
              "V": (1, spec.max_context, spec.num_key_value_heads, dh)}
    return shapes.get(name, (d,))


def source_shape(spec: BlockSpec, name: str) -> tuple[int, ...]:
    """A weight as checkpoints hold it: Wdown is [d, f]."""
    if name == "Wdown":
        return (spec.hidden_size, spec.intermediate_size)
    return tensor_shape(spec, name)


def _storage_class(name: str) -> str:
    if name in WEIGHTS:
        return "weight"
    return {"K": "kv", "V": "kv", "x": "input", "y": "output"}.get(name, "scratch")


def _strides(shape: tuple[int, ...]) -> list[int]:
    out = [1] * len(shape)
    for i in range(len(shape) - 2, -1, -1):
        out[i] = out[i + 1] * shape[i + 1]
    return out


def descriptors(spec: BlockSpec, dtype: str) -> list[dict]:
    """plan_core.py:193-205."""
    return [{"id": TID[n], "name": n, "shape": list(tensor_shape(spec, n)),
             "strides": _strides(tensor_shape(spec, n)), "dtype": dtype,
             "storage": _storage_class(n)} for n in TENSOR_NAMES]


def regions(spec: BlockSpec, names: tuple[str, ...], alignment: int, element_bytes: int) -> tuple[list[dict], int]:
    """Aligned byte ranges of ``names`` in order (plan_core.py:208-227)."""
    cursor, entries = 0, []
    for name in names:
        cursor += (-cursor) % alignment
        size = element_bytes * int(np.prod(tensor_shape(spec, name)))
        entries.append({"tensor": TID[name], "offset": cursor, "bytes": size, "alignment": alignment})
        cursor += size
    return entries, cursor


def align(value: int, alignment: int = 64) -> int:
    return value + (-value) % alignment


def split(rows: int, parts: int) -> list[tuple[int, int]]:
    """At most ``parts`` contiguous near-equal nonempty ranges (plan_core.py:275-278)."""
    count = min(rows, parts)
    return [(i * rows // count, (i + 1) * rows // count) for i in range(count)]


def ffn_chunks(spec: BlockSpec, workers: int) -> int:
    return len(split(spec.intermediate_size, workers))


def selection_slots(vocab_size: int, workers: int) -> int:
    return len(split(vocab_size, workers))


def _layer_graph(spec: BlockSpec, workers: int, chunking: dict, dtype: str) -> list[dict]:
    """One layer's tasks and minimal predecessors (plan_core.py:297-428)."""
    d, f, dh = spec.hidden_size, spec.intermediate_size, spec.head_dim
    nq, nkv = spec.num_attention_heads, spec.num_key_value_heads
    group = nq // nkv
    suffix = "_bf16" if dtype == "bfloat16" else "_f32"
    tasks: list[dict] = []

    def add(opcode, operands, output, predecessors, work) -> int:
        tasks.append({"id": len(tasks), "opcode": opcode + suffix, "operands": operands,
                      "output": output, "predecessors": sorted(set(predecessors)),
                      "estimated_work": work})
        return len(tasks) - 1

    def rows(tensor, begin, end):
        return {"tensor": TID[tensor], "rows": [begin, end]}

    kv_width = nkv * dh
    projection = []
    for begin, end in split(d + 2 * kv_width, workers):
        output = []
        if begin < d:
            output.append(rows("q", begin, min(end, d)))
        if begin < d + kv_width and end > d:
            output.append(rows("k", max(begin, d) - d, min(end, d + kv_width) - d))
        if end > d + kv_width:
            first = max(begin, d + kv_width) - d - kv_width
            output.append({"tensor": TID["V"], "position": "current", "rows": [first, end - d - kv_width]})
        projection.append((begin, end, add("qkv", {"rows": [begin, end]}, output, [], (end - begin) * d)))

    def producers(begin, end):
        return [t for first, last, t in projection if first < end and begin < last]

    chunks = chunking["attention_chunks"]
    steps = min(chunking["attention_chunk_steps"], spec.max_context)
    chunk_work = 2 * steps * dh * group
    values = []
    for kv_head in range(nkv):
        queries = [kv_head * group, (kv_head + 1) * group]
        inputs = producers(queries[0] * dh, queries[1] * dh)
        inputs += producers(d + kv_head * dh, d + (kv_head + 1) * dh)
        inputs += producers(d + kv_width + kv_head * dh, d + kv_width + (kv_head + 1) * dh)
        rotated = [rows("q_rot", queries[0] * dh, queries[1] * dh),
                   {"tensor": TID["K"], "position": "current", "head": kv_head}]
        group_scores = [add("attention_scores", {"kv_head": kv_head, "chunk": c},
                            [{"workspace": "scores", "chunk": c, "heads": queries}] + (rotated if c == 0 else []),
                            inputs, chunk_work) for c in range(chunks)]
        values += [add("attention_values", {"kv_head": kv_head, "chunk": c},
                       [{"workspace": "partials", "chunk": c, "heads": queries}], group_scores, chunk_work)
                   for c in range(chunks)]
    # MI355X re-partition (this planner's rule, not plan_core's): when attention runs on at most
    # half the workers, the output projection's rows are split over the others only, and
    # schedule() keeps them off the attention workers.  Those finish attention last, and rows of
    # theirs would be the projection wave's last to start.
    attention_tasks = nkv * chunks
    projection_workers = workers - attention_tasks if 2 * attention_tasks <= workers else workers
    attention = [add("output_projection", {"rows": [b, e]},
                     [rows("r", b, e)] + ([rows("attention", 0, d)] if b == 0 else []), values, (e - b) * d)
                 for b, e in split(d, projection_workers)]
    product = [add("ffn", {"rows": [b, e], "chunk": c},
                   [rows("product", b, e), {"workspace": "ffn_partials", "chunk": c}], attention, 3 * (e - b) * d)
               for c, (b, e) in enumerate(split(f, workers))]
    for b, e in split(d, workers):
        add("ffn_reduce", {"rows": [b, e]}, [rows("y", b, e)], product, (e - b) * len(product))
    return tasks


def program(spec: BlockSpec, dtype: str, workers: int, chunking: dict, layers: int,
            vocab_size: int | None) -> list[dict]:
    """Whole-token task graph in topological order (plan_core.py:431-521)."""
    suffix = "_bf16" if dtype == "bfloat16" else "_f32"
    d = spec.hidden_size
    tasks: list[dict] = []

    def stage(opcode, name, rows, predecessors, work, selection=False):
        ids = []
        for slot, (b, e) in enumerate(split(rows, workers)):
            operands: dict = {"rows": [b, e]}
            output: list[dict] = [{"stage": name, "rows": [b, e]}]
            if selection:
                operands["chunk"] = slot
                output.append({"workspace": "selection", "chunk": slot})
            ids.append(len(tasks))
            tasks.append({"id": len(tasks), "layer": None, "opcode": opcode + suffix, "operands": operands,
                          "output": output, "predecessors": sorted(predecessors),
                          "estimated_work": work(b, e)})
        return ids

    previous = stage("embedding", "embedding", d, [], lambda b, e: e - b) if vocab_size is not None else []
    template = _layer_graph(spec, workers, chunking, dtype)
    for layer in range(layers):
        offset = len(tasks)
        for task in template:
            repeated = json.loads(json.dumps(task))
            repeated["id"] += offset
            repeated["layer"] = layer
            repeated["predecessors"] = sorted([i + offset for i in task["predecessors"]]
                                              if task["predecessors"] else previous)
            tasks.append(repeated)
        previous = [t["id"] for t in tasks[offset:] if t["opcode"].startswith("ffn_reduce")]
    if vocab_size is not None:
        normalized = stage("final_rms_norm", "final_norm", d, previous, lambda b, e: d + e - b)
        stage("logits", "logits", vocab_size, normalized, lambda b, e: (e - b) * d, selection=True)
    return tasks


def schedule(tasks: list[dict], workers: int) -> list[dict]:
    """Earliest wave per task; within a wave, tasks in (-work, id) order go to the least
    loaded worker, lowest index on ties (plan_core.py:524-549).  An output projection wave
    that has no more tasks than the workers the preceding attention wave left idle goes to
    those workers alone (_layer_graph sizes it so)."""
    buckets: list[list[int]] = []
    for task in tasks:
        wave = 0 if not task["predecessors"] else 1 + max(tasks[p]["wave"] for p in task["predecessors"])
        task["wave"] = wave
        while len(buckets) <= wave:
            buckets.append([])
        buckets[wave].append(task["id"])
    result = []
    for wave, ids in enumerate(buckets):
        lanes: list[list[int]] = [[] for _ in range(workers)]
        loads = [0] * workers
        busy: set[int] = set()
        if wave > 0 and tasks[ids[0]]["opcode"].startswith("output_projection"):
            busy = {w for w, lane in enumerate(result[-1]["workers"]) if lane
                    and tasks[lane[0]]["opcode"].startswith("attention")}
            if len(ids) > workers - len(busy):
                busy = set()
        heap = [(0, w) for w in range(workers) if w not in busy]
        for task_id in sorted(ids, key=lambda i: (-tasks[i]["estimated_work"], i)):
            load, worker = heapq.heappop(heap)
            tasks[task_id]["worker"] = worker
            lanes[worker].append(task_id)
            loads[worker] = load + tasks[task_id]["estimated_work"]
            heapq.heappush(heap, (loads[worker], worker))
        result.append({"id": wave, "workers": lanes, "estimated_work": loads})
    return result


def mark_conditional_barriers(tasks: list[dict], waves: list[dict], fused: int) -> None:
    """A scores-only wave followed by a values-only wave ends with a barrier that is skipped
    while the visible prefix has at most ``fused`` steps (plan_core.py:552-568)."""
    def only(wave, opcode):
        ids = [t for lane in wave["workers"] for t in lane]
        return bool(ids) and all(tasks[i]["opcode"].startswith(opcode) for i in ids)

    for wave, following in zip(waves, waves[1:]):
        if only(wave, "attention_scores") and only(following, "attention_values"):
            wave["conditional_barrier"] = {"skip_up_to_length": fused}


def scheduled_program(spec, dtype, workers, chunking, layers=1, vocab_size=None):
    tasks = program(spec, dtype, workers, chunking, layers, vocab_size)
    waves = schedule(tasks, workers)
    mark_conditional_barriers(tasks, waves, chunking["attention_fused_steps"])
    return tasks, waves


def plan_target(probe: dict) -> dict:
    """The plan's record of a probed target (plan_core.py:611-621)."""
    return {"compute_capability": probe["device"]["compute_capability"],
            "sm_count": probe["device"]["sm_count"], "cooperative_launch": True,
            "worker_count": probe["launch"]["worker_count"],
            "threads_per_block": probe["launch"]["threads_per_block"],
            "kernel_fingerprint": probe["executor"]["fingerprint"],
            "attention_shared_bytes": probe["executor"]["attention_shared_bytes"]}


def model_section(fields: dict, block: BlockSpec, dtype: str, chunking: dict, workers: int) -> dict:
    return {**{k: v for k, v in fields.items() if k != "dtype"}, **numeric_policy(dtype), **chunking,
            "ffn_chunks": ffn_chunks(block, workers), "tensors": descriptors(block, dtype)}


def storage_section(block: BlockSpec, dtype: str, chunks: int, workers: int, layers: int,
                    input_bytes: int, output_bytes: int, weight_bytes: int | None = None) -> dict:
    """plan_core.py:657-699."""
    size = weight_size(dtype)
    weights, layer_weight_bytes = regions(block, WEIGHTS, 64, size)
    scratch, scratch_bytes = regions(block, SCRATCH, 16, size)
    kv, layer_kv_bytes = regions(block, ("K", "V"), 16, size)
    return {"input_bytes": input_bytes, "output_bytes": output_bytes, "scratch_bytes": scratch_bytes,
            "attention_bytes": block.num_attention_heads * block.max_context * size,
            "attention_partial_bytes": chunks * block.num_attention_heads * (block.head_dim + 2) * 4,
            "ffn_partial_bytes": ffn_chunks(block, workers) * block.hidden_size * 4,
            "scratch": scratch, "kv_bytes": layer_kv_bytes * layers, "kv": kv,
            "weight_bytes": layer_weight_bytes if weight_bytes is None else weight_bytes,
            "weights": weights}


def stack_layout(spec: StackSpec, dtype: str) -> tuple[dict, int]:
    """Offsets of the stack's regions in weights.bin (decoder_stack.py:223-248)."""
    block, size = spec.block, weight_size(dtype)
    embedding_bytes = spec.vocab_size * block.hidden_size * size
    _, layer_weight_bytes = regions(block, WEIGHTS, 64, size)
    _, layer_kv_bytes = regions(block, ("K", "V"), 16, size)
    layer_stride = align(layer_weight_bytes)
    layer_offset = align(embedding_bytes)
    norm_offset = align(layer_offset + spec.layers * layer_stride)
    total = norm_offset + block.hidden_size * size
    lm_offset = 0
    if not spec.tie_word_embeddings:
        lm_offset = align(total)
        total = lm_offset + embedding_bytes
    return {"embedding_offset": 0, "embedding_bytes": embedding_bytes,
            "layer_weights_offset": layer_offset, "layer_weight_stride": layer_stride,
            "layer_weight_bytes": layer_weight_bytes, "final_norm_offset": norm_offset,
            "final_norm_bytes": block.hidden_size * size, "lm_head_offset": lm_offset,
            "lm_head_alias": spec.tie_word_embeddings, "layer_kv_stride": layer_kv_bytes}, total


def assemble(kind: str, target: dict, model: dict, storage: dict, prog, weights_sha256: str) -> dict:
    tasks, waves = prog
    return {"header": {"format_version": FORMAT, "executor_abi": ABI, "generator": GENERATOR,
                       "model_kind": kind},
            "target": target, "model": model, "storage": storage, "tasks": tasks, "waves": waves,
            "integrity": {"weights_bytes": storage["weight_bytes"], "weights_sha256": weights_sha256}}


def stack_plan(spec: StackSpec, target: dict, dtype: str, weights_sha256: str,
               chunk_steps: int | None = None, fused_steps: int | None = None) -> dict:
    """Everything in a stack package but the weight bytes (decoder_stack.py:251-293)."""
    require(len(weights_sha256) == 64, "invalid weight hash")
    block, workers = spec.block, target["worker_count"]
    stack, total = stack_layout(spec, dtype)
    chunking = attention_chunking(block, dtype, target, chunk_steps, fused_steps)
    storage = storage_section(block, dtype, chunking["attention_chunks"], workers, spec.layers, 4,
                              spec.vocab_size * 4, total)
    return assemble(MODEL_KIND_STACK, target, model_section(spec.as_dict(), block, dtype, chunking, workers),
                    {**storage, "stack": stack,
                     "selection_bytes": CANDIDATE_BYTES * selection_slots(spec.vocab_size, workers)},
                    scheduled_program(block, dtype, workers, chunking, spec.layers, spec.vocab_size),
                    weights_sha256)


def block_plan(block: BlockSpec, target: dict, dtype: str, weights_sha256: str,
               chunk_steps: int | None = None, fused_steps: int | None = None) -> dict:
    """A single-layer block package (decoder_block.py:50-70)."""
    workers = target["worker_count"]
    chunking = attention_chunking(block, dtype, target, chunk_steps, fused_steps)
    size = weight_size(dtype)
    storage = storage_section(block, dtype, chunking["attention_chunks"], workers, 1,
                              block.hidden_size * size, block.hidden_size * size)
    return assemble(MODEL_KIND_BLOCK, target, model_section({**block.as_dict(), "layers": 1}, block, dtype, chunking, workers),
                    storage, scheduled_program(block, dtype, workers, chunking), weights_sha256)
