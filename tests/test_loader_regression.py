"""Structural package validation without a GPU, after the reference's loader regression
(tileinfer/tests/loader_regression.py:15-191,196-410): block (decoder_m1) and stack (decoder_m4)
packages in both dtypes, planned with two-step attention chunks (fused and split attention, a
conditional barrier), are loaded by the C++ loader against the fixture target after legal
rearrangements, which it must accept, and after mutations, which it must reject.

This worker synchronizes on data, not barriers, so its loader is stricter than the reference's in
one place: every wave holds one opcode of one layer, in program order (plan.cpp validate_program),
and with several attention chunks per K/V head a worker runs its chunks in ascending head order.
The accepted rearrangements below are the ones the reference accepts that keep to that rule
(another worker assignment, reversed lanes and task order, Q/K/V rows across the Q/K boundary,
renumbered FFN partial slots, permuted candidate slots, execution-only plans); the rejected cases
include the reference's dataflow mutations, which this loader refuses by the same rule.
"""

import copy
import json
import re
from pathlib import Path

import numpy as np
import pytest
import torch

from tiles_amd import runtime as R
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

GOLDEN = Path(__file__).parent / "golden"
TARGET = probe.mi355x_target()


def fixture(name: str):
    model = json.loads((GOLDEN / name / "model.json").read_text())
    block = P.BlockSpec(**{k: model[k] for k in P.BlockSpec.__dataclass_fields__ if k in model})
    with np.load(GOLDEN / name / "weights.npz", allow_pickle=False) as data:
        weights = {k: torch.from_numpy(data[k].copy()) for k in data.files}
    return model, block, weights


@pytest.fixture(scope="module")
def packages(tmp_path_factory):
    root = tmp_path_factory.mktemp("regression")
    out = {}
    for dtype in ("float32", "bfloat16"):
        _, block, weights = fixture("decoder_m1")
        K.build_block_package(block, weights, TARGET, root / f"block-{dtype}", dtype, 2, 2)
        out[("block", dtype)] = root / f"block-{dtype}"
        model, block, weights = fixture("decoder_m4")
        spec = P.StackSpec(block, model["layers"], model["vocab_size"], model["tie_word_embeddings"])
        K.build_stack_package(spec, weights, TARGET, root / f"stack-{dtype}", dtype, 2, 2)
        out[("stack", dtype)] = root / f"stack-{dtype}"
    return out


def load(package: Path, plan: dict, tmp_path: Path):
    """Loads `plan` (written as plain, non-canonical JSON) beside the package's weights."""
    dst = tmp_path / "mutated"
    dst.mkdir(exist_ok=True)
    (dst / "plan.json").write_text(json.dumps(plan))
    weights = dst / "weights.bin"
    if not weights.exists():
        weights.symlink_to(package / "weights.bin")
    return R.Plan(dst, True, R.target_from_probe(TARGET))


# ---------------------------------------------------------------- legal rearrangements

def rotate_workers(plan: dict) -> None:
    """Every task one worker on, lanes reversed within each wave, the task list reversed."""
    workers = plan["target"]["worker_count"]
    for task in plan["tasks"]:
        task["worker"] = (task["worker"] + 1) % workers
    for wave in plan["waves"]:
        wave["workers"] = wave["workers"][-1:] + wave["workers"][:-1]
        wave["estimated_work"] = wave["estimated_work"][-1:] + wave["estimated_work"][:-1]
        for lane in wave["workers"]:
            lane.reverse()
    plan["tasks"].reverse()


def execution_only(plan: dict) -> None:
    """Without the planner's metadata: no predecessors and no work estimates."""
    for task in plan["tasks"]:
        del task["predecessors"], task["estimated_work"]
    for wave in plan["waves"]:
        del wave["estimated_work"]


def layer0(plan: dict, opcode: str) -> list[dict]:
    return [t for t in plan["tasks"] if t["layer"] in (None, 0) and t["opcode"].rsplit("_", 1)[0] == opcode]


def remove_task(plan: dict, task: dict, merged_into: dict) -> None:
    """Deletes `task` and renumbers the later task IDs (IDs stay 0 .. n-1)."""
    gone = task["id"]
    plan["waves"][task["wave"]]["workers"][task["worker"]].remove(gone)
    plan["tasks"] = [t for t in plan["tasks"] if t["id"] != gone]
    renumber = lambda i: merged_into["id"] if i == gone else (i - 1 if i > gone else i)  # noqa: E731
    for t in plan["tasks"]:
        if "predecessors" in t:
            t["predecessors"] = sorted({renumber(i) for i in t["predecessors"]})
    for t in plan["tasks"]:
        t["id"] = renumber(t["id"])
    for wave in plan["waves"]:
        wave["workers"] = [[renumber(i) for i in lane] for lane in wave["workers"]]


def cross_qk_boundary(plan: dict) -> None:
    """The Q/K boundary inside one Q/K/V task: the last Q task and the first K task of layer 0
    become one task over both row ranges (at 256 workers the fixtures' tasks hold one row each,
    so the boundary cannot move inside a task without merging two); ownership stays complete."""
    d = plan["model"]["hidden_size"]
    tasks = sorted(layer0(plan, "qkv"), key=lambda t: t["operands"]["rows"][0])
    last_q = next(t for t in tasks if t["operands"]["rows"][1] == d)
    first_k = next(t for t in tasks if t["operands"]["rows"][0] == d)
    end = first_k["operands"]["rows"][1]
    last_q["operands"]["rows"][1] = end
    last_q["output"].append({"tensor": first_k["output"][0]["tensor"], "rows": [0, end - d]})
    if "estimated_work" in last_q:
        last_q["estimated_work"] += first_k["estimated_work"]
    remove_task(plan, first_k, last_q)


def ffn_chunk_slot(task: dict, chunk: int) -> None:
    task["operands"]["chunk"] = chunk
    task["output"][1]["chunk"] = chunk


def renumber_ffn_chunks(plan: dict) -> None:
    """Two FFN chunks swap partial slots: another summation order, still complete."""
    first, second = layer0(plan, "ffn")[:2]
    ffn_chunk_slot(first, 1)
    ffn_chunk_slot(second, 0)


def candidate_slot(task: dict, slot: int) -> None:
    task["operands"]["chunk"] = slot
    task["output"][-1]["chunk"] = slot


def swap_candidate_slots(plan: dict) -> None:
    first, second = [t for t in plan["tasks"] if t["opcode"].startswith("logits")][:2]
    slot = first["operands"]["chunk"]
    candidate_slot(first, second["operands"]["chunk"])
    candidate_slot(second, slot)


def move_task(plan: dict, task: dict, worker: int, wave: int | None = None, first: bool = False) -> None:
    lanes = plan["waves"][task["wave"]]["workers"]
    lanes[task["worker"]].remove(task["id"])
    task["worker"] = worker
    if wave is not None:
        task["wave"] = wave
    lane = plan["waves"][task["wave"]]["workers"][worker]
    lane.insert(0, task["id"]) if first else lane.append(task["id"])


def split_chunks(plan: dict) -> tuple[dict, dict]:
    """Layer 0's (head 1, chunk 0) scores task and the worker of its (head 0, chunk 1) task."""
    scores = layer0(plan, "attention_scores")
    h1c0 = next(t for t in scores if t["operands"] == {"kv_head": 1, "chunk": 0})
    h0c1 = next(t for t in scores if t["operands"] == {"kv_head": 0, "chunk": 1})
    return h1c0, h0c1


def chunks_in_head_order(plan: dict) -> None:
    """A worker runs two split chunks of different heads, lower head first."""
    h1c0, h0c1 = split_chunks(plan)
    move_task(plan, h1c0, h0c1["worker"])


ACCEPTED = {
    "canonical": lambda p: None,
    "planner metadata is not needed for execution": execution_only,
    "alternative assignment and ordering": rotate_workers,
    "Q/K/V rows across the Q/K boundary": cross_qk_boundary,
    "FFN partial slots out of row order": renumber_ffn_chunks,
    "two chunks of different heads on one worker, lower head first": chunks_in_head_order,
}
STACK_ACCEPTED = {"candidate slots out of row order": swap_candidate_slots}


@pytest.mark.parametrize("kind", ["block", "stack"])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_loader_accepts_legal_rearrangements(packages, tmp_path, kind, dtype):
    path = packages[(kind, dtype)]
    original = K.read_plan(path)
    cases = {**ACCEPTED, **(STACK_ACCEPTED if kind == "stack" else {})}
    for label, rearrange in cases.items():
        plan = copy.deepcopy(original)
        rearrange(plan)
        (tmp_path / label.replace(" ", "_").replace("/", "_")).mkdir()
        load(path, plan, tmp_path / label.replace(" ", "_").replace("/", "_"))


# ---------------------------------------------------------------- mutations

def delay_producer(plan: dict) -> None:
    """The first task one wave later, where its consumers already run."""
    task = plan["tasks"][0]
    move_task(plan, task, task["worker"], task["wave"] + 1)


def stale_scratch_read(plan: dict) -> None:
    """A layer-0 attention task in layer 1's attention wave, after layer 1 overwrote Q."""
    early = next(t for t in plan["tasks"] if t["layer"] == 0 and t["opcode"].startswith("attention_scores"))
    late = next(t for t in plan["tasks"] if t["layer"] == 1 and t["opcode"].startswith("attention_scores"))
    move_task(plan, early, early["worker"], late["wave"])


def drop_k_output(plan: dict) -> None:
    task = next(t for t in layer0(plan, "qkv") if t["operands"]["rows"][0] >= plan["model"]["hidden_size"])
    task["output"] = []


def rotate_in_later_chunk(plan: dict) -> None:
    scores = [t for t in plan["tasks"] if t["opcode"].startswith("attention_scores")]
    first = next(t for t in scores if t["operands"]["chunk"] == 0)
    later = next(t for t in scores if t["layer"] == first["layer"]
                 and t["operands"] == {"kv_head": first["operands"]["kv_head"], "chunk": 1})
    later["output"] += first["output"][1:]
    del first["output"][1:]


def duplicate_partial(plan: dict) -> None:
    ffn_chunk_slot(layer0(plan, "ffn")[1], 0)


def extra_chunk(plan: dict) -> None:
    plan["model"]["ffn_chunks"] += 1
    plan["storage"]["ffn_partial_bytes"] += plan["model"]["hidden_size"] * 4


def drop_last_reduce(plan: dict) -> None:
    """Layer 0's last FFN reduction task is gone: the last rows of y have no writer."""
    tasks = sorted(layer0(plan, "ffn_reduce"), key=lambda t: t["operands"]["rows"][0])
    remove_task(plan, tasks[-1], tasks[0])


def reduce_in_ffn_wave(plan: dict) -> None:
    for task in layer0(plan, "ffn_reduce"):
        move_task(plan, task, task["worker"], task["wave"] - 1)


def conditional_wave(plan: dict) -> dict:
    return next(wave for wave in plan["waves"] if "conditional_barrier" in wave)


def move_condition(plan: dict) -> None:
    wave = conditional_wave(plan)
    plan["waves"][wave["id"] - 1]["conditional_barrier"] = wave.pop("conditional_barrier")


def fuse_into_projection(plan: dict) -> None:
    """Layer 0's values tasks in the output projection's wave."""
    wave = conditional_wave(plan)
    values, projection = plan["waves"][wave["id"] + 1], plan["waves"][wave["id"] + 2]
    for worker, lane in enumerate(values["workers"]):
        for task_id in lane:
            plan["tasks"][task_id]["wave"] += 1
        projection["workers"][worker] = lane + projection["workers"][worker]
        values["workers"][worker] = []
    projection["conditional_barrier"] = wave.pop("conditional_barrier")


def swap_wave_contents(plan: dict) -> None:
    """Layer 0's Q/K/V wave and output projection wave trade places."""
    qkv = layer0(plan, "qkv")[0]["wave"]
    projection = layer0(plan, "output_projection")[0]["wave"]
    for task in plan["tasks"]:
        if task["wave"] in (qkv, projection):
            task["wave"] = projection if task["wave"] == qkv else qkv
    waves = plan["waves"]
    waves[qkv]["workers"], waves[projection]["workers"] = waves[projection]["workers"], waves[qkv]["workers"]


def empty_wave(plan: dict) -> None:
    workers = plan["target"]["worker_count"]
    plan["waves"].append({"id": len(plan["waves"]), "workers": [[] for _ in range(workers)],
                          "estimated_work": [0] * workers})


def chunks_out_of_head_order(plan: dict) -> None:
    """A worker runs (head 1, chunk 0) before (head 0, chunk 1): with the chunks of a head waiting
    for each other's statistics, two such workers could wait on each other."""
    h1c0, h0c1 = split_chunks(plan)
    move_task(plan, h1c0, h0c1["worker"], first=True)


def share_candidate_slot(plan: dict) -> None:
    first, second = [t for t in plan["tasks"] if t["opcode"].startswith("logits")][:2]
    candidate_slot(second, first["operands"]["chunk"])


def swapped_precision(opcode: str) -> str:
    return opcode.replace("_bf16", "_x").replace("_f32", "_bf16").replace("_x", "_f32")


# (label, mutation, message) — a message of None accepts any rejection.
MUTATIONS = [
    ("read before producer", delay_producer, "a wave mixes opcodes or layers"),
    ("mixed activation dtype", lambda p: p["model"].update(
        activation_dtype="float32" if p["model"]["weight_dtype"] == "bfloat16" else "bfloat16"),
     "inconsistent numeric policy"),
    ("cache dtype", lambda p: p["model"].update(
        kv_dtype="float32" if p["model"]["weight_dtype"] == "bfloat16" else "bfloat16"), "inconsistent numeric policy"),
    ("attention workspace", lambda p: p["storage"].update(attention_bytes=3), "invalid attention or FFN workspace"),
    ("opcode precision", lambda p: p["tasks"][0].update(opcode=swapped_precision(p["tasks"][0]["opcode"])),
     "opcode precision differs"),
    ("derived frequency overflow", lambda p: p["model"].update(rope_factor=1e-45), "invalid derived rotary frequency"),
    ("noninteger wave", lambda p: p["waves"][0].update(id=0.0), "program index must be an integer"),
    ("operand", lambda p: p["tasks"][0]["operands"].update(scale=15), "invalid task operands"),
    ("noninteger operand", lambda p: p["tasks"][0]["operands"].update(scale=1.0), "invalid task operands"),
    ("extra operand", lambda p: p["tasks"][0]["operands"].update(extra=0), "invalid task operands"),
    ("ID", lambda p: p["tasks"][1].update(id=0), "duplicate task ID"),
    ("wave", lambda p: p["tasks"][-1].update(wave=0), None),  # a wave/opcode rule fires first
    ("overlap", lambda p: p["tasks"].append(copy.deepcopy(p["tasks"][1])), "duplicate task ID"),
    ("context overflow", lambda p: p["model"].update(max_context=2**31 - 1), "context too long"),
    ("width overflow", lambda p: p["model"].update(intermediate_size=2**31 - 1), "odd intermediate size"),
    ("layers overflow", lambda p: p["model"].update(layers=2**31 - 1), None),
    ("byte offset overflow", lambda p: p["storage"]["weights"][1].update(offset=2**32 + 64), "invalid decoder tensor storage"),
    ("unsigned dimension", lambda p: p["model"].update(hidden_size=2**64 - 1), "invalid hidden_size"),
    ("epsilon underflow", lambda p: p["model"].update(rms_norm_eps=1e-300), "invalid rms_norm_eps"),
    ("worker index", lambda p: p["waves"][0]["workers"][0].append(2**64 - 1), "program index outside range"),
    ("missing task", lambda p: p["waves"][0]["workers"].__setitem__(0, []), "task is absent from the schedule"),
    ("missing conditional barrier", lambda p: conditional_wave(p).pop("conditional_barrier"),
     "invalid conditional barrier"),
    ("conditional barrier threshold", lambda p: conditional_wave(p)["conditional_barrier"].update(skip_up_to_length=3),
     "invalid conditional barrier"),
    ("conditional barrier before attention", move_condition, "invalid conditional barrier"),
    ("conditional barrier before a projection", fuse_into_projection, "a wave mixes opcodes or layers"),
    ("chunk steps beyond shared memory", lambda p: p["model"].update(attention_chunk_steps=1 << 20),
     "attention chunk exceeds the compiled worker's LDS"),
    ("fused beyond chunk steps", lambda p: p["model"].update(attention_fused_steps=3), "invalid attention chunking"),
    ("too few chunks", lambda p: p["model"].update(attention_chunks=1), "invalid attention chunking"),
    ("unaligned head", lambda p: p["model"].update(head_dim=6), "unsupported decoder dimensions"),
    ("undeclared K rows", drop_k_output, "invalid task operands or output ownership"),
    ("FFN chunk outside range", lambda p: layer0(p, "ffn")[0]["operands"].update(chunk=p["model"]["ffn_chunks"]),
     "program index outside range"),
    ("FFN partial slot shared", duplicate_partial, "missing or overlapping output rows"),
    ("FFN reduction before its partials", reduce_in_ffn_wave, "a wave mixes opcodes or layers"),
    ("FFN workspace", lambda p: p["storage"].update(ffn_partial_bytes=p["storage"]["ffn_partial_bytes"] + 4),
     "invalid attention or FFN workspace"),
    ("FFN chunks without tasks", extra_chunk, "invalid FFN chunking"),
    ("last output rows without a task", drop_last_reduce, "incomplete output ownership"),
    ("rotation in a later chunk", rotate_in_later_chunk, "invalid task operands or output ownership"),
    ("waves out of program order", swap_wave_contents, "waves out of program order"),
    ("empty wave", empty_wave, "empty wave"),
    ("split chunks out of K/V head order", chunks_out_of_head_order, "attention chunks of a worker out of K/V head order"),
]
STACK_MUTATIONS = [
    ("candidate slot outside range",
     lambda p: [t for t in p["tasks"] if t["opcode"].startswith("logits")][0]["operands"].update(
         chunk=len([t for t in p["tasks"] if t["opcode"].startswith("logits")])), "program index outside range"),
    ("candidate slot shared", share_candidate_slot, "missing or overlapping output rows"),
    ("selection workspace size", lambda p: p["storage"].update(selection_bytes=p["storage"]["selection_bytes"] + 8),
     "invalid greedy selection workspace"),
    ("unaligned selection workspace", lambda p: p["storage"].update(selection_bytes=p["storage"]["selection_bytes"] + 4),
     "invalid greedy selection workspace"),
    ("missing selection workspace", lambda p: p["storage"].pop("selection_bytes"), "missing field selection_bytes"),
    ("undeclared candidate", lambda p: [t for t in p["tasks"] if t["opcode"].startswith("logits")][0]["output"].pop(),
     "invalid task operands or output ownership"),
    ("layer outside range", lambda p: next(t for t in p["tasks"] if t["layer"] is not None).update(
        layer=p["model"]["layers"]), "program index outside range"),
    ("stage tagged as a layer", lambda p: p["tasks"][0].update(layer=0), "stack stage tagged with a layer"),
    ("scratch reused by a later layer", stale_scratch_read, "a wave mixes opcodes or layers"),
]
BLOCK_MUTATIONS = [
    ("block task without a layer", lambda p: p["tasks"][0].update(layer=None), "program index must be an integer"),
    ("selection workspace in a block", lambda p: p["storage"].update(selection_bytes=8), "invalid decoder block storage"),
]
VERSIONS = [(v, True) for v in (2, 3)] + [(v, False) for v in (6, 7, 8, 9)]


def cases(kind: str):
    return MUTATIONS + (STACK_MUTATIONS if kind == "stack" else BLOCK_MUTATIONS)


@pytest.mark.parametrize("kind", ["block", "stack"])
@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_loader_rejects_mutations(packages, tmp_path, kind, dtype):
    path = packages[(kind, dtype)]
    original = K.read_plan(path)
    for label, mutate, message in cases(kind):
        plan = copy.deepcopy(original)
        mutate(plan)
        where = tmp_path / re.sub(r"[^a-zA-Z0-9]+", "_", label)
        where.mkdir()
        with pytest.raises(RuntimeError, match=re.escape(message) if message else None) as raised:
            load(path, plan, where)
        assert str(raised.value), label
    for version, retired in VERSIONS:
        plan = copy.deepcopy(original)
        plan["header"].update(format_version=version, executor_abi=f"tileinfer-decoder-v{version}")
        if retired:
            plan["header"]["model_kind"] = f"llama_decoder_{kind}_f32"
            plan["model"]["dtype"] = "float32"
        where = tmp_path / f"version{version}"
        where.mkdir()
        with pytest.raises(RuntimeError, match="unsupported decoder plan header"):
            load(path, plan, where)


def test_every_ownership_and_wave_rule_has_a_case():
    """Each message of check_ownership and of the wave-order rules in plan.cpp is the expected
    rejection of at least one mutation above."""
    source = (Path(__file__).resolve().parent.parent / "tiles_amd" / "csrc" / "plan.cpp").read_text()
    expected = {m for _, _, m in MUTATIONS + STACK_MUTATIONS + BLOCK_MUTATIONS if m}
    for rule in ("missing or overlapping output rows", "incomplete output ownership",
                 "a wave mixes opcodes or layers", "waves out of program order", "empty wave",
                 "attention chunks of a worker out of K/V head order", "two attention chunks of one K/V head share a worker"):
        assert rule in source, rule
        if rule != "two attention chunks of one K/V head share a worker":
            assert any(rule in m for m in expected), rule
