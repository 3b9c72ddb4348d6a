"""Package format, planner and C++ loader checks that need no GPU.

Modelled on the reference's planner and loader tests (tileplan/tests/test_decoder_planning.py,
test_decoder_stack.py:75-151, tileinfer/tests/loader_regression.py:196-410,
plan_loader_test.cpp:21-35, cli_regression.py:8-80): packages are built for a fixture
target, loaded by the C++ loader against that target (no device call), and mutations must be
rejected with the loader's message.
"""

import copy
import ctypes
import ctypes as C
import hashlib
import json
import re
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from tiles_amd import runtime as R
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

ROOT = Path(__file__).resolve().parent.parent
GOLDEN = Path(__file__).parent / "golden"
TARGET = probe.mi355x_target()


def m4_spec():
    model = json.loads((GOLDEN / "decoder_m4" / "model.json").read_text())
    block = P.BlockSpec(**{k: model[k] for k in P.BlockSpec.__dataclass_fields__ if k in model})
    return P.StackSpec(block, model["layers"], model["vocab_size"], model["tie_word_embeddings"])


def m4_weights():
    with np.load(GOLDEN / "decoder_m4" / "weights.npz", allow_pickle=False) as data:
        return {k: torch.from_numpy(data[k].copy()) for k in data.files}


@pytest.fixture(scope="module")
def packages(tmp_path_factory):
    root = tmp_path_factory.mktemp("packages")
    out = {}
    for dtype in ("float32", "bfloat16"):
        K.build_stack_package(m4_spec(), m4_weights(), TARGET, root / dtype, dtype)
        out[dtype] = root / dtype
    return out


def load(path, verify=True):
    return R.Plan(path, verify, R.target_from_probe(TARGET))


def test_library_exports_every_declared_symbol():
    header = (ROOT / "include" / "tileinfer_amd.h").read_text()
    declared = set(re.findall(r"\b(ti_[a-z_0-9]+)\s*\(", header))
    lib = R.library()
    for name in declared:
        assert hasattr(lib, name), name
    assert set(R.EXPORTS) <= declared
    assert lib.ti_abi().decode() == P.ABI
    assert lib.ti_fingerprint().decode() == probe.FINGERPRINT


def test_stack_package_layout_and_schedule(packages):
    plan = K.read_plan(packages["bfloat16"])
    spec = m4_spec()
    # 1 + 6L + 2 waves (docs/architecture.md:151-161); conditional barrier skipped up to the
    # fused length, min(384, chunk capacity) (plan_core.py:102,125).
    assert len(plan["waves"]) == 1 + 6 * spec.layers + 2
    assert plan["model"]["attention_chunks"] == 1
    conditional = [w for w in plan["waves"] if "conditional_barrier" in w]
    assert len(conditional) == spec.layers
    assert all(w["conditional_barrier"] == {"skip_up_to_length": 384} for w in conditional)
    assert plan["storage"]["stack"]["lm_head_alias"] is True
    data = (packages["bfloat16"] / "weights.bin").read_bytes()
    assert hashlib.sha256(data).hexdigest() == plan["integrity"]["weights_sha256"]
    # bf16 packing rounds to nearest even, Wdown transposed [f, d]
    weights = K.read_weights(packages["bfloat16"], spec, "bfloat16")
    for name in ("L0.Wq", "L2.Wdown", "embedding"):
        torch.testing.assert_close(weights[name], m4_weights()[name].to(torch.bfloat16), atol=0, rtol=0)


def test_planner_matches_reference_counts_at_mi355x_scale():
    spec = P.llama32_1b(4160)
    plan = P.stack_plan(spec, P.plan_target(TARGET), "bfloat16", "0" * 64, 128)
    model = plan["model"]
    assert model["attention_chunks"] == 33 and model["ffn_chunks"] == 256
    assert plan["storage"]["selection_bytes"] == 8 * 256
    assert len(plan["waves"]) == 99
    qkv = [t for t in plan["tasks"] if t["opcode"] == "qkv_bf16" and t["layer"] == 0]
    assert [t["operands"]["rows"] for t in qkv][:2] == [[0, 12], [12, 24]]
    # earliest-wave, least-loaded schedule: equal-work QKV tasks go to workers in ID order
    assert [t["worker"] for t in qkv] == list(range(256))
    assert plan["storage"]["weight_bytes"] == 2471628800


def test_loader_accepts_and_encodes_streams(packages):
    for dtype, path in packages.items():
        info = load(path).inspect()
        assert info["workers"] == 256 and info["wave_count"] == 21
        assert info["weight_dtype"] == dtype
        # every worker reaches the same 20 barriers
        assert info["instruction_count"] == info["task_count"] + 20 * 256


def mutate(src: Path, dst: Path, edit) -> Path:
    plan = json.loads((src / "plan.json").read_text())
    edit(plan)
    dst.mkdir()
    (dst / "plan.json").write_bytes(P.json_bytes(plan))
    (dst / "weights.bin").write_bytes((src / "weights.bin").read_bytes())
    return dst


MUTATIONS = [
    ("version", lambda p: p["header"].update(format_version=9), "unsupported decoder plan header"),
    ("abi", lambda p: p["header"].update(executor_abi="other"), "unsupported decoder plan header"),
    ("policy", lambda p: p["model"].update(numeric_policy="x"), "inconsistent numeric policy"),
    ("hidden", lambda p: p["model"].update(hidden_size=48), "unsupported decoder dimensions"),
    ("chunks", lambda p: p["model"].update(attention_chunks=2), "invalid attention chunking"),
    ("kv_range", lambda p: p["model"].update(max_context=1 << 26),
     "K/V cache of one layer exceeds the worker's 2 GiB buffer addressing"),
    ("layers", lambda p: p["model"].update(layers=121), "more layers than the bf16 worker's exchange tags allow"),
    ("descriptor", lambda p: p["model"]["tensors"][2].update(shape=[1, 1]), "invalid tensor descriptors"),
    ("fingerprint", lambda p: p["target"].update(kernel_fingerprint="sm86"), "does not match compiled worker"),
    ("workers", lambda p: p["target"].update(worker_count=20), "does not match compiled worker"),
    ("scratch", lambda p: p["storage"].update(scratch_bytes=1), "invalid decoder tensor storage"),
    ("stack", lambda p: p["storage"]["stack"].update(layer_weight_stride=64), "invalid decoder stack storage"),
    ("hash", lambda p: p["integrity"].update(weights_sha256="0" * 64), "decoder weight checksum mismatch"),
    ("operands", lambda p: p["tasks"][300]["operands"].update(rows=[0, 1]), "invalid task operands"),
    ("duplicate", lambda p: p["tasks"][5].update(id=4), "duplicate task ID"),
    ("worker", lambda p: p["tasks"][40].update(worker=(p["tasks"][40]["worker"] + 1) % 256),
     "assigned to a different wave/worker"),
    ("conditional", lambda p: [w.pop("conditional_barrier", None) for w in p["waves"]], "invalid conditional barrier"),
    ("opcode", lambda p: p["tasks"][0].update(opcode="embedding_f32"), "opcode precision differs"),
]


@pytest.mark.parametrize("name,edit,message", MUTATIONS, ids=[m[0] for m in MUTATIONS])
def test_loader_rejects_mutations(packages, tmp_path, name, edit, message):
    path = mutate(packages["bfloat16"], tmp_path / name, edit)
    with pytest.raises(RuntimeError, match=re.escape(message)):
        load(path)


def test_loader_rejects_truncated_weights(packages, tmp_path):
    dst = tmp_path / "short"
    dst.mkdir()
    (dst / "plan.json").write_bytes((packages["float32"] / "plan.json").read_bytes())
    (dst / "weights.bin").write_bytes((packages["float32"] / "weights.bin").read_bytes()[:-64])
    with pytest.raises(RuntimeError, match="invalid decoder stack storage"):
        load(dst)


def test_unverified_load_trusts_declared_hash(packages, tmp_path):
    dst = tmp_path / "flip"
    dst.mkdir()
    (dst / "plan.json").write_bytes((packages["float32"] / "plan.json").read_bytes())
    raw = bytearray((packages["float32"] / "weights.bin").read_bytes())
    raw[100] ^= 1
    (dst / "weights.bin").write_bytes(bytes(raw))
    load(dst, verify=False)
    with pytest.raises(RuntimeError, match="checksum mismatch"):
        load(dst, verify=True)


def test_checkpoint_import_round_trip(tmp_path):
    spec = P.StackSpec(P.BlockSpec(hidden_size=2048, intermediate_size=8192, num_attention_heads=32,
                                   num_key_value_heads=8, head_dim=64, max_context=8), layers=1,
                       vocab_size=128256)
    weights = K.random_weights(spec, seed=3)
    assert float(weights["L0.Wq"].float().std()) == pytest.approx(0.02, rel=0.02)
    assert torch.equal(weights["final_norm"], torch.ones(2048, dtype=torch.bfloat16))
    checkpoint = K.write_checkpoint(spec, weights, tmp_path / "ckpt")
    config = json.loads((checkpoint / "config.json").read_text())
    assert config["rope_scaling"]["rope_type"] == "llama3" and config["num_hidden_layers"] == 1
    with pytest.raises(ValueError, match="unsupported Llama config num_hidden_layers"):
        K.read_checkpoint(checkpoint, 64)


CLI = ROOT / "tiles_amd" / "tile_runtime"


@pytest.mark.parametrize("args,message", [
    ([], "missing mode"),
    (["fly"], "unknown mode"),
    (["generate", "p", "i.json"], "missing required option"),
    (["generate", "p", "i.json", "--max-new-tokens", "0"], "invalid generation or benchmark arguments"),
    (["generate", "p", "i.json", "--max-new-tokens", "2", "--max-new-tokens", "3"], "duplicate option"),
    (["generate", "p", "i.json", "--max-new-tokens", "2", "--selection", "top-k"], "only greedy selection"),
    (["bench", "p", "i.json", "--new-tokens", "2", "--warmup", "1"], "missing required option"),
    (["generate", "p", "i.json", "--max-new-tokens", "x"], "invalid integer"),
])
def test_cli_argument_errors_fail_before_any_device_call(args, message):
    result = subprocess.run([str(CLI), *args], capture_output=True, text=True, env={"HIP_VISIBLE_DEVICES": ""})
    assert result.returncode == 2
    assert result.stderr.startswith("tile_runtime: ") and message in result.stderr


def test_probe_normalization():
    raw = {"device": TARGET["device"], "executor": TARGET["executor"]}
    assert probe.normalize(raw)["launch"]["worker_count"] == 256
    bad = copy.deepcopy(raw)
    bad["executor"]["abi"] = "tileinfer-decoder-v9"
    with pytest.raises(ValueError, match="lacks required decoder capabilities"):
        probe.normalize(bad)


def test_launch_records_match_the_c_layout(tmp_path):
    """The ctypes mirrors of the launch boundary (tiles_amd/runtime.py) have the C header's field
    offsets and sizes (a C program built with gcc from include/tileinfer_amd.h prints them)."""
    import shutil
    import subprocess

    if shutil.which("gcc") is None:
        pytest.skip("no C compiler")
    structs = {"ti_worker_program_view": R.ProgramView, "ti_worker_buffers": R.WorkerBuffers,
               "ti_token_input": R.TokenInput, "ti_selection": R.Selection, "ti_model_shape": R.ModelShape,
               "ti_layer_layout": R.LayerLayout, "ti_numeric_config": R.NumericConfig, "ti_stack_config": R.StackConfig,
               "ti_worker_task_range": R.TaskRange, "ti_task_record": R.TaskRecord}
    lines = ["#include <stddef.h>", "#include <stdio.h>", '#include "tileinfer_amd.h"', "int main(void) {"]
    for name, mirror in structs.items():
        lines.append(f'printf("{name} sizeof %zu\\n", sizeof({name}));')
        for field, _ in mirror._fields_:
            lines.append(f'printf("{name} {field} %zu\\n", offsetof({name}, {field}));')
    lines.append("return 0; }")
    (tmp_path / "layout.c").write_text("\n".join(lines))
    subprocess.run(["gcc", "-I", str(ROOT / "include"), str(tmp_path / "layout.c"), "-o", str(tmp_path / "layout")],
                   check=True)
    printed = subprocess.run([str(tmp_path / "layout")], check=True, capture_output=True, text=True).stdout
    for line in printed.splitlines():
        name, field, value = line.split()
        mirror = structs[name]
        expected = C.sizeof(mirror) if field == "sizeof" else getattr(mirror, field).offset
        assert int(value) == expected, line


def test_static_entry_point_rejects_an_oversized_exchange_before_any_device_call():
    """ti_enqueue_worker_static checks the model's exchange area against its device array before
    it touches a device (this container has none)."""
    view = R.ProgramView()
    view.shape.hidden_size, view.shape.intermediate_size, view.shape.kv_heads = 4096, 1 << 22, 8
    view.stack.layers, view.selection_slots, view.weight_dtype = 16, 256, 1
    buffers = R.WorkerBuffers()
    code = R.library().ti_enqueue_worker_static(None, C.byref(view), C.byref(buffers), 0, R.TokenInput(-1, None, 1),
                                                R.Selection(), None)
    assert code == 1 and "exceeds the static array" in R.library().ti_last_error_message().decode()


def test_timeline_record_sizes_follow_the_header():
    """The header's timeline record sizes (the reference's kTimelineFields = 3, launch.cuh:25-28,
    and this build's 4) are the ones the Python binding uses, and a launch asking for any other
    size is rejected before any device call."""
    header = (ROOT / "include" / "tileinfer_amd.h").read_text()
    assert re.search(r"#define TI_TIMELINE_REFERENCE_FIELDS 3\b", header)
    assert re.search(r"#define TI_TIMELINE_FIELDS 4\b", header)
    assert (R.TIMELINE_REFERENCE_FIELDS, R.TIMELINE_FIELDS) == (3, 4)
    view = R.ProgramView()
    s = view.shape
    s.hidden_size, s.intermediate_size, s.query_heads, s.kv_heads, s.head_dim = 2048, 8192, 32, 8, 64
    s.max_context, s.attention_chunks, s.attention_chunk_steps, s.attention_fused_steps, s.ffn_chunks = 321, 1, 1056, 384, 256
    view.stack.layers, view.stack.vocab_size, view.stack.full_stack = 16, 128256, 1
    view.stack.layer_weight_stride = 60_000_000
    view.workers, view.selection_slots, view.weight_dtype = 256, 256, 1
    view.instructions = view.streams = view.weights = 16
    view.rotary_frequencies = 16
    buffers = R.WorkerBuffers()
    for field in ("input", "output", "scratch", "kv", "logits", "attention_partials", "selection", "exchange"):
        setattr(buffers, field, 16)
    buffers.epoch, buffers.timeline_fields = 1, 5
    code = R.library().ti_enqueue_worker(None, C.byref(view), C.byref(buffers), 0, R.TokenInput(-1, None, 1),
                                         R.Selection())
    assert code == 1 and b"invalid timeline record size" in R.library().ti_last_error_message()
