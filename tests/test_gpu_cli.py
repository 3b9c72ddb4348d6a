"""The `tile_runtime` command a foreign host (the reference's generate.py) runs: `generate` and
`check` on the GPU, their JSON fields against the reference CLI's (tileinfer/src/runtime/
main.cpp:412-429 generate, :169-222 run_stack), and their values against the Python binding on the
same package (the same kernel, so bit-equal) and the oracle's tokens."""

import hashlib
import json
import subprocess
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import decoder as ref
from tiles_amd import runtime as R
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

pytestmark = pytest.mark.gpu
CLI = Path(__file__).resolve().parents[1] / "tiles_amd" / "tile_runtime"
GENERATE_FIELDS = {"prompt_tokens", "generated", "generated_count", "position", "stop_reason", "compute_us",
                   "plan_sha256", "weights_sha256"}
STEP_FIELDS = {"token_id", "position", "logits", "k", "v"}


@pytest.fixture(scope="module")
def package(tmp_path_factory):
    block = P.BlockSpec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                        head_dim=64, max_context=32)
    spec = P.StackSpec(block, 2, 512, True)
    weights = K.random_weights(spec, seed=31, std=0.08)
    path = tmp_path_factory.mktemp("cli") / "pkg"
    K.build_stack_package(spec, weights, probe.probe_library(), path, "bfloat16")
    ospec = ref.Spec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                     head_dim=64, max_context=32, layers=2, vocab_size=512)
    return spec, path, K.read_weights(path, spec, "bfloat16"), ospec


def run(*args) -> dict:
    out = subprocess.run([str(CLI), *map(str, args)], check=True, capture_output=True, text=True, timeout=120)
    return json.loads(out.stdout)


def test_generate_json(package, tmp_path):
    spec, path, packed, ospec = package
    (tmp_path / "in.json").write_text(json.dumps({"tokens": [7, 9]}))
    got = run("generate", path, tmp_path / "in.json", "--max-new-tokens", 6)
    assert GENERATE_FIELDS <= set(got), GENERATE_FIELDS - set(got)
    want = ref.generate([7, 9], 6, packed, ospec, torch.bfloat16)["tokens"]
    assert got["generated"] == want
    assert got["generated_count"] == 6 and got["prompt_tokens"] == 2 and got["position"] == 8
    assert got["stop_reason"] == "limit" and got["compute_us"] > 0
    assert got["plan_sha256"] == hashlib.sha256((path / "plan.json").read_bytes()).hexdigest()
    # An EOS id stops the generation after it is emitted.
    eos = want[2]
    stopped = run("generate", path, tmp_path / "in.json", "--max-new-tokens", 6, "--eos-id", eos)
    first = want.index(eos)
    assert stopped["generated"] == want[:first + 1] and stopped["stop_reason"] == "eos"
    assert stopped["position"] == 2 + first + 1


def test_check_json(package, tmp_path):
    spec, path, packed, ospec = package
    request = {"tokens": [7, 3, {"reset": True}, 5], "trace_blocks": True}
    (tmp_path / "check.json").write_text(json.dumps(request))
    got = run("check", path, tmp_path / "check.json")
    assert set(got) >= {"steps", "position", "valid"} and got["valid"] is True
    assert [s["token_id"] for s in got["steps"]] == [7, 3, 5]
    assert [s["position"] for s in got["steps"]] == [0, 1, 0]
    assert got["position"] == 1
    for s in got["steps"]:
        assert STEP_FIELDS | {"blocks"} <= set(s)
        assert len(s["k"]) == len(s["v"]) == spec.layers and len(s["k"][0]) == 64
        assert len(s["blocks"]) == spec.layers and len(s["blocks"][0]) == 256
    # The same decode through the Python binding: bit-equal logits, K/V rows and block outputs.
    ctx = R.DecoderModel(R.load_plan(path)).create_context()
    plan = K.read_plan(path)
    kv_at = {e["tensor"]: e["offset"] // 2 for e in plan["storage"]["kv"]}
    stride = plan["storage"]["stack"]["layer_kv_stride"] // 2
    for step, token in zip(got["steps"][:2], (7, 3)):
        snap = ctx.collect(ctx.enqueue_decode(token, logits=True, kv=True, block_outputs=True))
        np.testing.assert_array_equal(np.array(step["logits"], dtype=np.float32), snap["logits"])
        for layer in range(spec.layers):
            base = layer * stride + step["position"] * 64
            np.testing.assert_array_equal(np.array(step["k"][layer], dtype=np.float32),
                                          snap["kv"][kv_at[P.TID["K"]] + base:][:64])
            np.testing.assert_array_equal(np.array(step["v"][layer], dtype=np.float32),
                                          snap["kv"][kv_at[P.TID["V"]] + base:][:64])
            np.testing.assert_array_equal(np.array(step["blocks"][layer], dtype=np.float32),
                                          snap["block_outputs"][layer * 256:(layer + 1) * 256])
    # and the oracle's greedy token after each step
    cache = ref.StackCache.empty(ospec, torch.bfloat16)
    for step, token in zip(got["steps"][:2], (7, 3)):
        want = ref.decode_token(token, packed, ospec, cache)["logits"]
        assert int(np.argmax(step["logits"])) == ref.greedy(want)
