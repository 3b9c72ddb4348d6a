"""The controlled measurement protocol (tiles_amd/controlled.py, after the reference's
tileinfer/tests/controlled_decode.py:1-26) end to end on the GPU: two arms of a small bf16 stack
in resident servers, 2 blocks of 2 rounds at two contexts, the servers restarted in reverse
order halfway (block 1), and a clean exit.  The statistics themselves are pinned on the CPU
(tests/test_controlled.py)."""

import json
import math
import subprocess
import sys
from pathlib import Path

import pytest
import torch

from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

pytestmark = pytest.mark.gpu
ROOT = Path(__file__).resolve().parent.parent


@pytest.mark.timeout(600)
def test_controlled_protocol_two_arms(tmp_path):
    spec = P.StackSpec(P.BlockSpec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                                   head_dim=64, max_context=128), 2, 512, True)
    K.build_stack_package(spec, K.random_weights(spec, seed=17, std=0.08, dtype=torch.float32), probe.probe_library(),
                          tmp_path / "pkg", "bfloat16")
    out = tmp_path / "report.json"
    result = subprocess.run([sys.executable, "-m", "tiles_amd.controlled", "--arm", f"A={tmp_path / 'pkg'}",
                             "--arm", f"B={tmp_path / 'pkg'}", "--contexts", "1", "40", "--blocks", "2", "--rounds", "2",
                             "--tokens", "16", "--out", str(out)], cwd=ROOT, capture_output=True, text=True, timeout=540)
    print(result.stdout[-2000:], flush=True)
    assert result.returncode == 0, result.stderr[-3000:]
    report = json.loads(out.read_text())
    assert report["protocol"]["spawn_order_swapped_halfway"] and report["protocol"]["blocks"] == 2
    for arm in ("A", "B"):
        assert report["arms"][arm]["library"].endswith("libtileinfer_amd.so")
    for context in ("1", "40"):
        entry = report["contexts"][context]
        order = entry["spawn_order_by_block"]
        assert sorted(order["0"]) == ["A", "B"] and order["1"] == order["0"][::-1]  # restarted in reverse halfway
        summary = entry["summary"]
        for arm in ("A", "B"):
            assert math.isfinite(summary[arm]["median_us"]) and summary[arm]["median_us"] > 0
            assert len(summary[arm]["block_medians_us"]) == 2
        paired = summary["B"]["vs_A"]
        assert paired["pairs"] == 2 and all(math.isfinite(v) for v in (paired["mean_us"], *paired["ci95_us"]))
        assert paired["ci95_us"][0] <= paired["mean_us"] <= paired["ci95_us"][1]
        assert math.isfinite(paired["spawn_order_effect_us"])
        assert len(entry["blocks"]) == 4 and all(len(b["us_per_token"]) == 2 for b in entry["blocks"])
