"""include/tileinfer_amd.hpp, the C++ runtime API in the shape of the reference's runtime.hpp:
a host program (tests/cpp/runtime_host.cpp) builds against it and the library with g++ (CPU), and
on the GPU its results equal the Python binding's on the same package."""

import json
import subprocess
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
LIB = ROOT / "tiles_amd"


def build(tmp_path) -> Path:
    exe = tmp_path / "runtime_host"
    subprocess.run(["g++", "-std=c++20", "-O1", "-Wall", "-Werror", f"-I{ROOT / 'include'}",
                    str(ROOT / "tests" / "cpp" / "runtime_host.cpp"), f"-L{LIB}", "-ltileinfer_amd",
                    f"-Wl,-rpath,{LIB}", "-o", str(exe)], check=True)
    return exe


def test_cpp_host_builds_against_the_header(tmp_path):
    if not (LIB / "libtileinfer_amd.so").exists():
        pytest.skip("library not built")
    assert build(tmp_path).exists()


@pytest.mark.gpu
def test_cpp_host_matches_the_python_binding(tmp_path):
    import torch

    from oracle import decoder as ref
    from tiles_amd import runtime as R
    from tiles_amd.tileplan import package as K
    from tiles_amd.tileplan import plan as P
    from tiles_amd.tileplan import probe

    block = P.BlockSpec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                        head_dim=64, max_context=32)
    spec = P.StackSpec(block, 2, 512, True)
    weights = K.random_weights(spec, seed=21, std=0.08)
    K.build_stack_package(spec, weights, probe.probe_library(), tmp_path / "pkg", "bfloat16")
    # This process decodes first and keeps its contexts while the C++ host runs beside it: the
    # worker's launch must not claim the device for one process (a cooperative launch on ROCm does).
    model = R.DecoderModel(R.load_plan(tmp_path / "pkg"))
    a, b = model.create_context(), model.create_context()
    a.wait(a.enqueue_prefill([7]))
    ra = a.wait(a.enqueue_generate(5))
    b.wait(b.enqueue_prefill([3, 4]))
    tb = b.enqueue_decode(5, logits=True)
    logits = b.collect(tb)["logits"]
    rb = b.wait(tb)
    out = subprocess.run([str(build(tmp_path)), str(tmp_path / "pkg")], check=True, capture_output=True, text=True,
                         timeout=120)
    got = json.loads(out.stdout)
    assert got["generated"] == ra.generated and got["position"] == ra.position == 6
    assert got["stop"] == "limit"
    assert got["b_position"] == rb.position == 3
    assert got["b_logits"] == 512 and got["b_argmax"] == int(np.argmax(logits))
    assert got["b_kv"] == 0  # not requested: empty, as the reference's collect
    assert got["reset_position"] == 0
    head = model.create_context()
    want_head = head.wait(head.enqueue_lm_head_step(np.full(256, 0x3F80, dtype=np.uint16), rounds=2)).generated
    assert got["head_token"] == want_head[0]
    # and the tokens are the oracle's
    packed = K.read_weights(tmp_path / "pkg", spec, "bfloat16")
    ospec = ref.Spec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                     head_dim=64, max_context=32, layers=2, vocab_size=512)
    assert got["generated"] == ref.generate([7], 5, packed, ospec, torch.bfloat16)["tokens"]
