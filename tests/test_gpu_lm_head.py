"""BASELINE config 2, the isolated LM-head step, as a launch of its own
(ti_context_lm_head_step): a bf16 hidden vector h ~ N(0, 1) [2048] through the final RMSNorm
(weight 1.0) and the tied-embedding GEMV against a [128256 x 2048] bf16 matrix ~ N(0, 0.02), then
greedy argmax with ties to the lowest ID (ops.cuh:842-911).

The package is a one-layer Llama-3.2-1B-width stack whose layer weights are zero (the step never
runs the layer).  For several seeded vectors the token must equal, bit for bit, the argmax of
the contract evaluated exactly (tests/contract64.py: RMSNorm with each rounding, each logit one
float64 dot product rounded to bf16), lowest index among equal values, and the oracle's
(oracle/decoder.py final_norm and a bf16 matmul, decoder_stack.py:126-155).  The logits must be
the exact contract's in at least 99.9% of entries, and each within one bf16 spacing of its value
or within 2^-14: the worker sums each 2048-term dot product in FP32, so a dot product that lands
within FP32 error of a bf16 rounding boundary rounds to its neighbour, and near 0, where bf16
spacings are finer than that error (about 1e-6 for these terms), by more than one spacing."""

import numpy as np
import pytest
import torch

from oracle import decoder as ref
from tests import contract64 as C64
from tiles_amd import runtime as R
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

pytestmark = [pytest.mark.gpu, pytest.mark.slow]
HIDDEN, VOCAB = 2048, 128256


@pytest.fixture(scope="module")
def head(tmp_path_factory):
    block = P.BlockSpec(hidden_size=HIDDEN, intermediate_size=8192, num_attention_heads=32, num_key_value_heads=8,
                        head_dim=64, max_context=8)
    spec = P.StackSpec(block, 1, VOCAB, True)
    generator = torch.Generator().manual_seed(20)
    weights = {}
    for name in K.weight_names(spec):
        shape = K.weight_shape(spec, name)
        weights[name] = torch.ones(shape) if name.endswith("norm") else torch.zeros(shape)
    weights["embedding"] = torch.randn(VOCAB, HIDDEN, generator=generator) * 0.02
    weights = {k: v.to(torch.bfloat16) for k, v in weights.items()}
    path = tmp_path_factory.mktemp("lm_head") / "pkg"
    K.build_stack_package(spec, weights, probe.probe_library(), path, "bfloat16")
    ospec = ref.Spec(hidden_size=HIDDEN, intermediate_size=8192, num_attention_heads=32, num_key_value_heads=8,
                     head_dim=64, max_context=8, layers=1, vocab_size=VOCAB)
    return path, weights, ospec


def bits_of(h: torch.Tensor) -> np.ndarray:
    return h.contiguous().view(torch.int16).numpy().view(np.uint16)


def test_lm_head_step_token_is_the_contracts(head):
    path, weights, ospec = head
    model = R.DecoderModel(R.load_plan(path))
    ctx = model.create_context()
    table = C64.as64(weights["embedding"])
    contract = C64.Contract({"final_norm": weights["final_norm"]}, ospec)
    generator = torch.Generator().manual_seed(21)
    for case in range(4):
        h = torch.randn(HIDDEN, generator=generator).to(torch.bfloat16)
        ticket = ctx.enqueue_lm_head_step(bits_of(h), rounds=3, logits=True)
        logits = ctx.collect(ticket)["logits"]
        result = ctx.wait(ticket)
        token = result.generated[0]
        exact = C64.bf16(table @ contract.rms_norm(C64.as64(h), contract.w["final_norm"]))
        want = int(np.argmax(exact))  # the first maximum: ties go to the lowest ID
        with torch.inference_mode():
            normed = ref.final_norm(h, weights["final_norm"], ospec.rms_norm_eps)
            oracle = int(torch.argmax((weights["embedding"] @ normed).float()))
        top = np.sort(exact)[-2:]
        spacing = np.where(exact == 0, 2.0 ** -133, np.ldexp(1.0, np.frexp(exact)[1] - 8))  # bf16 spacing at each value
        equal = float((logits == exact).mean())
        off = np.abs(logits - exact)
        far = float((off / spacing).max())
        outside = int(((off > spacing) & (off > 2.0 ** -14)).sum())
        print(f"case {case}: token {token}, exact {want}, oracle {oracle}, top-2 {top.tolist()}, "
              f"logits equal {equal:.6f}, max {far:.2f} spacings (largest such |difference| "
              f"{float(off[off > spacing].max()) if (off > spacing).any() else 0.0:.2e}), {result.compute_us:.1f} us",
              flush=True)
        assert token == want == oracle
        assert equal >= 0.999 and outside == 0
        assert result.compute_us > 0 and result.position == 0


def test_lm_head_step_leaves_the_context_empty(head):
    """The step refuses a context holding a sequence, and the context it ran on decodes after it
    as a fresh one does (same logits bit for bit)."""
    path, weights, _ = head
    model = R.DecoderModel(R.load_plan(path))
    fresh, used = model.create_context(), model.create_context()
    h = torch.randn(HIDDEN, generator=torch.Generator().manual_seed(22)).to(torch.bfloat16)
    first = used.wait(used.enqueue_lm_head_step(bits_of(h), rounds=2)).generated
    assert used.wait(used.enqueue_lm_head_step(bits_of(h))).generated == first
    want = fresh.collect(fresh.enqueue_decode(5, logits=True))["logits"]
    got = used.collect(used.enqueue_decode(5, logits=True))["logits"]
    np.testing.assert_array_equal(got, want)
    with pytest.raises(RuntimeError, match="LM-head step requires an empty sequence context"):
        used.enqueue_lm_head_step(bits_of(h))
    used.wait(used.enqueue_reset())
    assert used.wait(used.enqueue_lm_head_step(bits_of(h))).generated == first


def test_lm_head_step_fp32_and_small_bf16(tmp_path):
    """The step on small stacks of both element types (hidden 256, vocabulary 512, one layer):
    fp32 logits within 1e-5 of the oracle's FP32 final norm and GEMV, bf16 logits bit-equal to the
    exactly evaluated contract in at least 99% of entries, and both tokens the oracle's wherever
    its top-2 gap exceeds that difference."""
    block = P.BlockSpec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                        head_dim=64, max_context=8)
    spec = P.StackSpec(block, 1, 512, True)
    ospec = ref.Spec(hidden_size=256, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                     head_dim=64, max_context=8, layers=1, vocab_size=512)
    weights = K.random_weights(spec, seed=23, std=0.08, dtype=torch.float32)
    generator = torch.Generator().manual_seed(24)
    for dtype, tdt in (("float32", torch.float32), ("bfloat16", torch.bfloat16)):
        path = tmp_path / dtype
        K.build_stack_package(spec, weights, probe.probe_library(), path, dtype)
        packed = K.read_weights(path, spec, dtype)
        ctx = R.DecoderModel(R.load_plan(path)).create_context()
        for _ in range(3):
            h = torch.randn(256, generator=generator).to(tdt)
            vector = h.numpy() if dtype == "float32" else bits_of(h)
            ticket = ctx.enqueue_lm_head_step(vector, rounds=1, logits=True)
            logits = ctx.collect(ticket)["logits"]
            token = ctx.wait(ticket).generated[0]
            with torch.inference_mode():
                want = (packed["embedding"] @ ref.final_norm(h, packed["final_norm"], ospec.rms_norm_eps)).float().numpy()
            if dtype == "float32":
                diff = float(np.abs(logits - want).max())
                assert diff <= 1e-5, diff
            else:
                contract = C64.Contract({"final_norm": packed["final_norm"]}, ospec)
                exact = C64.bf16(C64.as64(packed["embedding"]) @ contract.rms_norm(C64.as64(h), contract.w["final_norm"]))
                assert float((logits == exact).mean()) >= 0.99
                diff = float(np.abs(logits - want).max())
            top = np.sort(want)[-2:]
            print(f"{dtype}: token {token}, oracle {int(np.argmax(want))}, max |got - oracle| {diff:.3g}, "
                  f"top-2 gap {top[1] - top[0]:.3g}", flush=True)
            if top[1] - top[0] > diff:
                assert token == int(np.argmax(want))
