"""The reference's special cases, through small stack packages on the GPU:

* all-zero weights: every logit ties at 0 and greedy keeps the smallest token id, so two generated
  tokens are [0, 0] (tileinfer/tests/kernel_regression.py:263-297); every RMSNorm of the stack
  (attention, FFN, final) then normalizes a zero vector, which must stay exactly 0 (the
  zero-norm case of ops_unit.py:410-418);
* down projection + residual on ties-to-even boundaries (ops_unit.py:386-408);
* embedding rows with boundary values, +-0, the smallest bf16 subnormal, the smallest normal
  and +-the largest finite bf16, carried bit-exactly (ops_unit.py:419-436).

The reference checks the last two on its single-op harness; this worker has no single-op entry
point, so the cases are built into one-layer stacks whose other weights make the layer exact.
"""

import numpy as np
import pytest
import torch

from oracle import decoder as ref
from tiles_amd import runtime as R
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

pytestmark = pytest.mark.gpu
HIDDEN = 256


@pytest.fixture(scope="module")
def target():
    return probe.probe_library()


def tiny_stack(layers=1, vocab=512):
    block = P.BlockSpec(hidden_size=HIDDEN, intermediate_size=512, num_attention_heads=4, num_key_value_heads=1,
                        head_dim=64, max_context=16)
    return P.StackSpec(block, layers, vocab, True)


def oracle_spec(spec):
    b = spec.block
    return ref.Spec(hidden_size=b.hidden_size, intermediate_size=b.intermediate_size,
                    num_attention_heads=b.num_attention_heads, num_key_value_heads=b.num_key_value_heads,
                    head_dim=b.head_dim, max_context=b.max_context, layers=spec.layers, vocab_size=spec.vocab_size)


def zeros(spec):
    return {name: torch.zeros(K.weight_shape(spec, name)) for name in K.weight_names(spec)}


def context(spec, weights, target, path, dtype):
    K.build_stack_package(spec, weights, target, path, dtype)
    return R.DecoderModel(R.load_plan(path)).create_context()


def bits(values: np.ndarray) -> np.ndarray:
    return np.asarray(values, dtype=np.float32).view(np.uint32)


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_all_zero_weights_tie_to_the_smallest_token(target, tmp_path, dtype):
    spec = tiny_stack(layers=2)
    ctx = context(spec, zeros(spec), target, tmp_path / "zeros", dtype)
    got = ctx.collect(ctx.enqueue_decode(1, logits=True, block_outputs=True))
    # Zero inputs through every RMSNorm: exactly zero block outputs and logits, nothing non-finite.
    assert np.all(bits(got["block_outputs"]) == 0), "a zero vector's RMSNorm must stay +0"
    assert np.all(bits(got["logits"]) == 0)
    ctx.wait(ctx.enqueue_reset())
    ctx.wait(ctx.enqueue_prefill([1]))
    result = ctx.wait(ctx.enqueue_generate(2))
    assert result.generated == [0, 0], result.generated
    assert result.stop_reason == "limit"


def ties_weights(spec):
    """A one-layer stack whose block output is the ops_unit.py tie case in every element.

    Embedding row 0 is x = [+1/256] * 128 + [-1/256] * 128 and Wo = 0, so r = x.  The FFN has two
    live rows with p = round(round(silu(16)) * 1/16) = 1 exactly (gate and up read only z[0] > 0),
    and Wdown^T rows [s, s/256] for output sign s, so down = round(s (1 + 2^-8)) = s: a tie that
    rounds to the even mantissa.  y = round(r + down) = round(s/256 + s) = s: a tie again."""
    w = zeros(spec)
    half = HIDDEN // 2
    x = torch.cat([torch.full((half,), 1 / 256), torch.full((half,), -1 / 256)])
    w["embedding"][0] = x
    w["L0.attn_norm"][:] = 1.0
    w["L0.ffn_norm"][:] = 1.0
    w["final_norm"][:] = 1.0
    eps = spec.block.rms_norm_eps
    z0 = float(torch.tensor(float(x[0]) / np.sqrt(float((x * x).mean()) + eps)).to(torch.bfloat16))
    for row in (0, 1):
        w["L0.Wgate"][row, 0] = 16.0 / z0
        w["L0.Wup"][row, 0] = (1 / 16) / z0
    sign = torch.sign(x)
    w["L0.Wdown"][:, 0] = sign            # [hidden, intermediate]: column j multiplies product j
    w["L0.Wdown"][:, 1] = sign / 256
    return w, sign


def test_down_projection_and_residual_ties_to_even(target, tmp_path):
    """bf16 only: the ties are bf16 rounding points (in fp32 silu(16) is not 16, and both sums
    are exact)."""
    spec = tiny_stack()
    weights, sign = ties_weights(spec)
    weights = {k: v.to(torch.bfloat16) for k, v in weights.items()}
    want = sign.numpy()  # both additions tie, and round to the even neighbour, +-1
    with torch.inference_mode():
        cache = ref.StackCache.empty(oracle_spec(spec), torch.bfloat16)
        trace = ref.decode_token(0, weights, oracle_spec(spec), cache, keep_blocks=True)["blocks"][0]
    ffn = trace["ffn"].float().numpy()
    assert np.array_equal(ffn, want), "down = round(s (1 + 2^-8)) must tie to s"
    np.testing.assert_array_equal(trace["y"].float().numpy(), want)
    ctx = context(spec, weights, target, tmp_path / "ties", "bfloat16")
    got = ctx.collect(ctx.enqueue_decode(0, block_outputs=True))["block_outputs"]
    np.testing.assert_array_equal(bits(got), bits(want))


@pytest.mark.parametrize("dtype", ["float32", "bfloat16"])
def test_embedding_boundary_values_keep_their_bits(target, tmp_path, dtype):
    """Through a layer of zero weights y = round(round(x + 0) + 0): every value keeps its bits except
    -0, which x + (+0) turns into +0 in IEEE arithmetic (the oracle does the same)."""
    spec = tiny_stack()
    boundary = torch.tensor([0.0, -0.0, 2.0 ** -133, -(2.0 ** -133), 2.0 ** -126, (2.0 - 2.0 ** -7) * 2.0 ** 127,
                             -(2.0 - 2.0 ** -7) * 2.0 ** 127, 1.0], dtype=torch.float32)
    w = zeros(spec)
    w["embedding"][3] = boundary.repeat(HIDDEN // len(boundary))
    tdt = torch.bfloat16 if dtype == "bfloat16" else torch.float32
    w = {k: v.to(tdt) for k, v in w.items()}
    assert torch.equal(w["embedding"][3][:8].float().view(torch.int32), boundary.to(tdt).float().view(torch.int32))
    ctx = context(spec, w, target, tmp_path / "boundary", dtype)
    got = ctx.collect(ctx.enqueue_decode(3, logits=True, block_outputs=True))
    with torch.inference_mode():
        cache = ref.StackCache.empty(oracle_spec(spec), tdt)
        out = ref.decode_token(3, w, oracle_spec(spec), cache, keep_blocks=True)
    want = out["blocks"][0]["y"].float().numpy()
    x = w["embedding"][3].float().numpy()
    expected = np.where(bits(x) == 0x80000000, np.float32(0.0), x)  # -0 + 0 = +0
    np.testing.assert_array_equal(bits(want), bits(expected))
    np.testing.assert_array_equal(bits(got["block_outputs"]), bits(expected))
    assert np.isfinite(got["logits"]).all()
