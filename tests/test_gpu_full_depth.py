"""BASELINE configs 4 and 5 at full depth: the random-init Llama-3.2-1B (16 layers, vocabulary
128,256, the benchmark's seed-0 weights), a seeded uniform prompt of 4,096 or 32,768 tokens
prefilled through the matrix prefill, then one 64-token generate launch, as bench.py runs them.

The CPU cannot prefill 32,768 positions of a 16-layer model in a test's time, so the oracle's cache
(oracle/decoder.py, the reference's decoder_reference.py:190-270) and the exactly evaluated bf16
contract's (tests/contract64.py) are seeded from the GPU's K/V snapshot of every position before
the last prompt token, and both decode teacher-forced from there: the last prompt token, then the
generated tokens.  The prefill itself is checked where it depends on the prompt alone: layer 0's
K and V rows against the oracle's own (tests/test_gpu_prefill.py covers deeper layers on smaller
stacks).  Bars, as in the reference's bf16 comparisons (stack_regression.py:33-96,
kernel_regression.py:111-297) and its calibration rule (bf16_checkpoint_tolerances.json):

* every step's logits within max(2e-2, 1.25 x the drift between the oracle and the exact
  contract) of the oracle's, the RMS error within twice the drift's;
* the worker no further from the exact contract than the oracle is (largest and RMS error over
  the exactly evaluated steps), the share of logits within 2e-2 of it printed;
* the generated token equal to the oracle's greedy choice wherever its top-2 gap exceeds the bound.
"""

import numpy as np
import pytest
import torch

from oracle import decoder as ref
from tests import contract64 as C64
from tiles_amd import runtime as R
from tiles_amd import synthetic as S
from tiles_amd.tileplan import package as K
from tiles_amd.tileplan import plan as P
from tiles_amd.tileplan import probe

pytestmark = [pytest.mark.gpu, pytest.mark.slow]
NEW_TOKENS = 64


@pytest.fixture(scope="module")
def llama_weights():
    return K.random_weights(P.llama32_1b(64), seed=0)


def oracle_spec(max_context: int) -> ref.Spec:
    return ref.Spec(hidden_size=2048, intermediate_size=8192, num_attention_heads=32, num_key_value_heads=8,
                    head_dim=64, max_context=max_context, layers=16, vocab_size=128256)


def snapshot_kv(snapshot: np.ndarray, plan: dict, count: int):
    """K and V of the first `count` positions of every layer: float32 [layers, count, kv_heads, head_dim]."""
    m = plan["model"]
    width = m["num_key_value_heads"] * m["head_dim"]
    at = {e["tensor"]: e["offset"] // 2 for e in plan["storage"]["kv"]}
    stride = plan["storage"]["stack"]["layer_kv_stride"] // 2
    out = []
    for tid in (P.TID["K"], P.TID["V"]):
        rows = [snapshot[layer * stride + at[tid]:][: count * width] for layer in range(m["layers"])]
        out.append(np.stack(rows).reshape(m["layers"], count, m["num_key_value_heads"], m["head_dim"]))
    return out


def bf16_ulps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    ia = (np.asarray(a, dtype=np.float32).view(np.uint32) >> 16).astype(np.int64)
    ib = (np.asarray(b, dtype=np.float32).view(np.uint32) >> 16).astype(np.int64)
    ia = np.where(ia & 0x8000, -(ia & 0x7FFF), ia)
    ib = np.where(ib & 0x8000, -(ib & 0x7FFF), ib)
    return np.abs(ia - ib)


def scaled_ulps(got: np.ndarray, want: np.ndarray, rotated: bool) -> np.ndarray:
    """|got - want| in bf16 ulps of the scale of the element's terms: max(|want|, |got|, the RMS of
    its row (last axis)), and for a rotated element the norm of its rotation pair (i, i + dh/2),
    which the rotation keeps: bf16(a c) - bf16(b s) cancels far below |a|, |b|, where one ulp of
    difference in a, b or the bf16 cos/sin is many ulps of the small result (or flips its sign)."""
    got, want = np.asarray(got, dtype=np.float64), np.asarray(want, dtype=np.float64)
    rms = np.sqrt((want ** 2).mean(axis=-1, keepdims=True))
    scale = np.maximum(np.maximum(np.abs(want), np.abs(got)), rms)
    if rotated:
        half = want.shape[-1] // 2
        partner = np.concatenate((want[..., half:], want[..., :half]), axis=-1)
        scale = np.maximum(scale, np.sqrt(want ** 2 + partner ** 2))
    ulp = np.exp2(np.floor(np.log2(np.maximum(scale, 1e-30))) - 7)
    return np.abs(got - want) / ulp


def first_layer_kv(prompt: list[int], weights: dict, ospec: ref.Spec):
    """The oracle's layer-0 K and V rows of a prompt, batched (append_kv's operations per row)."""
    w = ref.layer_weights(weights, 0)
    with torch.inference_mode():
        u = ref.rms_norm(weights["embedding"][prompt], w["attn_norm"], ospec.rms_norm_eps)
        k = (u @ w["Wk"].T).reshape(len(prompt), ospec.num_key_value_heads, ospec.head_dim)
        v = (u @ w["Wv"].T).reshape(len(prompt), ospec.num_key_value_heads, ospec.head_dim)
        k = ref.apply_rope(k, torch.arange(len(prompt), dtype=torch.float32), ospec)
    return k.float().numpy(), v.float().numpy()


def check_config(tmp_path, weights, context: int, chunk_steps: int, prompt_seed: int, oracle_steps: int,
                 exact_steps: int):
    max_context = context + NEW_TOKENS
    path = tmp_path / f"llama{context}"
    S.llama_package(path, max_context, "bfloat16", seed=0, chunk_steps=chunk_steps, target=probe.probe_library(),
                    weights=weights)
    plan = K.read_plan(path)
    model = R.DecoderModel(R.load_plan(path, verify_weights=False))
    ctx = model.create_context()
    prompt = S.prompt(context, seed=prompt_seed)
    # The benchmark's request: prefill (matrices, then the worker for the last prompt token) and one
    # 64-token generate launch.
    ticket = ctx.enqueue_prefill(prompt, logits=True, kv=True)
    snap = ctx.collect(ticket)
    ctx.wait(ticket)
    generated = ctx.wait(ctx.enqueue_generate(NEW_TOKENS)).generated
    assert len(generated) == NEW_TOKENS
    print(f"ctx {context}: prefilled and generated {NEW_TOKENS} tokens in one launch", flush=True)
    # The same steps one at a time for their logits: the prefill's last step gives step 0's.
    ctx.wait(ctx.enqueue_reset())
    again = ctx.enqueue_prefill(prompt, logits=True)
    gpu_logits = [ctx.collect(again)["logits"]]
    ctx.wait(again)
    np.testing.assert_array_equal(gpu_logits[0], snap["logits"])
    for token in generated[: oracle_steps - 1]:
        gpu_logits.append(ctx.collect(ctx.enqueue_decode(token, logits=True))["logits"])
    gpu_logits = np.stack(gpu_logits)
    del ctx, model

    k, v = snapshot_kv(snap["kv"], plan, context)
    ospec = oracle_spec(max_context)
    # Layer 0's rows depend on the prompt alone: within 1 bf16 ulp of the oracle's in at least
    # 99.9% of elements, and every element within 2 ulps at the scale of its terms (scaled_ulps: a
    # dot product or a rotation that cancels far below its terms rounds differently in another
    # summation order).
    k0, v0 = first_layer_kv(prompt, weights, ospec)
    for name, got, want in (("K", k[0], k0), ("V", v[0], v0)):
        ulps, scaled = bf16_ulps(got, want), scaled_ulps(got, want, rotated=name == "K")
        print(f"ctx {context} layer 0 {name}: equal {float((ulps == 0).mean()):.5f}, within 1 ulp "
              f"{float((ulps <= 1).mean()):.5f}, max {int(ulps.max())} ulp, max {scaled.max():.2f} ulp of its terms' "
              f"scale ({int((scaled > 1).sum())} elements beyond 1)", flush=True)
        assert float((ulps <= 1).mean()) >= 0.999 and scaled.max() <= 2, name

    seeded = context - 1  # positions before the last prompt token
    cache = ref.StackCache.empty(ospec, torch.bfloat16)
    for layer, c in enumerate(cache.layers):
        c.k[:seeded] = torch.from_numpy(k[layer, :seeded]).to(torch.bfloat16)
        c.v[:seeded] = torch.from_numpy(v[layer, :seeded]).to(torch.bfloat16)
        c.position = seeded
    contract = C64.Contract(weights, ospec)
    contract.k[:, :seeded] = k[:, :seeded]
    contract.v[:, :seeded] = v[:, :seeded]
    contract.position = seeded
    forced = [prompt[-1]] + generated[: oracle_steps - 1]
    oracle_logits, oracle_tokens, exact_logits = [], [], []
    with torch.inference_mode():
        for step, token in enumerate(forced):
            out = ref.decode_token(token, weights, ospec, cache)["logits"].float()
            oracle_logits.append(out.numpy())
            oracle_tokens.append(ref.greedy(out))
            if step < exact_steps:
                exact_logits.append(contract.decode_token(token)["logits"])
    oracle_logits, exact_logits = np.stack(oracle_logits), np.stack(exact_logits)
    # The last prompt token's own K/V rows, computed by the worker and by the oracle from the same
    # cache (layer 0 from the same inputs: within the layer-0 bar).
    assert scaled_ulps(k[0, seeded], cache.layers[0].k[seeded].float().numpy(), rotated=True).max() <= 2

    drift = np.abs(exact_logits - oracle_logits[:exact_steps])
    bound = C64.calibrated_bound(float(drift.max()))
    errors = np.abs(gpu_logits - oracle_logits)
    to_exact = np.abs(gpu_logits[:exact_steps] - exact_logits)
    compared = 0
    for step in range(oracle_steps):
        top2 = np.sort(oracle_logits[step])[-2:]
        if top2[1] - top2[0] > bound:
            assert generated[step] == oracle_tokens[step], step
            compared += 1
    rms = lambda a: float(np.sqrt((a.astype(np.float64) ** 2).mean()))  # noqa: E731
    print(f"ctx {context}: worker-oracle max {errors.max():.4f} RMS {rms(errors):.5f} over {oracle_steps} steps "
          f"(bound {bound}); drift oracle-exact max {drift.max():.4f} RMS {rms(drift):.5f}; worker-exact max "
          f"{to_exact.max():.4f} RMS {rms(to_exact):.5f}, within 2e-2 of exact {float((to_exact <= 2e-2).mean()):.4f} "
          f"over {exact_steps} steps; tokens compared {compared}/{oracle_steps}", flush=True)
    assert errors.max() <= bound
    assert rms(errors) <= 2 * rms(drift) + 1e-4
    assert to_exact.max() <= drift.max() and rms(to_exact) <= rms(drift)


@pytest.mark.timeout(900)
def test_config4_ctx4096_full_depth(tmp_path, llama_weights):
    """Config 4: a 4,096-token prompt (seed 4096, the benchmark's), 130-step attention chunks (32 per
    K/V head at this context, the benchmark's package); all 64 generated steps against the oracle,
    the first 16 against the exact contract."""
    check_config(tmp_path, llama_weights, 4096, 130, 4096, oracle_steps=NEW_TOKENS, exact_steps=16)


@pytest.mark.timeout(900)
def test_config5_ctx32768_full_depth(tmp_path, llama_weights):
    """Config 5: a 32,768-token prompt (seed 32768), 1026-step chunks (32 per K/V head); the
    generated tokens of the 64-step launch, with the first 8 steps' logits against the oracle and
    4 against the exact contract (each oracle step attends over 32K positions in 16 layers on the
    CPU; the exact contract's float64 evaluation is the slower)."""
    check_config(tmp_path, llama_weights, 32768, 1026, 32768, oracle_steps=8, exact_steps=4)
