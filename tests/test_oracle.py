"""Pins the CPU oracle (oracle/decoder.py) before it is trusted as the GPU's checker.

* fp32 block and stack semantics: the reference's frozen fixtures
  tileplan/tests/fixtures/decoder_m1 and decoder_m4 (copied as data into tests/golden/),
  at their stated tolerance (model.json: atol = rtol = 2e-5).
* self-consistency: incremental decode equals full causal recomputation, as the
  reference's own test_decoder_reference.py:66-76 and test_decoder_stack.py:53-73 check.
* RoPE frequencies: a float64 closed form of the Llama-3 scaling rule
  (decoder_reference.py:139-156, plan.cpp:406-420) covering all three branches.
* bf16 rounding points (docs/architecture.md:284-312): restated with an independent
  numpy round-to-nearest-even, so a dropped or misplaced rounding fails.
"""

import json
import math
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import decoder as ref

GOLDEN = Path(__file__).parent / "golden"


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round float32 values to the nearest bfloat16 (ties to even), returned as float32."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    bits = (bits + 0x7FFF + ((bits >> 16) & 1)) & 0xFFFF0000
    return bits.astype(np.uint32).view(np.float32)


def load_spec(name: str) -> tuple[ref.Spec, dict]:
    model = json.loads((GOLDEN / name / "model.json").read_text())
    spec = ref.Spec.from_dict(model)
    if "layers" not in model:
        spec = ref.Spec.from_dict({**model, "layers": 1, "vocab_size": 0})
    return spec, model


def load_npz(path: Path) -> dict:
    with np.load(path, allow_pickle=False) as data:
        return {name: torch.from_numpy(data[name].copy()) for name in data.files}


def test_m1_block_matches_frozen_fixture():
    spec, model = load_spec("decoder_m1")
    weights = load_npz(GOLDEN / "decoder_m1" / "weights.npz")
    cases = load_npz(GOLDEN / "decoder_m1" / "reference_cases.npz")
    cache = ref.Cache.empty(spec, torch.float32)
    with torch.inference_mode():
        for step, x in enumerate(cases["x"]):
            out = ref.decode_one(x, weights, spec, cache)
            for name, key in [("q", "q"), ("k", "k"), ("v", "v"), ("attention", "attention"),
                              ("attn_residual", "attn_residual"), ("ffn", "ffn"), ("y", "y")]:
                torch.testing.assert_close(out[name], cases[key][step], atol=model["atol"], rtol=model["rtol"])
    torch.testing.assert_close(cache.k, cases["k_cache"][0], atol=model["atol"], rtol=model["rtol"])
    torch.testing.assert_close(cache.v, cases["v_cache"][0], atol=model["atol"], rtol=model["rtol"])


def test_m1_incremental_equals_full_prefix():
    spec, model = load_spec("decoder_m1")
    weights = load_npz(GOLDEN / "decoder_m1" / "weights.npz")
    tokens = load_npz(GOLDEN / "decoder_m1" / "reference_cases.npz")["x"]
    cache = ref.Cache.empty(spec, torch.float32)
    with torch.inference_mode():
        steps = [ref.decode_one(x, weights, spec, cache) for x in tokens]
        full = ref.recompute_prefix(tokens, weights, spec)
    for name in ("attention", "attn_residual", "ffn", "y"):
        torch.testing.assert_close(torch.stack([s[name] for s in steps]), full[name], atol=2e-5, rtol=2e-5)


def test_m4_stack_logits_and_cache_match_frozen_fixture():
    spec, model = load_spec("decoder_m4")
    weights = load_npz(GOLDEN / "decoder_m4" / "weights.npz")
    cases = load_npz(GOLDEN / "decoder_m4" / "reference_cases.npz")
    cache = ref.StackCache.empty(spec, torch.float32)
    with torch.inference_mode():
        for step, token in enumerate(cases["token_ids"].tolist()):
            logits = ref.decode_token(token, weights, spec, cache)["logits"]
            torch.testing.assert_close(logits, cases["logits"][step], atol=model["atol"], rtol=model["rtol"])
            full = ref.recompute_stack_prefix(cases["token_ids"][: step + 1].tolist(), weights, spec)
            torch.testing.assert_close(logits, full[-1], atol=2e-5, rtol=2e-5)
    for layer in range(spec.layers):
        torch.testing.assert_close(cache.layers[layer].k, cases["k_cache"][layer][0], atol=2e-5, rtol=2e-5)
        torch.testing.assert_close(cache.layers[layer].v, cases["v_cache"][layer][0], atol=2e-5, rtol=2e-5)


def test_m4_rejects_out_of_vocabulary_token():
    spec, _ = load_spec("decoder_m4")
    weights = load_npz(GOLDEN / "decoder_m4" / "weights.npz")
    with pytest.raises(ValueError, match="outside vocabulary"):
        ref.decode_token(spec.vocab_size, weights, spec, ref.StackCache.empty(spec, torch.float32))


def closed_form_frequencies(spec: ref.Spec) -> np.ndarray:
    """Llama-3 frequency scaling in float64, written from the published rule."""
    out = []
    for i in range(spec.head_dim // 2):
        inv = 1.0 / spec.rope_theta ** (2.0 * i / spec.head_dim)
        wavelength = 2.0 * math.pi / inv
        low = spec.rope_original_max_position_embeddings / spec.rope_low_freq_factor
        high = spec.rope_original_max_position_embeddings / spec.rope_high_freq_factor
        if wavelength < high:
            out.append(inv)
        elif wavelength > low:
            out.append(inv / spec.rope_factor)
        else:
            s = (spec.rope_original_max_position_embeddings / wavelength - spec.rope_low_freq_factor) / (
                spec.rope_high_freq_factor - spec.rope_low_freq_factor)
            out.append((1 - s) * inv / spec.rope_factor + s * inv)
    return np.array(out)


@pytest.mark.parametrize("spec", [load_spec("decoder_m1")[0], ref.LLAMA32_1B])
def test_rope_frequencies_closed_form(spec):
    got = ref.rope_inverse_frequencies(spec).double().numpy()
    want = closed_form_frequencies(spec)
    np.testing.assert_allclose(got, want, rtol=2e-6)
    # all three branches are exercised
    inv = 1.0 / spec.rope_theta ** (2.0 * np.arange(spec.head_dim // 2) / spec.head_dim)
    wl = 2 * math.pi / inv
    assert (wl < 2048).any() and (wl > 8192).any() and ((wl >= 2048) & (wl <= 8192)).any()


def test_bf16_rms_norm_rounds_before_scale():
    g = torch.Generator().manual_seed(251)
    x = torch.randn(4096, generator=g).to(torch.bfloat16)
    w = (1 + 0.05 * torch.randn(4096, generator=g)).to(torch.bfloat16)
    got = ref.rms_norm(x, w, 1e-5).float().numpy()
    xf = x.float().numpy().astype(np.float64)
    inv = 1.0 / np.sqrt(np.mean(xf * xf) + 1e-5)
    normalized = bf16_round((xf * inv).astype(np.float32))
    want = bf16_round((normalized.astype(np.float64) * w.float().numpy()).astype(np.float32))
    # the statistic differs from float64 in the last float32 bits only
    assert np.mean(got == want) > 0.99
    fused = bf16_round((xf * inv * w.float().numpy()).astype(np.float32))
    assert np.sum(got != fused) >= 500  # a fused (unrounded) norm is distinguishable


def test_bf16_rope_rounding_points():
    spec = ref.LLAMA32_1B
    g = torch.Generator().manual_seed(7)
    q = torch.randn(32, 64, generator=g).to(torch.bfloat16)
    pos = 3001
    got = ref.apply_rope(q, torch.tensor(pos, dtype=torch.float32), spec).float().numpy()
    freqs = ref.rope_inverse_frequencies(spec).numpy()
    angle = (np.float32(pos) * freqs).astype(np.float32)
    c = bf16_round(np.cos(angle.astype(np.float64)).astype(np.float32))
    s = bf16_round(np.sin(angle.astype(np.float64)).astype(np.float32))
    a, b = q.float().numpy()[:, :32], q.float().numpy()[:, 32:]
    first = bf16_round((bf16_round(a * c) - bf16_round(b * s)).astype(np.float32))
    second = bf16_round((bf16_round(b * c) + bf16_round(a * s)).astype(np.float32))
    want = np.concatenate([first, second], axis=1)
    # cos/sin of float32 angles may differ in the last ulp between libm versions
    assert np.mean(got == want) > 0.995
    np.testing.assert_allclose(got, want, atol=2 ** -6)


def test_bf16_projection_and_residual_rounding():
    g = torch.Generator().manual_seed(11)
    w = (0.02 * torch.randn(64, 2048, generator=g)).to(torch.bfloat16)
    u = torch.randn(2048, generator=g).to(torch.bfloat16)
    x = torch.randn(64, generator=g).to(torch.bfloat16)
    got = (x + w @ u).float().numpy()
    dot = w.double().numpy() @ u.double().numpy()
    want = bf16_round((bf16_round(dot.astype(np.float32)).astype(np.float64) + x.double().numpy()).astype(np.float32))
    assert np.mean(got == want) > 0.95
    np.testing.assert_allclose(got, want, atol=2 ** -6, rtol=2 ** -7)


def test_greedy_lowest_index_tie():
    logits = torch.tensor([0.5, 2.0, 2.0, -1.0])
    assert ref.greedy(logits) == 1
    assert ref.greedy(torch.zeros(48)) == 0


# ---- the oracle's bf16 path against the contract evaluated exactly (tests/contract64.py) ----

from tests import contract64 as C64  # noqa: E402


def test_exact_bf16_rounding_routine():
    """contract64.bf16 rounds float64 directly to bf16: equal to the float32 routine on float32
    values (ties to even, signs, subnormals), and free of double rounding."""
    rng = np.random.default_rng(3)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32) * 10.0 ** rng.integers(-40, 30, 10000),
                        np.array([1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, -(1.0 + 2.0 ** -8), 2.0 ** -130, 0.0],
                                 dtype=np.float32)]).astype(np.float32)
    assert np.array_equal(C64.bf16(x.astype(np.float64)), bf16_round(x).astype(np.float64))
    # 1 + 2^-8 + 2^-30 lies above the tie: exact rounding goes up, float32 first would tie to even
    assert C64.bf16(1.0 + 2.0 ** -8 + 2.0 ** -30) == 1.0 + 2.0 ** -7
    assert C64.bf16(1.0 + 2.0 ** -8) == 1.0


def ulp_distance(got: np.ndarray, want: np.ndarray) -> np.ndarray:
    """|got - want| in bf16 spacings of |want| (spacing 2^-133 at zero)."""
    _, exponent = np.frexp(want)
    return np.abs(got - want) / np.ldexp(1.0, np.maximum(exponent, -125) - 8)


def bf16_weights(weights: dict) -> dict:
    return {k: v.to(torch.bfloat16) for k, v in weights.items()}


FIELDS = ("q", "k", "v", "attention", "attn_residual", "ffn", "y")


def compare_block(out: dict, exact: dict, counts: dict) -> None:
    for name in FIELDS:
        got = out[name].double().numpy().reshape(-1)
        want = exact[name].reshape(-1)
        distance = ulp_distance(got, want)
        counts.setdefault(name, []).append(distance)


def test_m1_bf16_block_within_one_ulp_of_exact_contract():
    """The oracle's bf16 decode_one at the m1 shape (every fixture input, split attention over up
    to six positions) against the exact contract: every intermediate within one bf16 spacing, and
    at least 97% of elements identical."""
    spec, _ = load_spec("decoder_m1")
    weights = bf16_weights(load_npz(GOLDEN / "decoder_m1" / "weights.npz"))
    cases = load_npz(GOLDEN / "decoder_m1" / "reference_cases.npz")
    cache = ref.Cache.empty(spec, torch.bfloat16)
    contract = C64.Contract({f"L0.{k}": v for k, v in weights.items()}, spec)
    counts: dict = {}
    with torch.inference_mode():
        for step, x in enumerate(cases["x"].to(torch.bfloat16)):
            out = ref.decode_one(x, weights, spec, cache)
            exact = contract.block(C64.as64(x), 0, step)
            compare_block(out, exact, counts)
    for name, distances in counts.items():
        d = np.concatenate(distances)
        assert d.max() <= 1.0, (name, d.max())
        assert (d == 0).mean() >= 0.97, (name, (d == 0).mean())


def test_m4_bf16_stack_within_one_ulp_of_exact_contract():
    spec, _ = load_spec("decoder_m4")
    weights = bf16_weights(load_npz(GOLDEN / "decoder_m4" / "weights.npz"))
    cases = load_npz(GOLDEN / "decoder_m4" / "reference_cases.npz")
    cache = ref.StackCache.empty(spec, torch.bfloat16)
    contract = C64.Contract(weights, spec)
    logits, counts = [], {}
    with torch.inference_mode():
        for token in cases["token_ids"].tolist():
            out = ref.decode_token(token, weights, spec, cache, keep_blocks=True)
            exact = contract.decode_token(token, keep_blocks=True)
            for block, exact_block in zip(out["blocks"], exact["blocks"]):
                compare_block(block, exact_block, counts)
            logits.append(ulp_distance(out["logits"].double().numpy(), exact["logits"]))
    for name, distances in [*counts.items(), ("logits", logits)]:
        d = np.concatenate(distances)
        assert d.max() <= 1.0, (name, d.max())
        assert (d == 0).mean() >= 0.97, (name, (d == 0).mean())


def test_exact_contract_detects_a_dropped_rounding(monkeypatch):
    """The comparison above has teeth: the contract with the attention probabilities left
    unrounded (a plausible slip) drifts beyond one spacing from the oracle."""
    spec, _ = load_spec("decoder_m4")
    weights = bf16_weights(load_npz(GOLDEN / "decoder_m4" / "weights.npz"))
    cases = load_npz(GOLDEN / "decoder_m4" / "reference_cases.npz")
    cache = ref.StackCache.empty(spec, torch.bfloat16)
    contract = C64.Contract(weights, spec)
    original = C64.bf16
    calls = {"n": 0}

    def skip_probability_rounding(x):
        calls["n"] += 1
        values = np.asarray(x, dtype=np.float64)
        # the probabilities are the only rounded [kv_heads, group, t] values whose rows sum to ~1
        group = spec.num_attention_heads // spec.num_key_value_heads
        if values.ndim == 3 and values.shape[:2] == (spec.num_key_value_heads, group) and np.allclose(values.sum(-1), 1.0):
            return values
        return original(x)

    monkeypatch.setattr(C64, "bf16", skip_probability_rounding)
    worst = 0.0
    with torch.inference_mode():
        for token in cases["token_ids"].tolist():
            out = ref.decode_token(token, weights, spec, cache, keep_blocks=True)
            exact = contract.decode_token(token, keep_blocks=True)
            worst = max(worst, float(ulp_distance(out["logits"].double().numpy(), exact["logits"]).max()))
    assert calls["n"] > 0 and worst > 1.0
