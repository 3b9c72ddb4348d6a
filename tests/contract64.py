"""The bf16 numerical contract evaluated exactly — TEST INFRASTRUCTURE ONLY.

A float64 NumPy restatement of the decoder's bf16 policy ``hf-llama-eager-bf16-v1``
(tileplan/src/tileplan/plan_core.py:76-90, docs/architecture.md:284-312 of the reference): every
value the policy rounds to bf16 is computed in float64 from bf16 operands and rounded once, to
nearest even, directly to bf16.  The rounding points are

* RMSNorm: bf16(bf16(x * rsqrt(mean(x^2) + eps)) * w)        (decoder_reference.py:183-187)
* Q, K, V, gate, up, the LM head: bf16(W u)                    (decoder_reference.py:224-226)
* RoPE: angle = float32(pos * freq); c, s = bf16(cos), bf16(sin);
  out1 = bf16(bf16(a c) - bf16(b s)), out2 = bf16(bf16(b c) + bf16(a s))   (:159-171)
* scores: bf16(bf16(q . k) * head_dim^-1/2); P = bf16(exp(s - M) / S)     (:240-246)
* attention: bf16(sum_t P_t V_t); r = bf16(x + bf16(Wo a))                 (:246-249)
* SwiGLU: bf16(bf16(silu(g)) * u); down: bf16(Wd p); y = bf16(r + down)    (:250-253)

Two uses: (1) it pins the oracle's bf16 path at ulp level on the reference's m1/m4 shapes
(tests/test_oracle.py), where the FP32 internals of PyTorch and exact arithmetic should agree
on all but a handful of roundings; (2) it is a second valid evaluation of the same contract, so
the spread between it and the oracle measures how far two correct implementations drift apart
through last-bit FP32 differences.  The bf16 GPU tests bound the worker's error by that spread
with the reference's own calibration rule (tileinfer/tests/bf16_checkpoint_tolerances.json:
atol = max(floor, 1.25 x the largest spread)).
"""

from __future__ import annotations

import numpy as np
import torch

from oracle import decoder as ref


def bf16(x) -> np.ndarray:
    """Round float64 values to the nearest bf16 (ties to even), exactly: 8 significant bits,
    the float32 exponent range (subnormal spacing 2^-133)."""
    x = np.asarray(x, dtype=np.float64)
    mantissa, exponent = np.frexp(x)  # x = mantissa * 2^exponent, |mantissa| in [0.5, 1)
    exponent = np.maximum(exponent, -125)  # below the smallest normal the spacing stays 2^-133
    scale = np.ldexp(1.0, 8 - exponent)
    return np.rint(x * scale) / scale


def as64(t: torch.Tensor) -> np.ndarray:
    return t.detach().to(torch.float64).numpy()


class Contract:
    """A stack's weights (bf16 values held in float64) and the contract's exact evaluation."""

    def __init__(self, weights: dict, spec: ref.Spec):
        self.spec = spec
        self.w = {k: as64(v) for k, v in weights.items()}
        self.freq = ref.rope_inverse_frequencies(spec).numpy().astype(np.float32)
        shape = (spec.layers, spec.max_context, spec.num_key_value_heads, spec.head_dim)
        self.k = np.zeros(shape)
        self.v = np.zeros(shape)
        self.position = 0

    def layer(self, index: int) -> dict:
        return {name: self.w[f"L{index}.{name}"] for name in ref.WEIGHTS}

    def rms_norm(self, x: np.ndarray, scale: np.ndarray) -> np.ndarray:
        inv = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + self.spec.rms_norm_eps)
        return bf16(bf16(x * inv) * scale)

    def rope(self, values: np.ndarray, positions: np.ndarray) -> np.ndarray:
        """values [..., heads, head_dim] at positions [...]."""
        angles = (np.asarray(positions, dtype=np.float32)[..., None] * self.freq).astype(np.float64)
        c = bf16(np.cos(angles))[..., None, :]
        s = bf16(np.sin(angles))[..., None, :]
        half = values.shape[-1] // 2
        a, b = values[..., :half], values[..., half:]
        return np.concatenate((bf16(bf16(a * c) - bf16(b * s)), bf16(bf16(b * c) + bf16(a * s))), axis=-1)

    def qkv(self, x: np.ndarray, w: dict, positions):
        """Rows of x [..., hidden] at positions [...]: rotated q, rotated k, v."""
        sp = self.spec
        u = self.rms_norm(x, w["attn_norm"])
        q = bf16(u @ w["Wq"].T).reshape(*x.shape[:-1], sp.num_attention_heads, sp.head_dim)
        k = bf16(u @ w["Wk"].T).reshape(*x.shape[:-1], sp.num_key_value_heads, sp.head_dim)
        v = bf16(u @ w["Wv"].T).reshape(*x.shape[:-1], sp.num_key_value_heads, sp.head_dim)
        return self.rope(q, positions), self.rope(k, positions), v

    def prefill_first_layer(self, tokens: list[int]) -> None:
        """Layer 0's K/V rows of a prompt, batched (a one-layer stack's whole cache)."""
        p0 = self.position
        positions = np.arange(p0, p0 + len(tokens))
        _, k, v = self.qkv(self.w["embedding"][tokens], self.layer(0), positions)
        self.k[0, positions] = k
        self.v[0, positions] = v
        self.position = p0 + len(tokens)

    def block(self, x: np.ndarray, index: int, p: int) -> dict:
        sp = self.spec
        w = self.layer(index)
        q, k, v = self.qkv(x, w, p)
        self.k[index, p] = k
        self.v[index, p] = v
        group = sp.num_attention_heads // sp.num_key_value_heads
        grouped = q.reshape(sp.num_key_value_heads, group, sp.head_dim)            # [kv, g, dh]
        keys = self.k[index, : p + 1].transpose(1, 2, 0)                           # [kv, dh, t]
        values = self.v[index, : p + 1].transpose(1, 0, 2)                         # [kv, t, dh]
        scores = bf16(bf16(grouped @ keys) * sp.head_dim ** -0.5)                  # [kv, g, t]
        e = np.exp(scores - scores.max(axis=-1, keepdims=True))
        probabilities = bf16(e / e.sum(axis=-1, keepdims=True))
        attention = bf16(probabilities @ values).reshape(-1)
        r = bf16(x + bf16(w["Wo"] @ attention))
        z = self.rms_norm(r, w["ffn_norm"])
        g = bf16(w["Wgate"] @ z)
        product = bf16(bf16(g / (1.0 + np.exp(-g))) * bf16(w["Wup"] @ z))
        ffn = bf16(w["Wdown"] @ product)
        return {"q": q, "k": k, "v": v, "attention": attention, "attn_residual": r, "ffn": ffn,
                "y": bf16(r + ffn), "product": product}

    def decode_token(self, token: int, keep_blocks: bool = False) -> dict:
        sp = self.spec
        hidden = self.w["embedding"][token]
        p = self.position
        blocks = []
        for index in range(sp.layers):
            trace = self.block(hidden, index, p)
            hidden = trace["y"]
            if keep_blocks:
                blocks.append(trace)
        self.position = p + 1
        final = self.rms_norm(hidden, self.w["final_norm"])
        head = self.w["embedding"] if sp.tie_word_embeddings else self.w["lm_head"]
        return {"blocks": blocks, "final_hidden": final, "logits": bf16(head @ final)}


def calibrated_bound(spread: float, floor: float = 2e-2) -> float:
    """The reference's calibration rule for a bf16 comparison (bf16_checkpoint_tolerances.json):
    the larger of the floor and 1.25 x the spread between two valid evaluations, rounded up to
    0.01."""
    return max(floor, float(np.ceil(1.25 * spread * 100.0) / 100.0))
