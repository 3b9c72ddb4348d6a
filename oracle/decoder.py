"""CPU oracle for the TileInfer decode path — TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker (or the timed CPU baseline);
the product path in ``tiles_amd`` never calls it.

It restates, in PyTorch eager on the CPU, the reference's own decoder oracle:

* ``rope_inverse_frequencies``  follows tileplan/src/tileplan/decoder_reference.py:139-156
* ``apply_rope``                follows decoder_reference.py:159-171
* ``rms_norm``                  follows decoder_reference.py:183-187
* ``decode_one``                follows decoder_reference.py:213-270
* ``append_kv``                 decode_one's K/V rows alone (decoder_reference.py:223-237)
* ``recompute_prefix``          follows decoder_reference.py:273-312
* ``final_norm``                follows tileplan/src/tileplan/decoder_stack.py:126-132
* ``decode_token``              follows decoder_stack.py:135-155
* ``recompute_stack_prefix``    follows decoder_stack.py:158-173

PyTorch is the reference's arithmetic library (pinned there at 2.14.1); this
container runs 2.10 on the CPU.  fp32 results are pinned by the reference's frozen
fixtures ``decoder_m1`` / ``decoder_m4`` (tests/test_oracle.py).  bf16 results are
pinned by the bf16 contract evaluated exactly in float64 (tests/contract64.py): at the
m1/m4 shapes the oracle's logits are within 1 bf16 ulp of it (tests/test_oracle.py).
No bf16 golden exists in the reference.  At Llama-1B widths PyTorch's CPU bf16 matmuls
drift further from the exact contract, so the GPU tests there compare against the
exact contract and use the oracle for the drift that calibrates their bounds.
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F

WEIGHTS = ("attn_norm", "Wq", "Wk", "Wv", "Wo", "ffn_norm", "Wgate", "Wup", "Wdown")


@dataclass(frozen=True)
class Spec:
    """Model dimensions; field names follow decoder_reference.py:18-37 / decoder_stack.py:49-54."""

    hidden_size: int = 32
    intermediate_size: int = 64
    num_attention_heads: int = 4
    num_key_value_heads: int = 2
    head_dim: int = 8
    max_context: int = 6
    rms_norm_eps: float = 1e-5
    rope_theta: float = 500000.0
    rope_factor: float = 32.0
    rope_low_freq_factor: float = 1.0
    rope_high_freq_factor: float = 4.0
    rope_original_max_position_embeddings: int = 8192
    layers: int = 1
    vocab_size: int = 0
    tie_word_embeddings: bool = True

    @property
    def head_to_kv(self) -> list[int]:
        group = self.num_attention_heads // self.num_key_value_heads
        return [head // group for head in range(self.num_attention_heads)]

    @classmethod
    def from_dict(cls, source: dict) -> "Spec":
        names = {f for f in cls.__dataclass_fields__}
        return cls(**{k: v for k, v in source.items() if k in names})


LLAMA32_1B = Spec(
    hidden_size=2048,
    intermediate_size=8192,
    num_attention_heads=32,
    num_key_value_heads=8,
    head_dim=64,
    max_context=4096,
    layers=16,
    vocab_size=128256,
)


def rope_inverse_frequencies(spec: Spec) -> torch.Tensor:
    """Llama-3 scaled inverse frequencies (decoder_reference.py:139-156)."""
    indices = torch.arange(0, spec.head_dim, 2, dtype=torch.float32)
    inv = 1.0 / (spec.rope_theta ** (indices / spec.head_dim))
    wavelength = 2 * math.pi / inv
    low = spec.rope_original_max_position_embeddings / spec.rope_low_freq_factor
    high = spec.rope_original_max_position_embeddings / spec.rope_high_freq_factor
    smooth = (spec.rope_original_max_position_embeddings / wavelength - spec.rope_low_freq_factor) / (
        spec.rope_high_freq_factor - spec.rope_low_freq_factor
    )
    scaled = torch.where(wavelength > low, inv / spec.rope_factor, inv)
    medium = (wavelength >= high) & (wavelength <= low)
    blended = (1 - smooth) * scaled / spec.rope_factor + smooth * scaled
    return torch.where(medium, blended, scaled)


def apply_rope(values: torch.Tensor, positions: torch.Tensor, spec: Spec) -> torch.Tensor:
    """Split-half rotation; cos/sin rounded to the value dtype (decoder_reference.py:159-171)."""
    angles = positions.to(dtype=torch.float32).unsqueeze(-1) * rope_inverse_frequencies(spec)
    cosine = angles.cos().to(values.dtype).unsqueeze(-2)
    sine = angles.sin().to(values.dtype).unsqueeze(-2)
    first, second = values.chunk(2, dim=-1)
    return torch.cat((first * cosine - second * sine, second * cosine + first * sine), dim=-1)


def rms_norm(x: torch.Tensor, scale: torch.Tensor, eps: float) -> torch.Tensor:
    """FP32 statistic; the normalized value rounds to x.dtype before the scale (:183-187)."""
    normalized = x.float() * torch.rsqrt(x.float().square().mean(dim=-1, keepdim=True) + eps)
    return normalized.to(x.dtype) * scale


@dataclass
class Cache:
    """One layer's K/V cache, [max_context, kv_heads, head_dim] (decoder_reference.py:190-210)."""

    k: torch.Tensor
    v: torch.Tensor
    position: int = 0

    @classmethod
    def empty(cls, spec: Spec, dtype: torch.dtype) -> "Cache":
        shape = (spec.max_context, spec.num_key_value_heads, spec.head_dim)
        return cls(torch.zeros(shape, dtype=dtype), torch.zeros(shape, dtype=dtype))


@dataclass
class StackCache:
    layers: list[Cache] = field(default_factory=list)

    @classmethod
    def empty(cls, spec: Spec, dtype: torch.dtype) -> "StackCache":
        return cls([Cache.empty(spec, dtype) for _ in range(spec.layers)])

    @property
    def position(self) -> int:
        return self.layers[0].position


def _rotated_qkv(x: torch.Tensor, w: dict, spec: Spec, p: int):
    """The block's normalized input projected to q, k, v, with q and k rotated for position p
    (decoder_reference.py:223-233)."""
    u = rms_norm(x, w["attn_norm"], spec.rms_norm_eps)
    q = (w["Wq"] @ u).reshape(spec.num_attention_heads, spec.head_dim)
    k = (w["Wk"] @ u).reshape(spec.num_key_value_heads, spec.head_dim)
    v = (w["Wv"] @ u).reshape(spec.num_key_value_heads, spec.head_dim)
    position = torch.tensor(p, dtype=torch.float32)
    return apply_rope(q, position, spec), apply_rope(k, position, spec), v


def append_kv(x: torch.Tensor, w: dict, spec: Spec, cache: Cache) -> None:
    """The K/V row decode_one appends for input x, without the rest of the block: the same
    operations, so the cache holds the same bits.  A one-layer stack's cache depends on the
    tokens alone, so this fills long prefixes of such stacks without their attention."""
    if cache.position >= spec.max_context:
        raise ValueError("context capacity reached")
    p = cache.position
    _, k, v = _rotated_qkv(x, w, spec, p)
    cache.k[p] = k
    cache.v[p] = v
    cache.position = p + 1


def decode_one(x: torch.Tensor, w: dict, spec: Spec, cache: Cache) -> dict:
    """Append one token to one block (decoder_reference.py:213-270)."""
    if cache.position >= spec.max_context:
        raise ValueError("context capacity reached")
    p = cache.position
    q, k, v = _rotated_qkv(x, w, spec, p)
    cache.k[p] = k
    cache.v[p] = v
    keys = cache.k[: p + 1, spec.head_to_kv]
    values = cache.v[: p + 1, spec.head_to_kv]
    raw = torch.einsum("hd,thd->ht", q, keys)
    scores = raw / math.sqrt(spec.head_dim) if x.dtype == torch.float32 else raw * (spec.head_dim**-0.5)
    probabilities = torch.softmax(scores, dim=-1, dtype=torch.float32).to(x.dtype)
    attention = torch.einsum("ht,thd->hd", probabilities, values).reshape(spec.hidden_size)
    r = x + w["Wo"] @ attention
    z = rms_norm(r, w["ffn_norm"], spec.rms_norm_eps)
    ffn = w["Wdown"] @ (F.silu(w["Wgate"] @ z) * (w["Wup"] @ z))
    y = r + ffn
    cache.position = p + 1
    return {"q": q, "k": k, "v": v, "attention": attention, "attn_residual": r, "ffn": ffn, "y": y}


def recompute_prefix(tokens: torch.Tensor, w: dict, spec: Spec) -> dict:
    """Full causal block over every visible position (decoder_reference.py:273-312)."""
    length = tokens.shape[0]
    u = rms_norm(tokens, w["attn_norm"], spec.rms_norm_eps)
    q = (u @ w["Wq"].T).reshape(length, spec.num_attention_heads, spec.head_dim)
    k = (u @ w["Wk"].T).reshape(length, spec.num_key_value_heads, spec.head_dim)
    v = (u @ w["Wv"].T).reshape(length, spec.num_key_value_heads, spec.head_dim)
    positions = torch.arange(length, dtype=torch.float32)
    q = apply_rope(q, positions, spec)
    k = apply_rope(k, positions, spec)
    keys = k[:, spec.head_to_kv]
    values = v[:, spec.head_to_kv]
    raw = torch.einsum("thd,shd->ths", q, keys)
    scores = raw / math.sqrt(spec.head_dim) if tokens.dtype == torch.float32 else raw * (spec.head_dim**-0.5)
    future = torch.triu(torch.ones((length, length), dtype=torch.bool), diagonal=1)
    scores = scores.masked_fill(future[:, None, :], -torch.inf)
    probabilities = torch.softmax(scores, dim=-1, dtype=torch.float32).to(tokens.dtype)
    attention = torch.einsum("ths,shd->thd", probabilities, values).reshape(length, spec.hidden_size)
    r = tokens + attention @ w["Wo"].T
    z = rms_norm(r, w["ffn_norm"], spec.rms_norm_eps)
    ffn = (F.silu(z @ w["Wgate"].T) * (z @ w["Wup"].T)) @ w["Wdown"].T
    return {"q": q, "k": k, "v": v, "attention": attention, "attn_residual": r, "ffn": ffn, "y": r + ffn}


def final_norm(hidden: torch.Tensor, scale: torch.Tensor, eps: float) -> torch.Tensor:
    """fp32: no intermediate rounding; bf16: ``rms_norm`` (decoder_stack.py:126-132)."""
    if hidden.dtype == torch.float32:
        return hidden * torch.rsqrt(hidden.square().mean(dim=-1, keepdim=True) + eps) * scale
    return rms_norm(hidden, scale, eps)


def layer_weights(weights: dict, layer: int) -> dict:
    return {name: weights[f"L{layer}.{name}"] for name in WEIGHTS}


def decode_token(token_id: int, weights: dict, spec: Spec, cache: StackCache, keep_blocks: bool = False) -> dict:
    """Embedding → blocks → final norm → tied/untied LM head (decoder_stack.py:135-155)."""
    if not 0 <= token_id < spec.vocab_size:
        raise ValueError("token ID outside vocabulary")
    hidden = weights["embedding"][token_id]
    blocks = []
    for layer in range(spec.layers):
        trace = decode_one(hidden, layer_weights(weights, layer), spec, cache.layers[layer])
        hidden = trace["y"]
        if keep_blocks:
            blocks.append(trace)
    final_hidden = final_norm(hidden, weights["final_norm"], spec.rms_norm_eps)
    projection = weights["embedding"] if spec.tie_word_embeddings else weights["lm_head"]
    logits = projection @ final_hidden
    return {"blocks": blocks, "final_hidden": final_hidden, "logits": logits}


def recompute_stack_prefix(token_ids: list[int], weights: dict, spec: Spec) -> torch.Tensor:
    """Logits of every visible position from full causal matrices (decoder_stack.py:158-173)."""
    hidden = weights["embedding"][token_ids]
    for layer in range(spec.layers):
        hidden = recompute_prefix(hidden, layer_weights(weights, layer), spec)["y"]
    final_hidden = final_norm(hidden, weights["final_norm"], spec.rms_norm_eps)
    projection = weights["embedding"] if spec.tie_word_embeddings else weights["lm_head"]
    return final_hidden @ projection.T


def greedy(logits: torch.Tensor) -> int:
    """Largest logit, lowest index among equals (ops.cuh:865-889 candidate rule; torch.argmax
    returns the first maximum)."""
    return int(torch.argmax(logits.float()).item())


def generate(prompt: list[int], new_tokens: int, weights: dict, spec: Spec, dtype: torch.dtype,
             cache: StackCache | None = None, forced: list[int] | None = None) -> dict:
    """Greedy generation the way the worker does it: the last prompt step's logits pick the
    first new token, which is then decoded, and so on (worker_kernel.cu:189-217).

    ``forced`` (teacher forcing) feeds those tokens instead of the oracle's own choice, so a
    caller can keep comparing per-step logits after a tie-broken divergence.
    Returns the chosen tokens and the logits each choice was made from.
    """
    cache = cache or StackCache.empty(spec, dtype)
    with torch.inference_mode():
        out = None
        for token in prompt:
            out = decode_token(token, weights, spec, cache)
        chosen, step_logits = [], []
        for step in range(new_tokens):
            logits = out["logits"].float()
            step_logits.append(logits)
            token = greedy(logits)
            chosen.append(token)
            fed = forced[step] if forced is not None else token
            out = decode_token(fed, weights, spec, cache)
        return {"tokens": chosen, "logits": step_logits, "cache": cache, "last": out}
