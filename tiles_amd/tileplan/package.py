"""Package I/O, random-init Llama checkpoints and the checkpoint importer.

A package directory holds ``plan.json`` (canonical JSON), ``weights.bin`` (little-endian,
manifest order, 64-byte aligned regions, Wdown transposed, tied LM head aliasing the
embedding) and ``planning_report.json`` — the layout the reference writes
(plan_core.py:752-792, decoder_stack.py:314-340, llama32_import.py:211-331).
"""

from __future__ import annotations

import hashlib
import json
import mmap
import os
import shutil
import tempfile
from contextlib import contextmanager
from pathlib import Path

import numpy as np
import torch

from . import plan as P

# Hugging Face tensor names (llama32_import.py:22-32, 93-103).
HF_SUFFIXES = {
    "attn_norm": "input_layernorm.weight", "Wq": "self_attn.q_proj.weight",
    "Wk": "self_attn.k_proj.weight", "Wv": "self_attn.v_proj.weight",
    "Wo": "self_attn.o_proj.weight", "ffn_norm": "post_attention_layernorm.weight",
    "Wgate": "mlp.gate_proj.weight", "Wup": "mlp.up_proj.weight", "Wdown": "mlp.down_proj.weight",
}


def hf_names(spec: P.StackSpec) -> dict[str, str]:
    names = {"embedding": "model.embed_tokens.weight", "final_norm": "model.norm.weight"}
    for layer in range(spec.layers):
        for name in P.WEIGHTS:
            names[f"L{layer}.{name}"] = f"model.layers.{layer}.{HF_SUFFIXES[name]}"
    if not spec.tie_word_embeddings:
        names["lm_head"] = "lm_head.weight"
    return names


def weight_names(spec: P.StackSpec) -> list[str]:
    names = ["embedding"]
    for layer in range(spec.layers):
        names += [f"L{layer}.{n}" for n in P.WEIGHTS]
    names.append("final_norm")
    if not spec.tie_word_embeddings:
        names.append("lm_head")
    return names


def weight_shape(spec: P.StackSpec, name: str) -> tuple[int, ...]:
    if name in ("embedding", "lm_head"):
        return (spec.vocab_size, spec.block.hidden_size)
    if name == "final_norm":
        return (spec.block.hidden_size,)
    return P.source_shape(spec.block, name.split(".", 1)[1])


def random_weights(spec: P.StackSpec, seed: int = 0, std: float = 0.02,
                   dtype: torch.dtype = torch.bfloat16) -> dict[str, torch.Tensor]:
    """Random-init weights: matrices N(0, std) from one seeded generator in manifest order,
    norm weights 1.0, rounded once to ``dtype`` (the benchmark's synthetic Llama)."""
    generator = torch.Generator().manual_seed(seed)
    out = {}
    for name in weight_names(spec):
        shape = weight_shape(spec, name)
        if name.endswith("norm"):
            out[name] = torch.ones(shape, dtype=dtype)
        else:
            out[name] = (torch.randn(shape, generator=generator) * std).to(dtype)
    return out


def _pack(tensor: torch.Tensor, dtype: str) -> bytes:
    if dtype == "bfloat16":
        return tensor.to(torch.bfloat16).contiguous().view(torch.uint16).numpy().tobytes()
    return tensor.to(torch.float32).contiguous().numpy().astype("<f4").tobytes()


def pack_stack_weights(spec: P.StackSpec, weights: dict, dtype: str, out) -> None:
    """Write every weight at its stack offset into a writable buffer ``out``."""
    stack, total = P.stack_layout(spec, dtype)
    size = P.weight_size(dtype)
    entries, _ = P.regions(spec.block, P.WEIGHTS, 64, size)
    offsets = {P.TENSOR_NAMES[e["tensor"]]: e["offset"] for e in entries}

    def put(offset: int, tensor: torch.Tensor) -> None:
        raw = _pack(tensor, dtype)
        out[offset:offset + len(raw)] = raw

    put(0, weights["embedding"])
    for layer in range(spec.layers):
        base = stack["layer_weights_offset"] + layer * stack["layer_weight_stride"]
        for name in P.WEIGHTS:
            value = weights[f"L{layer}.{name}"]
            put(base + offsets[name], value.T if name == "Wdown" else value)
    put(stack["final_norm_offset"], weights["final_norm"])
    if not spec.tie_word_embeddings:
        put(stack["lm_head_offset"], weights["lm_head"])


@contextmanager
def new_package_dir(out: Path):
    """A scratch directory renamed to ``out`` only when the block completes."""
    if out.exists():
        raise FileExistsError(out)
    out.parent.mkdir(parents=True, exist_ok=True)
    temporary = Path(tempfile.mkdtemp(prefix=f".{out.name}-", dir=out.parent))
    try:
        yield temporary
        os.rename(temporary, out)
    except BaseException:
        shutil.rmtree(temporary, ignore_errors=True)
        raise


def summary(plan: dict, plan_sha256: str) -> dict:
    storage, model = plan["storage"], plan["model"]
    return {**P.numeric_policy(model["weight_dtype"]), "plan_sha256": plan_sha256,
            "weights_sha256": plan["integrity"]["weights_sha256"],
            "attention_bytes": storage["attention_bytes"], "layers": model["layers"],
            "vocab_size": model.get("vocab_size"), "max_context": model["max_context"],
            "attention_chunks": model["attention_chunks"],
            "attention_chunk_steps": model["attention_chunk_steps"],
            "attention_fused_steps": model["attention_fused_steps"],
            "task_count": len(plan["tasks"]), "wave_count": len(plan["waves"]),
            "weight_bytes": storage["weight_bytes"], "kv_bytes": storage["kv_bytes"]}


def build_stack_package(spec: P.StackSpec, weights: dict, target: dict, out: Path,
                        dtype: str = "bfloat16", chunk_steps: int | None = None,
                        fused_steps: int | None = None) -> dict:
    """Plan + pack a stack package; ``target`` is a probed target (schema 3)."""
    out = Path(out)
    plan_target = P.plan_target(target)
    _, total = P.stack_layout(spec, dtype)
    with new_package_dir(out) as directory:
        path = directory / "weights.bin"
        with path.open("w+b") as stream:
            stream.truncate(total)
            with mmap.mmap(stream.fileno(), 0) as mapping:
                pack_stack_weights(spec, weights, dtype, mapping)
                digest = hashlib.sha256(mapping).hexdigest()
                mapping.flush()
        plan = P.stack_plan(spec, plan_target, dtype, digest, chunk_steps, fused_steps)
        data = P.json_bytes(plan)
        (directory / "plan.json").write_bytes(data)
        report = summary(plan, hashlib.sha256(data).hexdigest())
        (directory / "planning_report.json").write_bytes(P.json_bytes(report))
    return report


def build_block_package(block: P.BlockSpec, weights: dict, target: dict, out: Path, dtype: str = "bfloat16",
                        chunk_steps: int | None = None, fused_steps: int | None = None) -> dict:
    """Plan + pack a single-layer block package (decoder_block.py:50-70): weights.bin holds the
    layer's weights (keys without a layer prefix, as decoder_m1's weights.npz) at their region
    offsets, Wdown transposed."""
    out = Path(out)
    size = P.weight_size(dtype)
    entries, total = P.regions(block, P.WEIGHTS, 64, size)
    raw = bytearray(total)
    for e in entries:
        name = P.TENSOR_NAMES[e["tensor"]]
        value = weights[name].T if name == "Wdown" else weights[name]
        data = _pack(value, dtype)
        raw[e["offset"]:e["offset"] + len(data)] = data
    with new_package_dir(out) as directory:
        (directory / "weights.bin").write_bytes(bytes(raw))
        plan = P.block_plan(block, P.plan_target(target), dtype, hashlib.sha256(raw).hexdigest(), chunk_steps, fused_steps)
        data = P.json_bytes(plan)
        (directory / "plan.json").write_bytes(data)
        report = summary(plan, hashlib.sha256(data).hexdigest())
        (directory / "planning_report.json").write_bytes(P.json_bytes(report))
    return report


def read_plan(package: Path) -> dict:
    return json.loads((Path(package) / "plan.json").read_text())


def hf_config(spec: P.StackSpec) -> dict:
    """A config.json the reference's importer accepts (llama32_import.py:35-75)."""
    b = spec.block
    return {"architectures": ["LlamaForCausalLM"], "model_type": "llama", "hidden_size": b.hidden_size,
            "intermediate_size": b.intermediate_size, "num_hidden_layers": spec.layers,
            "num_attention_heads": b.num_attention_heads, "num_key_value_heads": b.num_key_value_heads,
            "head_dim": b.head_dim, "vocab_size": spec.vocab_size, "rms_norm_eps": b.rms_norm_eps,
            "rope_theta": b.rope_theta, "max_position_embeddings": 131072, "hidden_act": "silu",
            "attention_bias": False, "attention_dropout": 0.0, "mlp_bias": False,
            "tie_word_embeddings": spec.tie_word_embeddings, "torch_dtype": "bfloat16",
            "rope_scaling": {"rope_type": "llama3", "factor": b.rope_factor,
                             "low_freq_factor": b.rope_low_freq_factor,
                             "high_freq_factor": b.rope_high_freq_factor,
                             "original_max_position_embeddings": b.rope_original_max_position_embeddings}}


def write_checkpoint(spec: P.StackSpec, weights: dict, out: Path) -> Path:
    """Save ``weights`` as one safetensors file with HF names, plus config.json."""
    from safetensors.torch import save_file

    out = Path(out)
    out.mkdir(parents=True, exist_ok=True)
    names = hf_names(spec)
    save_file({names[k]: v.contiguous() for k, v in weights.items()}, str(out / "model.safetensors"))
    (out / "config.json").write_text(json.dumps(hf_config(spec), indent=2) + "\n")
    return out


def read_checkpoint(checkpoint: Path, max_context: int) -> tuple[P.StackSpec, dict]:
    """Load a Llama checkpoint written with HF names; only the 1B architecture is accepted
    (llama32_import.py:35-90), with the context cap raised for the 32K configuration."""
    from safetensors.torch import load_file

    checkpoint = Path(checkpoint)
    config = json.loads((checkpoint / "config.json").read_text())
    spec = P.llama32_1b(max_context)
    expected = hf_config(spec)
    for key, value in expected.items():
        if key == "max_position_embeddings":
            continue
        P.require(config.get(key) == value, f"unsupported Llama config {key}")
    tensors = {}
    for path in sorted(checkpoint.glob("*.safetensors")):
        tensors.update(load_file(str(path)))
    names = hf_names(spec)
    weights = {}
    for internal, hf in names.items():
        P.require(hf in tensors, f"missing tensor {hf}")
        value = tensors[hf]
        P.require(tuple(value.shape) == weight_shape(spec, internal), f"invalid tensor shape {hf}")
        P.require(bool(torch.isfinite(value.float()).all()), f"non-finite tensor {hf}")
        weights[internal] = value
    return spec, weights


def import_checkpoint(checkpoint: Path, target: dict, out: Path, max_context: int = 4096,
                      dtype: str = "bfloat16", chunk_steps: int | None = None,
                      fused_steps: int | None = None) -> dict:
    spec, weights = read_checkpoint(checkpoint, max_context)
    return build_stack_package(spec, weights, target, out, dtype, chunk_steps, fused_steps)


def read_weights(package: Path, spec: P.StackSpec, dtype: str) -> dict[str, torch.Tensor]:
    """Unpack weights.bin into oracle-named tensors in source layout (Wdown back to [d, f])."""
    raw = np.memmap(Path(package) / "weights.bin", dtype=np.uint8, mode="r")
    stack, _ = P.stack_layout(spec, dtype)
    size = P.weight_size(dtype)
    entries, _ = P.regions(spec.block, P.WEIGHTS, 64, size)
    offsets = {P.TENSOR_NAMES[e["tensor"]]: e["offset"] for e in entries}

    def get(offset: int, shape: tuple[int, ...]) -> torch.Tensor:
        count = int(np.prod(shape))
        chunk = np.array(raw[offset:offset + count * size])
        if dtype == "bfloat16":
            return torch.from_numpy(chunk.view(np.int16).copy()).view(torch.bfloat16).reshape(shape)
        return torch.from_numpy(chunk.view("<f4").copy()).reshape(shape)

    out = {"embedding": get(0, weight_shape(spec, "embedding"))}
    for layer in range(spec.layers):
        base = stack["layer_weights_offset"] + layer * stack["layer_weight_stride"]
        for name in P.WEIGHTS:
            shape = P.tensor_shape(spec.block, name)
            value = get(base + offsets[name], shape)
            out[f"L{layer}.{name}"] = value.T.contiguous() if name == "Wdown" else value
    out["final_norm"] = get(stack["final_norm_offset"], (spec.block.hidden_size,))
    if not spec.tie_word_embeddings:
        out["lm_head"] = get(stack["lm_head_offset"], weight_shape(spec, "lm_head"))
    return out
