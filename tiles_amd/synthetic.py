"""Synthetic Llama-3.2-1B workloads shared by the benchmark and the GPU tests.

Random-init weights N(0, 0.02) from a seed with norm weights 1.0, packed
into a v10 package for the live target, plus seeded uniform prompts.
"""

from __future__ import annotations

import tempfile
from pathlib import Path

import numpy as np
import torch

from .tileplan import package as K
from .tileplan import plan as P
from .tileplan import probe

BOS = 128000


def prompt(length: int, seed: int, vocab: int = 128256) -> list[int]:
    """A prompt drawn uniformly from the vocabulary with the seed."""
    return np.random.default_rng(seed).integers(0, vocab, size=length).tolist()


def llama_package(out: Path, max_context: int, dtype: str = "bfloat16", seed: int = 0, chunk_steps: int | None = None,
                  target: dict | None = None, weights: dict | None = None) -> tuple[P.StackSpec, dict]:
    """Writes a random-init Llama-3.2-1B package; returns the spec and the weights as packed."""
    spec = P.llama32_1b(max_context)
    weights = weights if weights is not None else K.random_weights(spec, seed=seed)
    target = target if target is not None else probe.probe_library()
    K.build_stack_package(spec, weights, target, Path(out), dtype, chunk_steps=chunk_steps)
    return spec, weights


def scratch_dir() -> Path:
    return Path(tempfile.mkdtemp(prefix="tiles_amd_", dir="/tmp"))
