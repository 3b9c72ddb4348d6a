"""A host of the launch boundary alone — TEST INFRASTRUCTURE ONLY.

Drives ``ti_enqueue_worker`` (and ``ti_enqueue_worker_static``) the way a foreign host would
(INTEGRATION.md): the uploaded model's program view from ``ti_model_program_view``, every worker
buffer owned by the caller (PyTorch device tensors here), the exchange area zeroed once, and the
epoch advanced by exactly ``ti_epochs_per_launch`` from one launch to the next.  Buffer sizes come
from plan.json's storage section, as the reference's host takes them from LoadedPlan
(tileinfer/src/runtime/context_buffers.cuh:18-66).
"""

from __future__ import annotations

import ctypes as C

import numpy as np
import torch

from tiles_amd import runtime as R

MAX_STEPS = 64


def _ptr(t: torch.Tensor) -> int:
    return t.data_ptr()


class LaunchHost:
    def __init__(self, model: R.DecoderModel, plan: dict, static: bool = False):
        self.lib = R.library()
        self.view = model.program_view()
        self.static = static
        storage, m = plan["storage"], plan["model"]
        self.elem = 2 if m["weight_dtype"] == "bfloat16" else 4
        self.hidden, self.vocab = m["hidden_size"], m.get("vocab_size", 1)
        self.max_context = m["max_context"]
        self.layers = self.view.stack.layers
        dev = torch.device("cuda", 0)
        byte = lambda n: torch.zeros(max(int(n), 16), dtype=torch.uint8, device=dev)  # noqa: E731
        self.input = byte(self.hidden * self.elem)
        self.output = byte(self.hidden * self.elem)
        self.scratch = byte(storage["scratch_bytes"])
        self.kv = byte(storage["kv_bytes"])
        self.logits = torch.zeros(max(1, self.vocab), dtype=torch.float32, device=dev)
        self.scores = byte(storage["attention_bytes"])
        self.partials = byte(storage["attention_partial_bytes"] + storage["ffn_partial_bytes"])
        self.candidates = byte(8 * max(1, self.view.selection_slots))
        words = self.lib.ti_exchange_words(C.byref(self.view.shape), self.layers, self.view.selection_slots)
        self.exchange = torch.zeros(words, dtype=torch.int64, device=dev)  # zeroed once
        self.tokens = torch.zeros(self.max_context + MAX_STEPS, dtype=torch.int32, device=dev)
        self.generated = torch.full((self.max_context,), -1, dtype=torch.int32, device=dev)
        self.status = torch.zeros(3, dtype=torch.int32, device=dev)
        self.timeout = torch.zeros(1, dtype=torch.int32, device=dev)
        self.epoch = 1
        self.position = 0
        self.timeline = None  # optional device tensor of 64-bit words, timeline_fields per instruction
        self.timeline_fields = 0
        self.stream = torch.cuda.current_stream().cuda_stream

    def buffers(self) -> R.WorkerBuffers:
        b = R.WorkerBuffers()
        b.input, b.output, b.scratch, b.kv = map(_ptr, (self.input, self.output, self.scratch, self.kv))
        b.logits, b.attention_scores, b.attention_partials = map(_ptr, (self.logits, self.scores, self.partials))
        b.selection = _ptr(self.candidates)
        b.exchange = _ptr(self.exchange)
        b.epoch = self.epoch
        if self.timeline is not None:
            b.timeline = _ptr(self.timeline)
        b.timeline_fields = self.timeline_fields
        return b

    def _launch(self, steps: int, token: R.TokenInput, selection: R.Selection) -> None:
        b = self.buffers()
        if self.static:
            code = self.lib.ti_enqueue_worker_static(self.stream, C.byref(self.view), C.byref(b), self.position, token,
                                                     selection, _ptr(self.timeout))
        else:
            code = self.lib.ti_enqueue_worker(self.stream, C.byref(self.view), C.byref(b), self.position, token,
                                              selection)
        R._check(code)
        self.epoch += self.lib.ti_epochs_per_launch(self.layers)
        self.position += steps

    def feed(self, ids: list[int]) -> None:
        """Decodes host tokens (prefill or forced decode), 64 per launch."""
        self.tokens[: len(ids)] = torch.tensor(ids, dtype=torch.int32)
        for first in range(0, len(ids), MAX_STEPS):
            steps = min(MAX_STEPS, len(ids) - first)
            self._launch(steps, R.TokenInput(-1, _ptr(self.tokens) + 4 * first, steps), R.Selection())

    def generate(self, count: int, eos: int = -1) -> list[int]:
        """Greedy tokens, 64 steps per launch, selected on the device.  After an early stop the
        epoch follows the last launch that ran (ti_epoch_after_generation)."""
        self.status.zero_()
        self.generated.fill_(-1)
        start, epochs = self.position, []
        for first in range(0, count, MAX_STEPS):
            steps = min(MAX_STEPS, count - first)
            epochs.append(self.epoch)
            self._launch(steps, R.TokenInput(-1, None, steps), R.Selection(_ptr(self.generated), _ptr(self.status), first, eos))
        torch.cuda.synchronize()
        n = int(self.status[0].item())
        if not self.static:
            array = (C.c_uint32 * len(epochs))(*epochs)
            self.epoch = self.lib.ti_epoch_after_generation(self.epoch, array, len(epochs), n, self.layers)
        self.position = start + n
        return self.generated[:n].tolist()

    def kv_values(self) -> np.ndarray:
        torch.cuda.synchronize()
        raw = self.kv.cpu()
        if self.elem == 2:
            return raw.view(torch.bfloat16).float().numpy()
        return raw.view(torch.float32).numpy()

    def logits_values(self) -> np.ndarray:
        torch.cuda.synchronize()
        return self.logits.cpu().numpy().copy()
