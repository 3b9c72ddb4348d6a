"""Python binding of the decode worker's C ABI (include/tileinfer_amd.h) through ctypes.

Mirrors the reference runtime API (tileinfer/src/runtime/runtime.hpp:18-124): ``load_plan``,
``DecoderModel``, ``SequenceContext.enqueue_prefill / enqueue_decode / enqueue_generate /
enqueue_reset / ready / wait / collect``.  Errors raise ``RuntimeError`` carrying the C++
runtime's message (the reference's messages, e.g. "sequence context capacity reached").
There is no fallback: without the built library every call raises.
"""

from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from pathlib import Path

import numpy as np

LIBRARY = Path(__file__).resolve().parent / "libtileinfer_amd.so"

token_id = C.c_int32


class TaskRecord(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("opcode", "layer", "begin", "end", "kv_head", "chunk")]


class ModelShape(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("hidden_size", "intermediate_size", "query_heads", "kv_heads", "head_dim",
                                         "max_context", "attention_chunks", "attention_chunk_steps",
                                         "attention_fused_steps", "ffn_chunks")]


class TaskRange(C.Structure):
    _fields_ = [("begin", C.c_uint32), ("count", C.c_uint32)]


class LayerLayout(C.Structure):
    _fields_ = [(n, C.c_uint32) for n in ("q", "k", "q_rot", "attention", "r", "product", "key", "value", "attn_norm",
                                          "Wq", "Wk", "Wv", "Wo", "ffn_norm", "Wgate", "Wup", "Wdown")]


class NumericConfig(C.Structure):
    _fields_ = [(n, C.c_float) for n in ("rms_norm_eps", "rope_theta", "rope_factor", "rope_low_freq_factor",
                                         "rope_high_freq_factor", "rope_original_context")]


class StackConfig(C.Structure):
    _fields_ = [(n, C.c_int32) for n in ("layers", "vocab_size", "embedding_offset", "layer_weights_offset",
                                         "layer_weight_stride", "final_norm_offset", "lm_head_offset",
                                         "layer_kv_stride", "full_stack")]


class ProgramView(C.Structure):
    """ti_worker_program_view (WorkerProgramView, launch.cuh:10-23)."""
    _fields_ = [("instructions", C.c_void_p), ("streams", C.c_void_p), ("layout", LayerLayout), ("weights", C.c_void_p),
                ("rotary_frequencies", C.c_void_p), ("shape", ModelShape), ("workers", C.c_int32),
                ("selection_slots", C.c_int32), ("numeric", NumericConfig), ("stack", StackConfig),
                ("weight_dtype", C.c_int32)]


# Words per instruction of a worker timeline record (include/tileinfer_amd.h): the reference's
# {start cycles, end cycles, start ns} and this build's {start, first read, inputs complete, end}.
TIMELINE_REFERENCE_FIELDS = 3
TIMELINE_FIELDS = 4


class WorkerBuffers(C.Structure):
    """ti_worker_buffers (WorkerBuffers, launch.cuh:31-45, plus the exchange area and its epoch)."""
    _fields_ = [(n, C.c_void_p) for n in ("input", "output", "scratch", "kv", "logits", "block_trace",
                                          "attention_scores", "attention_partials", "selection", "ffn_trace",
                                          "timeline", "exchange")] + [("epoch", C.c_uint32), ("timeline_fields", C.c_int32)]


class TokenInput(C.Structure):
    """ti_token_input (TokenInput, launch.cuh:49-54)."""
    _fields_ = [("immediate", token_id), ("ids", C.c_void_p), ("steps", C.c_int32)]


class Selection(C.Structure):
    """ti_selection (Selection, launch.cuh:79-85)."""
    _fields_ = [("generated", C.c_void_p), ("status", C.c_void_p), ("first", C.c_int32), ("eos_id", token_id)]


class Target(C.Structure):
    _fields_ = [("name", C.c_char * 256), ("arch", C.c_char * 64)] + [
        (n, C.c_int32) for n in ("major", "minor", "sm_count", "cooperative_launch", "active_blocks_per_sm",
                                 "registers_per_thread", "static_shared_bytes", "max_threads_per_sm",
                                 "threads_per_block", "attention_shared_bytes")] + [
        ("global_memory_bytes", C.c_uint64)] + [
        (n, C.c_int32) for n in ("driver_version", "runtime_version", "f32_registers", "f32_shared_bytes",
                                 "f32_active_blocks", "bf16_registers", "bf16_shared_bytes", "bf16_active_blocks")]


class DiagnosticRequest(C.Structure):
    _fields_ = [("logits", C.c_int32), ("kv", C.c_int32), ("block_outputs", C.c_int32)]


class Completion(C.Structure):
    _fields_ = [("count", C.c_int32), ("position", C.c_int32), ("stop_reason", C.c_int32), ("compute_us", C.c_double)]


STOP_REASONS = {0: "none", 1: "limit", 2: "eos"}
EXPORTS = ("ti_error_string", "ti_last_error_message", "ti_abi", "ti_fingerprint", "ti_describe_target",
           "ti_exchange_words", "ti_epochs_per_launch", "ti_epoch_after_generation", "ti_enqueue_worker",
           "ti_enqueue_worker_static", "ti_static_exchange_words", "ti_model_program_view", "ti_enqueue_zero_unused_kv",
           "ti_enqueue_widen", "ti_measure_stream_read", "ti_load_plan", "ti_load_plan_for_target", "ti_plan_free", "ti_plan_inspect_json",
           "ti_model_create", "ti_model_free", "ti_context_create", "ti_context_free", "ti_context_prefill",
           "ti_context_decode", "ti_context_generate", "ti_context_reset", "ti_context_ready", "ti_context_wait",
           "ti_context_diagnostic_sizes", "ti_context_collect", "ti_context_intermediate_sizes",
           "ti_context_collect_intermediates", "ti_ticket_free", "ti_context_set_timeline",
           "ti_context_timeline", "ti_context_set_matrix_prefill", "ti_context_lm_head_step",
           "ti_set_worker_spin_limit", "ti_relayout_weights")
DEFAULT_SPIN_LIMIT = 1 << 20  # TI_DEFAULT_SPIN_LIMIT

_lib = None


def library_path() -> Path:
    """The in-tree library this process uses: libtileinfer_amd.so, or another build of it in the
    package directory named by TILES_AMD_LIBRARY (the delay-injection stress build,
    libtileinfer_amd_delay.so)."""
    name = os.environ.get("TILES_AMD_LIBRARY", LIBRARY.name)
    if "/" in name or not name.startswith("libtileinfer_amd") or not name.endswith(".so"):
        raise RuntimeError(f"TILES_AMD_LIBRARY must name a build of the library in {LIBRARY.parent}")
    return LIBRARY.parent / name


def library() -> C.CDLL:
    """The loaded C-ABI library; raises if it was not built (no CPU fallback exists)."""
    global _lib
    if _lib is None:
        path = library_path()
        if not path.exists():
            raise RuntimeError(f"{path} is missing: run python -m tiles_amd.build (hipcc, gfx950)")
        lib = C.CDLL(str(path), mode=os.RTLD_NOW | C.RTLD_GLOBAL)
        P = C.c_void_p
        lib.ti_error_string.restype = C.c_char_p
        lib.ti_last_error_message.restype = C.c_char_p
        lib.ti_abi.restype = C.c_char_p
        lib.ti_fingerprint.restype = C.c_char_p
        lib.ti_describe_target.argtypes = [C.POINTER(Target)]
        lib.ti_exchange_words.argtypes = [C.POINTER(ModelShape), C.c_int32, C.c_int32]
        lib.ti_exchange_words.restype = C.c_size_t
        lib.ti_epochs_per_launch.argtypes = [C.c_int32]
        lib.ti_epochs_per_launch.restype = C.c_uint32
        lib.ti_epoch_after_generation.argtypes = [C.c_uint32, C.POINTER(C.c_uint32), C.c_int32, C.c_int32, C.c_int32]
        lib.ti_epoch_after_generation.restype = C.c_uint32
        lib.ti_enqueue_worker.argtypes = [C.c_void_p, C.POINTER(ProgramView), C.POINTER(WorkerBuffers), C.c_int32,
                                          TokenInput, Selection]
        lib.ti_enqueue_worker_static.argtypes = [C.c_void_p, C.POINTER(ProgramView), C.POINTER(WorkerBuffers), C.c_int32,
                                                 TokenInput, Selection, C.c_void_p]
        lib.ti_static_exchange_words.restype = C.c_size_t
        lib.ti_model_program_view.argtypes = [P, C.POINTER(ProgramView)]
        lib.ti_measure_stream_read.argtypes = [C.c_size_t, C.c_int32, C.POINTER(C.c_double)]
        lib.ti_load_plan.argtypes = [C.c_char_p, C.c_int32, C.POINTER(P)]
        lib.ti_load_plan_for_target.argtypes = [C.c_char_p, C.POINTER(Target), C.c_int32, C.POINTER(P)]
        lib.ti_plan_free.argtypes = [P]
        lib.ti_plan_free.restype = None
        lib.ti_plan_inspect_json.argtypes = [P]
        lib.ti_plan_inspect_json.restype = C.c_char_p
        lib.ti_model_create.argtypes = [P, C.POINTER(P)]
        lib.ti_model_free.argtypes = [P]
        lib.ti_model_free.restype = None
        lib.ti_context_create.argtypes = [P, C.POINTER(P)]
        lib.ti_context_free.argtypes = [P]
        lib.ti_context_free.restype = None
        lib.ti_context_prefill.argtypes = [P, C.POINTER(token_id), C.c_size_t, DiagnosticRequest, C.POINTER(P)]
        lib.ti_context_decode.argtypes = [P, token_id, DiagnosticRequest, C.POINTER(P)]
        lib.ti_context_generate.argtypes = [P, C.c_int32, token_id, DiagnosticRequest, C.POINTER(P)]
        lib.ti_context_reset.argtypes = [P, C.POINTER(P)]
        lib.ti_context_lm_head_step.argtypes = [P, P, C.c_int32, DiagnosticRequest, C.POINTER(P)]
        lib.ti_context_ready.argtypes = [P, P]
        lib.ti_context_wait.argtypes = [P, P, C.POINTER(Completion), C.POINTER(token_id), C.c_size_t]
        lib.ti_context_diagnostic_sizes.argtypes = [P, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        lib.ti_context_collect.argtypes = [P, P, C.POINTER(C.c_float), C.POINTER(C.c_float), C.POINTER(C.c_float)]
        lib.ti_context_intermediate_sizes.argtypes = [P, C.POINTER(C.c_size_t), C.POINTER(C.c_size_t)]
        lib.ti_context_collect_intermediates.argtypes = [P, P, C.POINTER(C.c_float), C.POINTER(C.c_float)]
        lib.ti_ticket_free.argtypes = [P]
        lib.ti_ticket_free.restype = None
        lib.ti_context_set_timeline.argtypes = [P, C.c_int32]
        lib.ti_context_set_matrix_prefill.argtypes = [P, C.c_int32]
        lib.ti_set_worker_spin_limit.argtypes = [C.c_uint32]
        lib.ti_set_worker_spin_limit.restype = None
        lib.ti_context_timeline.argtypes = [P, C.POINTER(C.c_uint64), C.c_size_t, C.POINTER(C.c_size_t)]
        _lib = lib
    return _lib


def _check(code: int) -> None:
    if code != 0:
        message = library().ti_last_error_message().decode()
        raise RuntimeError(message or library().ti_error_string(code).decode())


def describe_target() -> Target:
    target = Target()
    _check(library().ti_describe_target(C.byref(target)))
    return target


def measure_stream_read(bytes_: int = 2 << 30, repeats: int = 3) -> float:
    """Best streaming-read GB/s of the device (the roofline the byte floor is quoted against)."""
    best = C.c_double()
    _check(library().ti_measure_stream_read(bytes_, repeats, C.byref(best)))
    return best.value


def target_from_probe(probe: dict) -> Target:
    """A Target matching a normalized probe document (for loading packages without a device,
    as the reference's loader tests do with a fake capability)."""
    t = Target()
    device, executor = probe["device"], probe["executor"]
    t.name = device.get("name", "").encode()[:255]
    t.major, t.minor = device["compute_capability"]
    t.sm_count = device["sm_count"]
    t.cooperative_launch = 1 if device["cooperative_launch"] else 0
    t.active_blocks_per_sm = executor["active_blocks_per_sm"]
    t.threads_per_block = executor["threads_per_block"]
    t.attention_shared_bytes = executor["attention_shared_bytes"]
    return t


class Plan:
    """A validated package (LoadedPlan, plan.hpp:238-266)."""

    def __init__(self, package: str | Path, verify_weights: bool = True, target: Target | None = None):
        handle = C.c_void_p()
        path = str(package).encode()
        if target is None:
            _check(library().ti_load_plan(path, int(verify_weights), C.byref(handle)))
        else:
            _check(library().ti_load_plan_for_target(path, C.byref(target), int(verify_weights), C.byref(handle)))
        self._handle = handle

    def inspect(self) -> dict:
        import json

        return json.loads(library().ti_plan_inspect_json(self._handle).decode())

    def __del__(self):
        if getattr(self, "_handle", None) and _lib is not None:
            _lib.ti_plan_free(self._handle)
            self._handle = None


def load_plan(package: str | Path, verify_weights: bool = True) -> Plan:
    return Plan(package, verify_weights)


@dataclass
class Result:
    generated: list[int]
    position: int
    stop_reason: str
    compute_us: float


class Ticket:
    def __init__(self, context: "SequenceContext", handle: C.c_void_p, kind: str, requested: int = 0):
        self._context, self._handle, self.kind, self.requested = context, handle, kind, requested

    def __del__(self):
        if getattr(self, "_handle", None) and _lib is not None:
            _lib.ti_ticket_free(self._handle)
            self._handle = None


class DecoderModel:
    """Uploads one validated package; shareable by sequence contexts."""

    def __init__(self, plan: Plan):
        handle = C.c_void_p()
        _check(library().ti_model_create(plan._handle, C.byref(handle)))
        self._handle = handle
        self.plan = plan

    def program_view(self) -> ProgramView:
        """The uploaded model's launch-boundary view (device pointers owned by this model)."""
        view = ProgramView()
        _check(library().ti_model_program_view(self._handle, C.byref(view)))
        return view

    def create_context(self) -> "SequenceContext":
        return SequenceContext(self)

    def __del__(self):
        if getattr(self, "_handle", None) and _lib is not None:
            _lib.ti_model_free(self._handle)
            self._handle = None


class SequenceContext:
    """One sequence's stream, K/V cache and tickets; calls must be serialized by the caller."""

    def __init__(self, model: DecoderModel):
        handle = C.c_void_p()
        _check(library().ti_context_create(model._handle, C.byref(handle)))
        self._handle = handle
        self.model = model
        sizes = [C.c_size_t() for _ in range(3)]
        _check(library().ti_context_diagnostic_sizes(handle, *[C.byref(s) for s in sizes]))
        self.logits_size, self.kv_size, self.blocks_size = (s.value for s in sizes)

    def __del__(self):
        if getattr(self, "_handle", None) and _lib is not None:
            _lib.ti_context_free(self._handle)
            self._handle = None

    @staticmethod
    def _request(logits=False, kv=False, block_outputs=False) -> DiagnosticRequest:
        return DiagnosticRequest(int(logits), int(kv), int(block_outputs))

    def enqueue_prefill(self, token_ids, logits=False, kv=False, block_outputs=False) -> Ticket:
        ids = (token_id * len(token_ids))(*[int(t) for t in token_ids])
        handle = C.c_void_p()
        _check(library().ti_context_prefill(self._handle, ids, len(token_ids),
                                            self._request(logits, kv, block_outputs), C.byref(handle)))
        return Ticket(self, handle, "prefill")

    def enqueue_decode(self, token: int, logits=False, kv=False, block_outputs=False) -> Ticket:
        handle = C.c_void_p()
        _check(library().ti_context_decode(self._handle, int(token), self._request(logits, kv, block_outputs),
                                           C.byref(handle)))
        return Ticket(self, handle, "prefill")

    def enqueue_generate(self, max_new_tokens: int, eos_id: int | None = None, logits=False, kv=False,
                         block_outputs=False) -> Ticket:
        handle = C.c_void_p()
        _check(library().ti_context_generate(self._handle, int(max_new_tokens), -1 if eos_id is None else int(eos_id),
                                             self._request(logits, kv, block_outputs), C.byref(handle)))
        return Ticket(self, handle, "generate", max(0, int(max_new_tokens)))

    def enqueue_reset(self) -> Ticket:
        handle = C.c_void_p()
        _check(library().ti_context_reset(self._handle, C.byref(handle)))
        return Ticket(self, handle, "reset")

    def ready(self, ticket: Ticket) -> bool:
        code = library().ti_context_ready(self._handle, ticket._handle)
        if code < 0:
            _check(-code)
        return code == 1

    def wait(self, ticket: Ticket) -> Result:
        done = Completion()
        ids = (token_id * max(1, ticket.requested))()
        _check(library().ti_context_wait(self._handle, ticket._handle, C.byref(done), ids, ticket.requested))
        return Result(list(ids[: done.count]) if ticket.requested else [], done.position,
                      STOP_REASONS.get(done.stop_reason, "none"), done.compute_us)

    def enqueue_lm_head_step(self, hidden, rounds: int = 1, logits: bool = False) -> Ticket:
        """The isolated LM-head step, `rounds` times, on an empty context: `hidden` (hidden_size
        values, bf16 bits as uint16 for a bf16 package, float32 otherwise) through the final
        RMSNorm, the LM head and greedy selection by the worker's logits tasks.  wait() gives
        the token and, as compute_us, the median round's worker launch."""
        import numpy as np
        view = self.model.program_view()
        vector = np.ascontiguousarray(hidden, dtype=np.uint16 if view.weight_dtype == 1 else np.float32)
        if vector.size != view.shape.hidden_size:
            raise ValueError("hidden vector of the wrong size")
        handle = C.c_void_p()
        _check(library().ti_context_lm_head_step(self._handle, vector.ctypes.data_as(C.c_void_p), int(rounds),
                                                 self._request(logits, False, False), C.byref(handle)))
        return Ticket(self, handle, "lm_head", 1)

    def set_matrix_prefill(self, enabled: bool) -> None:
        """Prefills of more than 64 tokens on bf16 stacks run all but the last token as matrices
        (on by default); off, every token goes through the worker."""
        _check(library().ti_context_set_matrix_prefill(self._handle, int(enabled)))

    def set_timeline(self, enabled: bool) -> None:
        _check(library().ti_context_set_timeline(self._handle, int(enabled)))

    def timeline(self) -> np.ndarray:
        """[instructions, 4] device-clock stamps (100 MHz) of the last launch's last step: start,
        first exchange read returned, inputs complete, end."""
        count = C.c_size_t()
        _check(library().ti_context_timeline(self._handle, None, 0, C.byref(count)))
        words = np.zeros(4 * count.value, dtype=np.uint64)
        _check(library().ti_context_timeline(self._handle, words.ctypes.data_as(C.POINTER(C.c_uint64)), words.size,
                                             C.byref(count)))
        return words.reshape(-1, 4)

    def collect(self, ticket: Ticket) -> dict:
        logits = np.zeros(self.logits_size, dtype=np.float32)
        kv = np.zeros(self.kv_size, dtype=np.float32)
        blocks = np.zeros(self.blocks_size, dtype=np.float32)
        fp = C.POINTER(C.c_float)
        _check(library().ti_context_collect(self._handle, ticket._handle, logits.ctypes.data_as(fp),
                                            kv.ctypes.data_as(fp), blocks.ctypes.data_as(fp)))
        return {"logits": logits, "kv": kv, "block_outputs": blocks}

    def collect_intermediates(self, ticket: Ticket) -> dict:
        """Scratch vectors (widened, in plan.json's storage.scratch layout) and each layer's FFN
        output before the residual, of a request made with block_outputs=True."""
        scratch, ffn = C.c_size_t(), C.c_size_t()
        _check(library().ti_context_intermediate_sizes(self._handle, C.byref(scratch), C.byref(ffn)))
        out = {"scratch": np.zeros(scratch.value, dtype=np.float32), "ffn": np.zeros(ffn.value, dtype=np.float32)}
        fp = C.POINTER(C.c_float)
        _check(library().ti_context_collect_intermediates(self._handle, ticket._handle, out["scratch"].ctypes.data_as(fp),
                                                          out["ffn"].ctypes.data_as(fp)))
        return out
