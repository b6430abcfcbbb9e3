"""Python bindings of libtgx's C ABI (include/tgx.h), shaped like the reference's model API:
`Decoder` as crates/graph/src/decode.rs's (`new`/`with_batch`, `load`, `step`, `step_rows`,
`set_rows`, `start`, `output`, `timings`), `Row` and `Batch` as its placement types, and
`Decoder.prefill` as crates/graph/src/prefill.rs's `Prefill::run`.

The library is the only thing that computes: if libtgx.so is missing these bindings raise, they
never fall back to anything else.
"""

from __future__ import annotations

import atexit
import itertools
import ctypes
import os
import sys
import weakref
from dataclasses import dataclass, field
from pathlib import Path
from typing import Optional, Sequence

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = Path(os.environ.get("TGX_LIB", HERE.parent / "libtgx.so"))

SPARE = 0xFFFFFFFF

F32, BF16, F16 = 0, 1, 2

STATUS = {
    0: "ok",
    1: "shape",
    2: "hip",
    3: "kernels",
    4: "weights",
    5: "not_finite",
    6: "timeout",
    7: "busy",
    8: "arg",
    9: "no_device",
}


class TgxError(RuntimeError):
    """A failed call: `kind` names its status class (graph::Error's, crates/graph/src/lib.rs:41-59)."""

    def __init__(self, status: int, message: str):
        self.status = status
        self.kind = STATUS.get(status, str(status))
        super().__init__(f"{self.kind}: {message}")


class _Shape(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int),
        ("inner", ctypes.c_int),
        ("heads", ctypes.c_int),
        ("kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("layers", ctypes.c_int),
        ("capacity", ctypes.c_int),
        ("eps", ctypes.c_float),
        ("rope_theta", ctypes.c_float),
        ("rope", ctypes.c_int),
        ("rope_factors", ctypes.POINTER(ctypes.c_double)),
    ]


class _Batch(ctypes.Structure):
    _fields_ = [
        ("rows", ctypes.c_int),
        ("slots", ctypes.c_int),
        ("block_tokens", ctypes.c_int),
        ("blocks", ctypes.c_int),
    ]


class _Row(ctypes.Structure):
    _fields_ = [("position", ctypes.c_uint32), ("slot", ctypes.c_uint32)]


class _Run(ctypes.Structure):
    _fields_ = [("slot", ctypes.c_uint32), ("start", ctypes.c_uint32), ("len", ctypes.c_uint32)]


class _PatchShape(ctypes.Structure):
    _fields_ = [("feat_dim", ctypes.c_int), ("patch_size", ctypes.c_int), ("timesteps", ctypes.c_int), ("rows", ctypes.c_int)]


class _HeadsShape(ctypes.Structure):
    _fields_ = [("encoder", ctypes.c_int), ("dit", ctypes.c_int), ("latent", ctypes.c_int), ("levels", ctypes.c_int)]


class _Timing(ctypes.Structure):
    _fields_ = [("label", ctypes.c_char * 32), ("ms", ctypes.c_float)]


class _Calibration(ctypes.Structure):
    _fields_ = [("ticks", ctypes.c_uint64), ("monotonic_ns", ctypes.c_uint64), ("deviation_ns", ctypes.c_uint64),
                ("period_ns", ctypes.c_float)]


class _Report(ctypes.Structure):
    _fields_ = [
        ("name", ctypes.c_char * 64),
        ("arch", ctypes.c_char * 32),
        ("compute_units", ctypes.c_int),
        ("clock_khz", ctypes.c_int),
        ("memory_clock_khz", ctypes.c_int),
        ("memory_bytes", ctypes.c_size_t),
        ("wavefront", ctypes.c_int),
    ]


EXPORTS = [
    "tgx_last_error",
    "tgx_context_create",
    "tgx_context_destroy",
    "tgx_context_report",
    "tgx_stream_read",
    "tgx_decoder_create",
    "tgx_decoder_destroy",
    "tgx_decoder_load",
    "tgx_decoder_set_rows",
    "tgx_decoder_start",
    "tgx_decoder_wait",
    "tgx_decoder_output",
    "tgx_decoder_step_rows",
    "tgx_decoder_step",
    "tgx_decoder_release_slot",
    "tgx_decoder_reserve",
    "tgx_decoder_free_blocks",
    "tgx_decoder_launch",
    "tgx_decoder_elapsed_ms",
    "tgx_decoder_dispatches",
    "tgx_decoder_device_bytes",
    "tgx_decoder_read_cache",
    "tgx_decoder_set_timed",
    "tgx_decoder_set_graph",
    "tgx_decoder_timings",
    "tgx_shape_check",
    "tgx_batch_placement",
    "tgx_prefill_run",
    "tgx_prefill_runs",
    "tgx_prefill_launch",
    "tgx_prefill_runs_noalloc",
    "tgx_euler_steps",
    "tgx_sampler_create",
    "tgx_sampler_destroy",
    "tgx_sampler_load",
    "tgx_sampler_sample",
    "tgx_sampler_launch",
    "tgx_sampler_wait",
    "tgx_sampler_elapsed_ms",
    "tgx_sampler_set_timed",
    "tgx_sampler_timings",
    "tgx_sampler_dispatches",
    "tgx_lm_side_create",
    "tgx_lm_side_destroy",
    "tgx_lm_side_load",
    "tgx_lm_side_decoder",
    "tgx_lm_side_set_rows",
    "tgx_lm_side_step",
    "tgx_lm_side_launch",
    "tgx_lm_side_wait",
    "tgx_lm_side_elapsed_ms",
    "tgx_lm_side_read",
    "tgx_lm_side_dispatches",
    "tgx_patch_launch",
    "tgx_patch_elapsed_ms",
    "tgx_encoder_create",
    "tgx_encoder_destroy",
    "tgx_encoder_load",
    "tgx_encoder_encode",
    "tgx_encoder_dispatches",
    "tgx_patch_step_create",
    "tgx_patch_step_destroy",
    "tgx_patch_step_run",
    "tgx_patch_step_launch",
    "tgx_patch_step_wait",
    "tgx_patch_step_elapsed_ms",
    "tgx_checkpoint_open",
    "tgx_checkpoint_close",
    "tgx_checkpoint_count",
    "tgx_checkpoint_name",
    "tgx_checkpoint_shape",
    "tgx_checkpoint_read",
    "tgx_checkpoint_gather",
    "tgx_decoder_load_checkpoint",
    "tgx_lm_side_load_checkpoint",
    "tgx_sampler_load_checkpoint",
    "tgx_encoder_load_checkpoint",
    "tgx_prompter_create",
    "tgx_prompter_destroy",
    "tgx_prompter_max_rows",
    "tgx_prompter_embed",
    "tgx_prompter_embeddings",
    "tgx_prompter_run_rows",
    "tgx_prompter_run",
    "tgx_prompter_run_cached",
    "tgx_prompter_read",
    "tgx_prompt_cache_create",
    "tgx_prompt_cache_destroy",
    "tgx_prompt_cache_bytes",
    "tgx_prompt_cache_voices",
    "tgx_engine_create",
    "tgx_engine_destroy",
    "tgx_engine_slots",
    "tgx_engine_start",
    "tgx_engine_sample_after",
    "tgx_engine_step",
    "tgx_engine_levels",
    "tgx_engine_take_frames",
    "tgx_engine_finish",
    "tgx_engine_prompt_cache",
    "tgx_alloc",
    "tgx_free",
    "tgx_memory_info",
    "tgx_write",
    "tgx_read",
    "tgx_tiles_bytes",
    "tgx_write_tiles",
    "tgx_rope_tables",
    "tgx_kernel_count",
    "tgx_kernel_find",
    "tgx_kernel_info",
    "tgx_kernel_binding",
    "tgx_kernel_constant",
    "tgx_program_begin",
    "tgx_program_launch",
    "tgx_program_end",
    "tgx_program_start",
    "tgx_program_wait",
    "tgx_program_run",
    "tgx_program_timings",
    "tgx_program_elapsed_ms",
    "tgx_program_destroy",
    "tgx_copy_regions",
]

_lib: Optional[ctypes.CDLL] = None

# Every open handle, closed before the interpreter exits: the HIP runtime tears itself down in the
# C library's exit handlers, after which no handle may be freed. Decoders, samplers and LM sides
# (everything made from a context) go before contexts, newest first: a patch step or an engine
# before the encoder, LM side and sampler it uses, which must outlive it.
_open_decoders: "weakref.WeakSet" = weakref.WeakSet()
_open_contexts: "weakref.WeakSet" = weakref.WeakSet()
_open_order = itertools.count()


def _opened(handle) -> None:
    """Registers a handle made from a context, to be closed before it, newest first."""
    handle._open_seq = next(_open_order)
    _open_decoders.add(handle)


def _newest_first(handles) -> list:
    return sorted(handles, key=lambda h: getattr(h, "_open_seq", -1), reverse=True)


@atexit.register
def _close_all() -> None:
    for d in _newest_first(list(_open_decoders)):
        d.close()
    for c in list(_open_contexts):
        c.close()


def library() -> ctypes.CDLL:
    """libtgx.so, loaded once; raises when it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise TgxError(3, f"{LIB_PATH} is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(LIB_PATH))
    P = ctypes.c_void_p
    lib.tgx_last_error.restype = ctypes.c_char_p
    lib.tgx_context_create.argtypes = [ctypes.c_int, ctypes.POINTER(P)]
    lib.tgx_context_destroy.argtypes = [P]
    lib.tgx_context_destroy.restype = None
    lib.tgx_context_report.argtypes = [P, ctypes.POINTER(_Report)]
    lib.tgx_context_set_fence_spin.argtypes = [P, ctypes.c_uint64]
    lib.tgx_context_calibrate.argtypes = [P, ctypes.POINTER(_Calibration)]
    lib.tgx_stream_read.argtypes = [P, ctypes.c_size_t, ctypes.c_int, ctypes.POINTER(ctypes.c_float), ctypes.POINTER(ctypes.c_float)]
    lib.tgx_decoder_create.argtypes = [P, ctypes.POINTER(_Shape), ctypes.POINTER(_Batch), ctypes.POINTER(P)]
    lib.tgx_decoder_destroy.argtypes = [P]
    lib.tgx_decoder_destroy.restype = None
    lib.tgx_decoder_load.argtypes = [P, ctypes.c_char_p, P, ctypes.c_int, ctypes.c_size_t]
    lib.tgx_decoder_set_rows.argtypes = [P, ctypes.POINTER(_Row), ctypes.c_int, P]
    lib.tgx_decoder_start.argtypes = [P]
    lib.tgx_decoder_wait.argtypes = [P]
    lib.tgx_decoder_output.argtypes = [P, P]
    lib.tgx_decoder_step_rows.argtypes = [P, ctypes.POINTER(_Row), ctypes.c_int, P, P]
    lib.tgx_decoder_step.argtypes = [P, ctypes.c_uint32, P, P]
    lib.tgx_decoder_release_slot.argtypes = [P, ctypes.c_uint32]
    lib.tgx_decoder_reserve.argtypes = [P, ctypes.c_uint32, ctypes.c_uint32]
    lib.tgx_decoder_free_blocks.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_decoder_launch.argtypes = [P, ctypes.c_int, ctypes.c_int]
    lib.tgx_decoder_elapsed_ms.argtypes = [P, ctypes.POINTER(ctypes.c_float)]
    lib.tgx_decoder_dispatches.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_decoder_device_bytes.argtypes = [P, ctypes.POINTER(ctypes.c_size_t)]
    lib.tgx_decoder_read_cache.argtypes = [P, ctypes.c_uint32, ctypes.c_uint32, P, P]
    lib.tgx_decoder_set_timed.argtypes = [P, ctypes.c_int]
    lib.tgx_decoder_set_graph.argtypes = [P, ctypes.c_int]
    lib.tgx_decoder_timings.argtypes = [P, ctypes.c_int, ctypes.POINTER(_Timing), ctypes.POINTER(ctypes.c_int)]
    lib.tgx_shape_check.argtypes = [ctypes.POINTER(_Shape), ctypes.POINTER(_Batch)]
    lib.tgx_batch_placement.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(_Row), ctypes.c_int, ctypes.POINTER(ctypes.c_uint32)]
    lib.tgx_prefill_run.argtypes = [P, ctypes.c_uint32, ctypes.c_uint32, ctypes.c_uint32, P, P]
    lib.tgx_prefill_runs.argtypes = [P, ctypes.POINTER(_Run), ctypes.c_int, P, P]
    lib.tgx_prefill_launch.argtypes = [P, ctypes.c_int]
    lib.tgx_prefill_runs_noalloc.argtypes = [P, ctypes.POINTER(_Run), ctypes.c_int, P, P]
    FP = ctypes.POINTER(ctypes.c_float)
    lib.tgx_euler_steps.argtypes = [ctypes.c_int, ctypes.c_int, FP, FP, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_sampler_create.argtypes = [P, ctypes.POINTER(_Shape), ctypes.POINTER(_PatchShape), ctypes.POINTER(P)]
    lib.tgx_sampler_destroy.argtypes = [P]
    lib.tgx_sampler_destroy.restype = None
    lib.tgx_sampler_load.argtypes = [P, ctypes.c_char_p, P, ctypes.c_int, ctypes.c_size_t]
    lib.tgx_sampler_sample.argtypes = [P, P, P, P, P, P]
    lib.tgx_sampler_launch.argtypes = [P, ctypes.c_int]
    lib.tgx_sampler_wait.argtypes = [P]
    lib.tgx_sampler_elapsed_ms.argtypes = [P, FP]
    lib.tgx_sampler_set_timed.argtypes = [P, ctypes.c_int]
    lib.tgx_sampler_timings.argtypes = [P, ctypes.c_int, ctypes.POINTER(_Timing), ctypes.POINTER(ctypes.c_int)]
    lib.tgx_sampler_dispatches.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_lm_side_create.argtypes = [P, ctypes.POINTER(_Shape), ctypes.POINTER(_Shape), ctypes.POINTER(_Batch),
                                       ctypes.POINTER(_HeadsShape), ctypes.POINTER(P)]
    lib.tgx_lm_side_destroy.argtypes = [P]
    lib.tgx_lm_side_destroy.restype = None
    lib.tgx_lm_side_load.argtypes = [P, ctypes.c_char_p, P, ctypes.c_int, ctypes.c_size_t]
    lib.tgx_lm_side_decoder.argtypes = [P, ctypes.c_int, ctypes.POINTER(P)]
    lib.tgx_lm_side_set_rows.argtypes = [P, ctypes.POINTER(_Row), ctypes.c_int, P]
    lib.tgx_lm_side_step.argtypes = [P, ctypes.POINTER(_Row), ctypes.c_int, P, P, P]
    lib.tgx_lm_side_launch.argtypes = [P, ctypes.c_int, ctypes.c_int]
    lib.tgx_lm_side_wait.argtypes = [P]
    lib.tgx_lm_side_elapsed_ms.argtypes = [P, FP]
    lib.tgx_lm_side_read.argtypes = [P, ctypes.c_char_p, P, ctypes.c_size_t]
    lib.tgx_lm_side_dispatches.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_patch_launch.argtypes = [P, P, ctypes.c_int]
    lib.tgx_patch_elapsed_ms.argtypes = [P, FP]
    lib.tgx_encoder_create.argtypes = [P, ctypes.POINTER(_Shape), ctypes.POINTER(_PatchShape), ctypes.POINTER(P)]
    lib.tgx_encoder_destroy.argtypes = [P]
    lib.tgx_encoder_destroy.restype = None
    lib.tgx_encoder_load.argtypes = [P, ctypes.c_char_p, P, ctypes.c_int, ctypes.c_size_t]
    lib.tgx_encoder_encode.argtypes = [P, P, P]
    lib.tgx_encoder_dispatches.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_patch_step_create.argtypes = [P, P, P, ctypes.POINTER(P)]
    lib.tgx_patch_step_destroy.argtypes = [P]
    lib.tgx_patch_step_destroy.restype = None
    lib.tgx_patch_step_run.argtypes = [P, ctypes.POINTER(_Row), ctypes.c_int, P, P, P, P, P]
    lib.tgx_patch_step_launch.argtypes = [P, ctypes.c_int, ctypes.c_int]
    lib.tgx_patch_step_wait.argtypes = [P]
    lib.tgx_patch_step_elapsed_ms.argtypes = [P, FP]
    lib.tgx_checkpoint_open.argtypes = [ctypes.c_char_p, ctypes.POINTER(P)]
    lib.tgx_checkpoint_close.argtypes = [P]
    lib.tgx_checkpoint_close.restype = None
    lib.tgx_checkpoint_count.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_checkpoint_name.argtypes = [P, ctypes.c_int, ctypes.c_char_p, ctypes.c_size_t]
    lib.tgx_checkpoint_shape.argtypes = [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64), ctypes.c_int,
                                         ctypes.POINTER(ctypes.c_int), ctypes.POINTER(ctypes.c_int)]
    lib.tgx_checkpoint_read.argtypes = [P, ctypes.c_char_p, P, ctypes.c_size_t]
    lib.tgx_checkpoint_gather.argtypes = [P, ctypes.c_char_p, P, ctypes.c_int, P]
    lib.tgx_decoder_load_checkpoint.argtypes = [P, P, ctypes.c_char_p]
    lib.tgx_lm_side_load_checkpoint.argtypes = [P, P]
    lib.tgx_sampler_load_checkpoint.argtypes = [P, P]
    lib.tgx_encoder_load_checkpoint.argtypes = [P, P]
    lib.tgx_prompter_create.argtypes = [P, ctypes.c_int, ctypes.POINTER(P)]
    lib.tgx_prompter_destroy.argtypes = [P]
    lib.tgx_prompter_destroy.restype = None
    lib.tgx_prompter_max_rows.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_prompter_embed.argtypes = [P, P, P]
    lib.tgx_prompter_embeddings.argtypes = [P, P, P, P, P]
    lib.tgx_prompter_run_rows.argtypes = [P, _Row, P, P, P, ctypes.c_int]
    lib.tgx_prompter_run.argtypes = [P, ctypes.c_uint32, P, P]
    lib.tgx_prompter_run_cached.argtypes = [P, ctypes.c_uint32, P, P, P, ctypes.c_size_t, P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_prompter_read.argtypes = [P, ctypes.c_char_p, P, ctypes.c_size_t]
    lib.tgx_prompt_cache_create.argtypes = [P, ctypes.c_size_t, ctypes.POINTER(P)]
    lib.tgx_prompt_cache_destroy.argtypes = [P]
    lib.tgx_prompt_cache_destroy.restype = None
    lib.tgx_prompt_cache_bytes.argtypes = [P, ctypes.POINTER(ctypes.c_size_t)]
    lib.tgx_prompt_cache_voices.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_engine_create.argtypes = [P, P, P, P, P, P, P, ctypes.c_int, ctypes.c_int, P, ctypes.POINTER(P)]
    lib.tgx_engine_destroy.argtypes = [P]
    lib.tgx_engine_destroy.restype = None
    lib.tgx_engine_slots.argtypes = [P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_engine_start.argtypes = [P, ctypes.c_int, P, P, ctypes.c_size_t, ctypes.c_int, ctypes.c_float, ctypes.c_float,
                                     ctypes.POINTER(ctypes.c_int)]
    lib.tgx_engine_sample_after.argtypes = [P, ctypes.c_int, P]
    lib.tgx_engine_step.argtypes = [P, P, P, P, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_engine_levels.argtypes = [P, ctypes.c_int, P]
    lib.tgx_engine_take_frames.argtypes = [P, ctypes.c_int, P, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_engine_finish.argtypes = [P, ctypes.c_int, P, ctypes.c_int, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_engine_prompt_cache.argtypes = [P, ctypes.POINTER(ctypes.c_size_t), ctypes.POINTER(ctypes.c_int)]
    for name in EXPORTS:
        if name.startswith("tgx_") and name not in ("tgx_last_error",):
            fn = getattr(lib, name)
            if fn.restype is not None and fn.restype is not ctypes.c_char_p:
                fn.restype = ctypes.c_int
    lib.tgx_context_destroy.restype = None
    lib.tgx_decoder_destroy.restype = None
    lib.tgx_sampler_destroy.restype = None
    lib.tgx_lm_side_destroy.restype = None
    lib.tgx_encoder_destroy.restype = None
    lib.tgx_patch_step_destroy.restype = None
    lib.tgx_checkpoint_close.restype = None
    lib.tgx_prompter_destroy.restype = None
    lib.tgx_prompt_cache_destroy.restype = None
    lib.tgx_engine_destroy.restype = None
    _lib = lib
    return lib


def _check(status: int) -> None:
    if status != 0:
        msg = library().tgx_last_error().decode(errors="replace")
        raise TgxError(status, msg)


def _ptr(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


@dataclass
class Shape:
    """decode::Shape (crates/graph/src/decode.rs:65-82)."""

    hidden: int = 1024
    inner: int = 4096
    heads: int = 16
    kv_heads: int = 2
    head_dim: int = 64
    layers: int = 24
    capacity: int = 1024
    eps: float = 1e-5
    rope_theta: float = 10000.0
    rope: bool = True
    rope_factors: Optional[Sequence[float]] = None

    def weight_bytes(self, element: int = 2) -> int:
        """Shape::weight_bytes (decode.rs:130-135) for `element`-byte weights."""
        h, i, d = self.hidden, self.inner, self.head_dim
        qkv = (self.heads + 2 * self.kv_heads) * d * h
        layer = qkv + self.heads * d * h + 2 * i * h + i * h + 2 * h
        return element * (self.layers * layer + h)

    def kv_bytes_per_position(self, element: int = 2) -> int:
        """Keys and values of one position over every layer."""
        return self.layers * 2 * self.kv_heads * self.head_dim * element


def _shape_struct(shape: "Shape"):
    s = _Shape(shape.hidden, shape.inner, shape.heads, shape.kv_heads, shape.head_dim, shape.layers,
               shape.capacity, shape.eps, shape.rope_theta, 1 if shape.rope else 0, None)
    keep = None
    if shape.rope_factors is not None:
        keep = np.ascontiguousarray(shape.rope_factors, dtype=np.float64)
        s.rope_factors = keep.ctypes.data_as(ctypes.POINTER(ctypes.c_double))
    return s, keep


def check_shape(shape: "Shape", batch: "Batch") -> None:
    """The decoder's shape checks on the host alone (Shape::new, decode_batch_graph)."""
    s, _keep = _shape_struct(shape)
    b = _Batch(batch.rows, batch.slots, batch.block_tokens, batch.blocks)
    _check(library().tgx_shape_check(ctypes.byref(s), ctypes.byref(b)))


def placement(slots: int, capacity: int, rows: Sequence[Optional["Row"]]) -> list:
    """Batch::placement (decode.rs:198-227) on the host: positions then slots, SPARE for spare rows."""
    arr = (_Row * max(1, len(rows)))()
    for i, r in enumerate(rows):
        arr[i].position, arr[i].slot = (SPARE, SPARE) if r is None else (r.position, r.slot)
    words = (ctypes.c_uint32 * max(1, 2 * len(rows)))()
    _check(library().tgx_batch_placement(slots, capacity, arr, len(rows), words))
    return list(words)[: 2 * len(rows)]


@dataclass(frozen=True)
class Row:
    """decode::Row (decode.rs:230-235)."""

    position: int
    slot: int


@dataclass(frozen=True)
class Batch:
    """decode::Batch (decode.rs:171-178) with the paged cache's block pool."""

    rows: int = 1
    slots: int = 1
    blocks: int = 0
    block_tokens: int = 64


class Context:
    """vulkan::Context (crates/vulkan/src/context.rs:237-540): a device and its stream."""

    def __init__(self, device: int = 0):
        lib = library()
        self._h = ctypes.c_void_p()
        _check(lib.tgx_context_create(device, ctypes.byref(self._h)))
        _open_contexts.add(self)

    def report(self) -> dict:
        r = _Report()
        _check(library().tgx_context_report(self._h, ctypes.byref(r)))
        return {
            "name": r.name.decode(),
            "arch": r.arch.decode(),
            "compute_units": r.compute_units,
            "clock_khz": r.clock_khz,
            "memory_clock_khz": r.memory_clock_khz,
            "memory_bytes": r.memory_bytes,
            "wavefront": r.wavefront,
        }

    def set_fence_spin(self, ns: int) -> None:
        """Context::set_fence_spin: every wait for this context's work polls for up to `ns`
        nanoseconds before it sleeps between polls (0, the default, sleeps at once)."""
        _check(library().tgx_context_set_fence_spin(self._h, int(ns)))

    def calibrate(self) -> dict:
        """Context::calibrate: the GPU clock's `ticks` read while CLOCK_MONOTONIC read
        `monotonic_ns` (give or take `deviation_ns`), `period_ns` nanoseconds a tick."""
        c = _Calibration()
        _check(library().tgx_context_calibrate(self._h, ctypes.byref(c)))
        return {"ticks": c.ticks, "monotonic_ns": c.monotonic_ns, "deviation_ns": c.deviation_ns, "period_ns": c.period_ns}

    def stream_read(self, nbytes: int, times: int = 10) -> dict:
        """The stream-read floor (stream_read.comp): `nbytes` read once a launch, the best and mean
        of `times` launches; GB/s at the best."""
        best, mean = ctypes.c_float(), ctypes.c_float()
        _check(library().tgx_stream_read(self._h, nbytes, times, ctypes.byref(best), ctypes.byref(mean)))
        unit = 256 * 8 * 16
        read = nbytes - nbytes % unit
        return {"bytes": read, "best_ms": best.value, "mean_ms": mean.value, "GB_s": read / (best.value * 1e-3) / 1e9}

    def close(self) -> None:
        if self._h:
            for d in _newest_first(list(_open_decoders)):
                if getattr(d, "ctx", None) is self:
                    d.close()
            library().tgx_context_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


class Decoder:
    """decode::Decoder (decode.rs:778-913): the stack's weights, its paged KV cache and the step
    recorded as a HIP graph."""

    def __init__(self, ctx: Context, shape: Shape, batch: Batch = Batch()):
        self.ctx = ctx
        self.shape = shape
        self.batch = batch
        s, self._factors = _shape_struct(shape)
        b = _Batch(batch.rows, batch.slots, batch.block_tokens, batch.blocks)
        self._h = ctypes.c_void_p()
        _check(library().tgx_decoder_create(ctx._h, ctypes.byref(s), ctypes.byref(b), ctypes.byref(self._h)))
        _opened(self)

    # -- weights --
    def load_checkpoint(self, checkpoint, prefix: str = "") -> None:
        """load_stack (decode.rs:738-776) from a tgx.checkpoint.Checkpoint: the layers under
        `prefix` ("base_lm.", "residual_lm." or ""), q/k/v and gate/up joined along their rows."""
        _check(library().tgx_decoder_load_checkpoint(self._h, checkpoint._h, prefix.encode()))

    def load(self, name: str, values: np.ndarray) -> None:
        """load_stack's write of one tensor (decode.rs:740-776): f32, bf16 (uint16 bits) or f16."""
        a = np.ascontiguousarray(values)
        if a.dtype == np.float32:
            dtype = F32
        elif a.dtype == np.uint16:
            dtype = BF16
        elif a.dtype == np.float16:
            dtype = F16
        else:
            a = np.ascontiguousarray(a, dtype=np.float32)
            dtype = F32
        _check(library().tgx_decoder_load(self._h, name.encode(), _ptr(a), dtype, a.size))

    def load_all(self, weights: dict) -> None:
        for name, values in weights.items():
            self.load(name, values)

    # -- steps --
    def _rows(self, rows: Sequence[Optional[Row]]):
        arr = (_Row * len(rows))()
        for i, r in enumerate(rows):
            if r is None:
                arr[i].position, arr[i].slot = SPARE, SPARE
            else:
                arr[i].position, arr[i].slot = r.position, r.slot
        return arr

    def set_rows(self, rows: Sequence[Optional[Row]], x: np.ndarray) -> None:
        x = np.ascontiguousarray(x, dtype=np.float32)
        _check(library().tgx_decoder_set_rows(self._h, self._rows(rows), len(rows), _ptr(x)))

    def start(self) -> None:
        _check(library().tgx_decoder_start(self._h))

    def wait(self) -> None:
        _check(library().tgx_decoder_wait(self._h))

    def output(self) -> np.ndarray:
        out = np.empty((self.batch.rows, self.shape.hidden), dtype=np.float32)
        _check(library().tgx_decoder_output(self._h, _ptr(out)))
        return out

    def step_rows(self, rows: Sequence[Optional[Row]], x: np.ndarray) -> np.ndarray:
        """Decoder::step_rows (decode.rs:849-853): x [rows][hidden] -> out [rows][hidden]."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty((len(rows), self.shape.hidden), dtype=np.float32)
        _check(library().tgx_decoder_step_rows(self._h, self._rows(rows), len(rows), _ptr(x), _ptr(out)))
        return out

    def step(self, position: int, x: np.ndarray) -> np.ndarray:
        """Decoder::step (decode.rs:833-837): batch 1, slot 0."""
        x = np.ascontiguousarray(x, dtype=np.float32).reshape(1, -1)
        out = np.empty((1, self.shape.hidden), dtype=np.float32)
        _check(library().tgx_decoder_step(self._h, position, _ptr(x), _ptr(out)))
        return out[0]

    def release_slot(self, slot: int) -> None:
        _check(library().tgx_decoder_release_slot(self._h, slot))

    def reserve(self, slot: int, positions: int) -> None:
        _check(library().tgx_decoder_reserve(self._h, slot, positions))

    def free_blocks(self) -> int:
        n = ctypes.c_int()
        _check(library().tgx_decoder_free_blocks(self._h, ctypes.byref(n)))
        return n.value

    def launch(self, times: int = 1, advance: bool = False) -> None:
        _check(library().tgx_decoder_launch(self._h, times, 1 if advance else 0))

    def elapsed_ms(self) -> float:
        v = ctypes.c_float()
        _check(library().tgx_decoder_elapsed_ms(self._h, ctypes.byref(v)))
        return v.value

    def set_timed(self, timed: bool) -> None:
        """Decoder::new's `timed`: launch dispatch by dispatch, each timed."""
        _check(library().tgx_decoder_set_timed(self._h, 1 if timed else 0))

    def set_graph(self, use_graph: bool) -> None:
        """Launch steps as the recorded HIP graph (default) or dispatch by dispatch."""
        _check(library().tgx_decoder_set_graph(self._h, 1 if use_graph else 0))

    def timings(self) -> list:
        """Decoder::timings (decode.rs:891-893): [(label, ms)] of the last timed step."""
        n = ctypes.c_int()
        _check(library().tgx_decoder_timings(self._h, 0, None, ctypes.byref(n)))
        arr = (_Timing * max(1, n.value))()
        _check(library().tgx_decoder_timings(self._h, n.value, arr, ctypes.byref(n)))
        return [(arr[i].label.decode(), arr[i].ms) for i in range(n.value)]

    def dispatches(self) -> int:
        v = ctypes.c_int()
        _check(library().tgx_decoder_dispatches(self._h, ctypes.byref(v)))
        return v.value

    def device_bytes(self) -> int:
        v = ctypes.c_size_t()
        _check(library().tgx_decoder_device_bytes(self._h, ctypes.byref(v)))
        return v.value

    def read_cache(self, slot: int, positions: int):
        s = self.shape
        k = np.empty((s.layers, s.kv_heads, positions, s.head_dim), dtype=np.float32)
        v = np.empty_like(k)
        _check(library().tgx_decoder_read_cache(self._h, slot, positions, _ptr(k), _ptr(v)))
        return k, v

    # -- prefill --
    def prefill(self, start: int, x: np.ndarray, slot: int = 0) -> np.ndarray:
        """Prefill::run (prefill.rs:473-503): x [len][hidden] from `start` of `slot`."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        n = x.shape[0]
        out = np.empty((n, self.shape.hidden), dtype=np.float32)
        _check(library().tgx_prefill_run(self._h, slot, start, n, _ptr(x), _ptr(out)))
        return out

    def prefill_runs(self, runs: Sequence[tuple], x: np.ndarray) -> np.ndarray:
        """Several runs (slot, start, len) at once, x their hidden states one run after another."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        arr = (_Run * len(runs))()
        for i, (slot, start, n) in enumerate(runs):
            arr[i].slot, arr[i].start, arr[i].len = slot, start, n
        out = np.empty_like(x)
        _check(library().tgx_prefill_runs(self._h, arr, len(runs), _ptr(x), _ptr(out)))
        return out

    def prefill_runs_noalloc(self, runs: Sequence[tuple], x: np.ndarray) -> np.ndarray:
        """prefill_runs with its tensors in the GPU's fixed scratch array, allocating no device
        memory (tgx_prefill_runs_noalloc): the same outputs and cache writes."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        arr = (_Run * len(runs))()
        for i, (slot, start, n) in enumerate(runs):
            arr[i].slot, arr[i].start, arr[i].len = slot, start, n
        out = np.empty_like(x)
        _check(library().tgx_prefill_runs_noalloc(self._h, arr, len(runs), _ptr(x), _ptr(out)))
        return out

    def prefill_launch(self, times: int = 1) -> None:
        """The last prefill again, `times` times, over its input on the device."""
        _check(library().tgx_prefill_launch(self._h, times))

    def close(self) -> None:
        if self._h:
            library().tgx_decoder_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass
