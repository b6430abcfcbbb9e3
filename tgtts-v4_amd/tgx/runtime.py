"""The runtime beneath the models (include/tgx.h, tgx_alloc .. tgx_copy_regions), shaped like
crates/vulkan's: `Memory` as its Memory/Buffer (memory.rs), `kernels()` as the graph crate's
KernelInfo table (crates/graph/src/kernels.rs:27-161), `Program` as a Recording of dispatches run
as often as needed (recording.rs:116-760), `copy_regions` as copy_in / copy_out.
"""

from __future__ import annotations

import ctypes
import struct
from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import F16, F32, BF16, Shape, TgxError, _check, _opened, _ptr, _shape_struct, library

U32 = 3
DEVICE, UPLOAD, READBACK = 0, 1, 2
READ, WRITE = 0, 1
TILES_16, TILES_4, TILES_QKV, TILES_QKV128 = 0, 1, 2, 3

_DTYPES = {np.dtype(np.float32): F32, np.dtype(np.float16): F16}


class _BindingInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 24), ("access", ctypes.c_int), ("element", ctypes.c_int), ("optional", ctypes.c_int)]


class _Binding(ctypes.Structure):
    _fields_ = [("memory", ctypes.c_void_p), ("offset", ctypes.c_uint64), ("size", ctypes.c_uint64)]


class _Dispatch(ctypes.Structure):
    _fields_ = [
        ("kernel", ctypes.c_int),
        ("bindings", ctypes.POINTER(_Binding)),
        ("nbindings", ctypes.c_int),
        ("constants", ctypes.POINTER(ctypes.c_uint32)),
        ("nconstants", ctypes.c_int),
        ("groups", ctypes.c_uint32 * 3),
        ("barrier", ctypes.c_int),
    ]


class _Region(ctypes.Structure):
    _fields_ = [("src_offset", ctypes.c_uint64), ("dst_offset", ctypes.c_uint64), ("bytes", ctypes.c_uint64)]


class _Timing(ctypes.Structure):
    _fields_ = [("label", ctypes.c_char * 32), ("ms", ctypes.c_float)]


_ready = False


def _lib() -> ctypes.CDLL:
    global _ready
    lib = library()
    if _ready:
        return lib
    P, U64 = ctypes.c_void_p, ctypes.c_uint64
    lib.tgx_alloc.argtypes = [P, U64, ctypes.c_int, ctypes.POINTER(P)]
    lib.tgx_free.argtypes = [P]
    lib.tgx_memory_info.argtypes = [P, ctypes.POINTER(U64), ctypes.POINTER(ctypes.c_int)]
    lib.tgx_write.argtypes = [P, U64, P, U64]
    lib.tgx_read.argtypes = [P, U64, P, U64]
    lib.tgx_tiles_bytes.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.tgx_tiles_bytes.restype = U64
    lib.tgx_attention_tile.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.tgx_attention_tile.restype = ctypes.c_int
    lib.tgx_write_tiles.argtypes = [P, U64, P, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int]
    lib.tgx_rope_tables.argtypes = [P, P, P]
    lib.tgx_kernel_count.argtypes = []
    lib.tgx_kernel_count.restype = ctypes.c_int
    lib.tgx_kernel_find.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int)]
    lib.tgx_kernel_info.argtypes = [ctypes.c_int, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(ctypes.c_int),
                                    ctypes.POINTER(ctypes.c_int)]
    lib.tgx_kernel_binding.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(_BindingInfo)]
    lib.tgx_kernel_constant.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.POINTER(ctypes.c_char_p)]
    lib.tgx_program_begin.argtypes = [P, ctypes.c_int, ctypes.POINTER(P)]
    lib.tgx_program_launch.argtypes = [P, ctypes.POINTER(_Dispatch)]
    lib.tgx_program_end.argtypes = [P]
    lib.tgx_program_start.argtypes = [P]
    lib.tgx_program_wait.argtypes = [P]
    lib.tgx_program_run.argtypes = [P]
    lib.tgx_program_timings.argtypes = [P, ctypes.c_int, ctypes.POINTER(_Timing), ctypes.POINTER(ctypes.c_int)]
    lib.tgx_program_elapsed_ms.argtypes = [P, ctypes.POINTER(ctypes.c_float)]
    lib.tgx_program_destroy.argtypes = [P]
    lib.tgx_program_ends.argtypes = [P, ctypes.POINTER(U64)]
    lib.tgx_context_dispatch.argtypes = [P, ctypes.POINTER(_Dispatch), ctypes.POINTER(ctypes.c_float)]
    lib.tgx_program_reset.argtypes = [P, ctypes.c_int]
    lib.tgx_copy_regions.argtypes = [P, P, P, ctypes.POINTER(_Region), ctypes.c_int]
    _ready = True
    return lib


@dataclass(frozen=True)
class BindingInfo:
    name: str
    access: int
    element: int
    optional: bool


@dataclass(frozen=True)
class KernelInfo:
    """kernels.rs KernelInfo: a kernel's name, its bindings in order, and its constants in order."""

    index: int
    name: str
    bindings: tuple
    constants: tuple


def kernels() -> list:
    """Every kernel the library dispatches by name (host only: no device needed)."""
    lib = _lib()
    out = []
    for i in range(lib.tgx_kernel_count()):
        name, nb, nc = ctypes.c_char_p(), ctypes.c_int(), ctypes.c_int()
        _check(lib.tgx_kernel_info(i, ctypes.byref(name), ctypes.byref(nb), ctypes.byref(nc)))
        bindings = []
        for j in range(nb.value):
            b = _BindingInfo()
            _check(lib.tgx_kernel_binding(i, j, ctypes.byref(b)))
            bindings.append(BindingInfo(b.name.decode(), b.access, b.element, bool(b.optional)))
        constants = []
        for j in range(nc.value):
            c = ctypes.c_char_p()
            _check(lib.tgx_kernel_constant(i, j, ctypes.byref(c)))
            constants.append(c.value.decode())
        out.append(KernelInfo(i, name.value.decode(), tuple(bindings), tuple(constants)))
    return out


def kernel(name: str) -> KernelInfo:
    i = ctypes.c_int()
    _check(_lib().tgx_kernel_find(name.encode(), ctypes.byref(i)))
    return kernels()[i.value]


def tiles_bytes(tiles: int, rows: int, cols: int) -> int:
    return int(_lib().tgx_tiles_bytes(tiles, rows, cols))


def attention_tile(heads: int, kv_heads: int, head_dim: int) -> int:
    """The most positions an attention_rows tile may hold for the shape (0: not taken)."""
    return int(_lib().tgx_attention_tile(heads, kv_heads, head_dim))


def rope_tables(shape: Shape) -> tuple:
    """Shape::rope_tables (decode.rs:143-168): cos and sin [capacity][head_dim / 2] f32."""
    half = shape.head_dim // 2
    cos = np.zeros((shape.capacity, half), np.float32)
    sin = np.zeros((shape.capacity, half), np.float32)
    s, _keep = _shape_struct(shape)
    _check(_lib().tgx_rope_tables(ctypes.byref(s), _ptr(cos), _ptr(sin)))
    return cos, sin


def f32_bits(v: float) -> int:
    """An f32 constant as the u32 a dispatch carries."""
    return struct.unpack("<I", struct.pack("<f", v))[0]


class Memory:
    """Context::memory_in (context.rs:495-498): `nbytes` of zeroed memory in a residence."""

    def __init__(self, ctx, nbytes: int, residence: int = DEVICE):
        self.ctx = ctx
        self._h = ctypes.c_void_p()
        _check(_lib().tgx_alloc(ctx._h, nbytes, residence, ctypes.byref(self._h)))
        self.nbytes = nbytes
        self.residence = residence
        _opened(self)

    def write(self, data: np.ndarray, offset: int = 0) -> None:
        a = np.ascontiguousarray(data)
        _check(_lib().tgx_write(self._h, offset, _ptr(a), a.nbytes))

    def read(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.zeros(count, dtype)
        _check(_lib().tgx_read(self._h, offset, _ptr(out), out.nbytes))
        return out

    def write_tiles(self, w: np.ndarray, tiles: int, offset: int = 0) -> None:
        """A row-major [rows][cols] weight (f32 or f16; bf16 bits as uint16) as the kernels' tiles."""
        a = np.ascontiguousarray(w)
        dtype = BF16 if a.dtype == np.uint16 else _DTYPES[a.dtype]
        _check(_lib().tgx_write_tiles(self._h, offset, _ptr(a), dtype, tiles, a.shape[0], a.shape[1]))

    def binding(self, offset: int = 0, size: int = 0) -> "_Binding":
        return _Binding(self._h, offset, size)

    def close(self) -> None:
        if self._h:
            _check(_lib().tgx_free(self._h))
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            if self._h:
                _lib().tgx_free(self._h)
                self._h = ctypes.c_void_p()
        except Exception:
            pass


def _bindings(items: Sequence) -> "ctypes.Array":
    arr = (_Binding * max(1, len(items)))()
    for i, b in enumerate(items):
        if b is None:
            arr[i] = _Binding(None, 0, 0)
        elif isinstance(b, Memory):
            arr[i] = b.binding()
        elif isinstance(b, tuple):  # (memory, offset, size)
            m, off, size = (b + (0,))[:3]
            arr[i] = m.binding(off, size)
        else:
            arr[i] = b
    return arr


class Program:
    """A Recording's program (context.rs:507-518, recording.rs:116-760): dispatches added by
    `dispatch`, recorded as a HIP graph by `end`, then `run` (or `start` and `wait`) as often as
    needed. `timed`: each dispatch launched alone between events of its own (`timings`)."""

    def __init__(self, ctx, timed: bool = False):
        self.ctx = ctx
        self._h = ctypes.c_void_p()
        _check(_lib().tgx_program_begin(ctx._h, 1 if timed else 0, ctypes.byref(self._h)))
        _opened(self)

    def dispatch(self, kernel_name: str, bindings: Sequence, constants: Sequence[int], barrier: bool = True,
                 groups: tuple = (0, 0, 0)) -> None:
        k = ctypes.c_int()
        _check(_lib().tgx_kernel_find(kernel_name.encode(), ctypes.byref(k)))
        self.dispatch_index(k.value, bindings, constants, barrier, groups)

    def dispatch_index(self, kernel_index: int, bindings: Sequence, constants: Sequence[int], barrier: bool = True,
                       groups: tuple = (0, 0, 0)) -> None:
        b = _bindings(bindings)
        c = (ctypes.c_uint32 * max(1, len(constants)))(*[int(v) & 0xFFFFFFFF for v in constants])
        d = _Dispatch(kernel_index, b, len(bindings), c, len(constants), (ctypes.c_uint32 * 3)(*groups), 1 if barrier else 0)
        _check(_lib().tgx_program_launch(self._h, ctypes.byref(d)))

    def end(self) -> None:
        _check(_lib().tgx_program_end(self._h))

    def start(self) -> None:
        _check(_lib().tgx_program_start(self._h))

    def wait(self) -> None:
        _check(_lib().tgx_program_wait(self._h))

    def run(self) -> None:
        _check(_lib().tgx_program_run(self._h))

    def timings(self) -> list:
        n = ctypes.c_int()
        _check(_lib().tgx_program_timings(self._h, 0, None, ctypes.byref(n)))
        arr = (_Timing * max(1, n.value))()
        _check(_lib().tgx_program_timings(self._h, n.value, arr, ctypes.byref(n)))
        return [(arr[i].label.decode(), arr[i].ms) for i in range(n.value)]

    def elapsed_ms(self) -> float:
        v = ctypes.c_float()
        _check(_lib().tgx_program_elapsed_ms(self._h, ctypes.byref(v)))
        return v.value

    def ends(self) -> tuple:
        """Recording::ends: the GPU clock's ticks when the last run started and ended."""
        e = (ctypes.c_uint64 * 2)()
        _check(_lib().tgx_program_ends(self._h, e))
        return int(e[0]), int(e[1])

    def reset(self, timed: bool = False) -> None:
        """Recording::replace_program: drop the dispatches; new ones follow, then `end`."""
        _check(_lib().tgx_program_reset(self._h, 1 if timed else 0))

    def close(self) -> None:
        if self._h:
            _check(_lib().tgx_program_destroy(self._h))
            self._h = ctypes.c_void_p()

    def __del__(self):
        try:
            if self._h:
                _lib().tgx_program_destroy(self._h)
                self._h = ctypes.c_void_p()
        except Exception:
            pass


def dispatch(ctx, kernel_name: str, bindings: Sequence, constants: Sequence[int], groups: tuple = (0, 0, 0)) -> float:
    """Context::dispatch: one dispatch run alone and waited for; its GPU time in ms."""
    k = ctypes.c_int()
    _check(_lib().tgx_kernel_find(kernel_name.encode(), ctypes.byref(k)))
    b = _bindings(bindings)
    c = (ctypes.c_uint32 * max(1, len(constants)))(*[int(v) & 0xFFFFFFFF for v in constants])
    d = _Dispatch(k.value, b, len(bindings), c, len(constants), (ctypes.c_uint32 * 3)(*groups), 1)
    ms = ctypes.c_float()
    _check(_lib().tgx_context_dispatch(ctx._h, ctypes.byref(d), ctypes.byref(ms)))
    return ms.value


def copy_regions(ctx, dst: Memory, src: Memory, regions: Sequence[tuple]) -> None:
    """Recording::copy_in / copy_out (recording.rs:522-597): (src_offset, dst_offset, bytes) each."""
    arr = (_Region * max(1, len(regions)))(*[_Region(*r) for r in regions])
    _check(_lib().tgx_copy_regions(ctx._h, dst._h, src._h, arr, len(regions)))


__all__ = [
    "BindingInfo", "KernelInfo", "Memory", "Program", "copy_regions", "f32_bits", "kernel", "kernels", "rope_tables",
    "tiles_bytes", "attention_tile", "dispatch", "DEVICE", "UPLOAD", "READBACK", "READ", "WRITE", "TILES_16", "TILES_4", "TILES_QKV", "TILES_QKV128", "U32", "TgxError",
]
