"""graph::checkpoint (crates/graph/src/checkpoint.rs): a safetensors file read a tensor at a time,
through libtgx's reader (tgx_checkpoint_*), which the model loaders take to write a checkpoint's
tensors under the names the reference's loaders read them by."""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import numpy as np

from . import _check, _ptr, library

_DTYPES = {0: "F32", 1: "BF16", 2: "F16"}


class Checkpoint:
    """Checkpoint::open (checkpoint.rs:36-71): the header parsed and checked on opening; each
    tensor's bytes read from its offsets when asked for."""

    def __init__(self, path: str):
        self.path = str(path)
        self._h = ctypes.c_void_p()
        _check(library().tgx_checkpoint_open(self.path.encode(), ctypes.byref(self._h)))

    def names(self) -> list:
        """The tensors' names, sorted (the header is read into a BTreeMap, checkpoint.rs:31)."""
        lib = library()
        n = ctypes.c_int()
        _check(lib.tgx_checkpoint_count(self._h, ctypes.byref(n)))
        out = []
        buf = ctypes.create_string_buffer(1024)
        for i in range(n.value):
            _check(lib.tgx_checkpoint_name(self._h, i, buf, len(buf)))
            out.append(buf.value.decode())
        return out

    def _shape(self, name: str):
        dims = (ctypes.c_int64 * 8)()
        nd = ctypes.c_int()
        dt = ctypes.c_int()
        _check(library().tgx_checkpoint_shape(self._h, name.encode(), dims, 8, ctypes.byref(nd), ctypes.byref(dt)))
        return tuple(int(dims[i]) for i in range(nd.value)), _DTYPES[dt.value]

    def shape(self, name: str) -> Optional[tuple]:
        """Checkpoint::shape (checkpoint.rs:74-76): None when the file has no such tensor."""
        if name not in self.names():
            return None
        return self._shape(name)[0]

    def dtype(self, name: str) -> str:
        return self._shape(name)[1]

    def f32(self, name: str) -> np.ndarray:
        """Checkpoint::f16 (checkpoint.rs:106-125) in f32, exact from BF16 and F16, shaped."""
        shape, _ = self._shape(name)
        out = np.empty(int(np.prod(shape, dtype=np.int64)), dtype=np.float32)
        _check(library().tgx_checkpoint_read(self._h, name.encode(), _ptr(out), out.size))
        return out.reshape(shape)

    def gather(self, name: str, rows: Sequence[int]) -> np.ndarray:
        """Checkpoint::gather_f16 (checkpoint.rs:127-139) in f32: those rows of a 2-D tensor alone."""
        shape, _ = self._shape(name)
        cols = shape[1] if len(shape) == 2 else 0
        idx = np.ascontiguousarray(rows, dtype=np.int64)
        out = np.empty((len(idx), cols), dtype=np.float32)
        _check(library().tgx_checkpoint_gather(self._h, name.encode(), _ptr(idx), len(idx), _ptr(out)))
        return out

    def close(self) -> None:
        if self._h:
            library().tgx_checkpoint_close(self._h)
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
