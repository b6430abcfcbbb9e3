"""Python bindings of the patch sampler and the LM side (include/tgx.h), shaped like the
reference's `local::dit::Sampler` (crates/graph/src/local/dit.rs:264-318) and `lm_side::LmSide`
(crates/graph/src/lm_side.rs:544-660). Like the decoder's, they only call libtgx: nothing here
computes."""

from __future__ import annotations

import ctypes
import sys
from dataclasses import dataclass
from typing import Optional, Sequence

import numpy as np

from . import (
    BF16,
    F16,
    F32,
    SPARE,
    Context,
    Decoder,
    Row,
    Batch,
    Shape,
    _Batch,
    _HeadsShape,
    _opened,
    _PatchShape,
    _ptr,
    _Row,
    _shape_struct,
    _Timing,
    _check,
    library,
)

MU_TOKENS = 2


def _weights(values: np.ndarray):
    a = np.ascontiguousarray(values)
    if a.dtype == np.float32:
        return a, F32
    if a.dtype == np.uint16:
        return a, BF16
    if a.dtype == np.float16:
        return a, F16
    return np.ascontiguousarray(a, dtype=np.float32), F32


def euler_steps(timesteps: int) -> list:
    """euler_steps (dit.rs:61-79) as the library computes it: [(t, dt)] of each DiT evaluation."""
    n = ctypes.c_int()
    _check(library().tgx_euler_steps(timesteps, 0, None, None, ctypes.byref(n)))
    t = (ctypes.c_float * max(1, n.value))()
    dt = (ctypes.c_float * max(1, n.value))()
    _check(library().tgx_euler_steps(timesteps, n.value, t, dt, ctypes.byref(n)))
    return [(t[i], dt[i]) for i in range(n.value)]


@dataclass(frozen=True)
class PatchShape:
    """What sampler_graph takes besides the DiT's stack (dit.rs:114-131)."""

    feat_dim: int = 64
    patch_size: int = 4
    timesteps: int = 10
    rows: int = 1

    @property
    def tokens(self) -> int:
        return MU_TOKENS + 1 + 2 * self.patch_size


class Sampler:
    """local::dit::Sampler: the local DiT's weights and the sample recorded as one HIP graph."""

    def __init__(self, ctx: Context, stack: Shape, patch: PatchShape):
        self.ctx = ctx
        self.stack = stack
        self.patch = patch
        s, self._factors = _shape_struct(stack)
        p = _PatchShape(patch.feat_dim, patch.patch_size, patch.timesteps, patch.rows)
        self._h = ctypes.c_void_p()
        _check(library().tgx_sampler_create(ctx._h, ctypes.byref(s), ctypes.byref(p), ctypes.byref(self._h)))
        _opened(self)

    def load(self, name: str, values: np.ndarray) -> None:
        a, dtype = _weights(values)
        _check(library().tgx_sampler_load(self._h, name.encode(), _ptr(a), dtype, a.size))

    def load_all(self, weights: dict) -> None:
        for name, values in weights.items():
            self.load(name, values)

    def load_checkpoint(self, checkpoint) -> None:
        """load_sampler (crates/graph/src/local/dit.rs:329-365): feat_decoder.estimator.* from a tgx.checkpoint.Checkpoint."""
        _check(library().tgx_sampler_load_checkpoint(self._h, checkpoint._h))

    def _inputs(self, mu, cond, noise, sampling):
        P = self.patch
        mu = np.ascontiguousarray(mu, dtype=np.float32).reshape(P.rows, MU_TOKENS, self.stack.hidden)
        cond = np.ascontiguousarray(cond, dtype=np.float32).reshape(P.rows, P.feat_dim, P.patch_size)
        noise = np.ascontiguousarray(noise, dtype=np.float32).reshape(P.rows, P.feat_dim, P.patch_size)
        sampling = np.ascontiguousarray(sampling, dtype=np.float32).reshape(P.rows, 2)
        return mu, cond, noise, sampling

    def sample(self, mu, cond, noise, sampling) -> np.ndarray:
        """Sampler::sample (dit.rs:294-309): each row's patch [feat_dim][patch_size]."""
        mu, cond, noise, sampling = self._inputs(mu, cond, noise, sampling)
        out = np.empty_like(noise)
        _check(library().tgx_sampler_sample(self._h, _ptr(mu), _ptr(cond), _ptr(noise), _ptr(sampling), _ptr(out)))
        return out

    def launch(self, times: int = 1) -> None:
        _check(library().tgx_sampler_launch(self._h, times))

    def wait(self) -> None:
        _check(library().tgx_sampler_wait(self._h))

    def elapsed_ms(self) -> float:
        v = ctypes.c_float()
        _check(library().tgx_sampler_elapsed_ms(self._h, ctypes.byref(v)))
        return v.value

    def set_timed(self, timed: bool) -> None:
        _check(library().tgx_sampler_set_timed(self._h, 1 if timed else 0))

    def timings(self) -> list:
        n = ctypes.c_int()
        _check(library().tgx_sampler_timings(self._h, 0, None, ctypes.byref(n)))
        arr = (_Timing * max(1, n.value))()
        _check(library().tgx_sampler_timings(self._h, n.value, arr, ctypes.byref(n)))
        return [(arr[i].label.decode(), arr[i].ms) for i in range(n.value)]

    def dispatches(self) -> int:
        v = ctypes.c_int()
        _check(library().tgx_sampler_dispatches(self._h, ctypes.byref(v)))
        return v.value

    def close(self) -> None:
        if self._h:
            library().tgx_sampler_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


@dataclass(frozen=True)
class HeadsShape:
    """LmSideShape's widths besides the LMs' (lm_side.rs:59-72)."""

    encoder: int = 1024
    dit: int = 1024
    latent: int = 256
    levels: int = 9


class LmSide:
    """lm_side::LmSide: both LMs' decoders over one batch and the layers between them."""

    TENSORS = ("embed", "base_out", "levels", "lm_hidden", "residual_in", "residual_out", "stop_hidden", "mu",
               "stop_logits")

    def __init__(self, ctx: Context, base: Shape, residual: Shape, batch: Batch, heads: HeadsShape = HeadsShape()):
        self.ctx = ctx
        self.base_shape = base
        self.residual_shape = residual
        self.batch = batch
        self.heads = heads
        b, self._fb = _shape_struct(base)
        r, self._fr = _shape_struct(residual)
        bt = _Batch(batch.rows, batch.slots, batch.block_tokens, batch.blocks)
        hs = _HeadsShape(heads.encoder, heads.dit, heads.latent, heads.levels)
        self._h = ctypes.c_void_p()
        _check(library().tgx_lm_side_create(ctx._h, ctypes.byref(b), ctypes.byref(r), ctypes.byref(bt), ctypes.byref(hs),
                                            ctypes.byref(self._h)))
        _opened(self)

    def load(self, name: str, values: np.ndarray) -> None:
        a, dtype = _weights(values)
        _check(library().tgx_lm_side_load(self._h, name.encode(), _ptr(a), dtype, a.size))

    def load_all(self, weights: dict) -> None:
        for name, values in weights.items():
            self.load(name, values)

    def load_checkpoint(self, checkpoint) -> None:
        """load_lm_side (crates/graph/src/lm_side.rs:496-533): base_lm.*, residual_lm.* and the heads from a tgx.checkpoint.Checkpoint."""
        _check(library().tgx_lm_side_load_checkpoint(self._h, checkpoint._h))

    def decoder(self, which: int) -> Decoder:
        """The base LM's (0) or the residual LM's (1) decoder, owned by the LM side."""
        h = ctypes.c_void_p()
        _check(library().tgx_lm_side_decoder(self._h, which, ctypes.byref(h)))
        d = Decoder.__new__(Decoder)
        d.ctx = self.ctx
        d.shape = self.base_shape if which == 0 else self.residual_shape
        d.batch = self.batch
        d._factors = None
        d._h = h
        return d

    def _rows(self, rows: Sequence[Optional[Row]]):
        arr = (_Row * len(rows))()
        for i, r in enumerate(rows):
            arr[i].position, arr[i].slot = (SPARE, SPARE) if r is None else (r.position, r.slot)
        return arr

    def step_rows(self, rows: Sequence[Optional[Row]], enc: np.ndarray):
        """LmSide::step_rows (lm_side.rs:599-625): enc [rows][encoder] -> (mu [rows][2 dit],
        stop logits [rows][2])."""
        enc = np.ascontiguousarray(enc, dtype=np.float32)
        mu = np.empty((len(rows), 2 * self.heads.dit), dtype=np.float32)
        stop = np.empty((len(rows), 2), dtype=np.float32)
        _check(library().tgx_lm_side_step(self._h, self._rows(rows), len(rows), _ptr(enc), _ptr(mu), _ptr(stop)))
        return mu, stop

    def set_rows(self, rows: Sequence[Optional[Row]], enc: Optional[np.ndarray]) -> None:
        e = None if enc is None else np.ascontiguousarray(enc, dtype=np.float32)
        _check(library().tgx_lm_side_set_rows(self._h, self._rows(rows), len(rows), None if e is None else _ptr(e)))

    def launch(self, times: int = 1, advance: bool = False) -> None:
        _check(library().tgx_lm_side_launch(self._h, times, 1 if advance else 0))

    def wait(self) -> None:
        _check(library().tgx_lm_side_wait(self._h))

    def elapsed_ms(self) -> float:
        v = ctypes.c_float()
        _check(library().tgx_lm_side_elapsed_ms(self._h, ctypes.byref(v)))
        return v.value

    def read(self, tensor: str) -> np.ndarray:
        R, h = self.batch.rows, self.base_shape.hidden
        width = {"levels": self.heads.latent, "mu": 2 * self.heads.dit, "stop_logits": 2}.get(tensor, h)
        out = np.empty((R, width), dtype=np.float32)
        _check(library().tgx_lm_side_read(self._h, tensor.encode(), _ptr(out), out.size))
        return out

    def dispatches(self) -> int:
        v = ctypes.c_int()
        _check(library().tgx_lm_side_dispatches(self._h, ctypes.byref(v)))
        return v.value

    def close(self) -> None:
        if self._h:
            library().tgx_lm_side_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


def patch_launch(side: LmSide, sampler: Sampler, times: int = 1) -> None:
    """`times` patch steps back to back over what the device holds: the LM side (rows moving on a
    position each step), then the sampler on its mu (patch.rs:356-415, without the local encoder).
    side.wait() waits; patch_elapsed_ms(side) times them."""
    _check(library().tgx_patch_launch(side._h, sampler._h, times))


def patch_elapsed_ms(side: LmSide) -> float:
    v = ctypes.c_float()
    _check(library().tgx_patch_elapsed_ms(side._h, ctypes.byref(v)))
    return v.value


class Encoder:
    """local::encoder::Encoder (crates/graph/src/local/encoder.rs:164-198): each row's patch to
    its embedding through the local encoder's stack, recorded as one HIP graph."""

    def __init__(self, ctx: Context, stack: Shape, patch: PatchShape):
        self.ctx = ctx
        self.stack = stack
        self.patch = patch
        s, self._factors = _shape_struct(stack)
        p = _PatchShape(patch.feat_dim, patch.patch_size, patch.timesteps, patch.rows)
        self._h = ctypes.c_void_p()
        _check(library().tgx_encoder_create(ctx._h, ctypes.byref(s), ctypes.byref(p), ctypes.byref(self._h)))
        _opened(self)

    def load(self, name: str, values: np.ndarray) -> None:
        a, dtype = _weights(values)
        _check(library().tgx_encoder_load(self._h, name.encode(), _ptr(a), dtype, a.size))

    def load_all(self, weights: dict) -> None:
        for name, values in weights.items():
            self.load(name, values)

    def load_checkpoint(self, checkpoint) -> None:
        """load_encoder (crates/graph/src/local/encoder.rs:129-162): feat_encoder.* from a tgx.checkpoint.Checkpoint."""
        _check(library().tgx_encoder_load_checkpoint(self._h, checkpoint._h))

    def encode(self, patches) -> np.ndarray:
        """Encoder::encode (encoder.rs:194-198): [rows][feat_dim][patch_size] -> [rows][hidden]."""
        P = self.patch
        patches = np.ascontiguousarray(patches, dtype=np.float32).reshape(P.rows, P.feat_dim, P.patch_size)
        out = np.empty((P.rows, self.stack.hidden), dtype=np.float32)
        _check(library().tgx_encoder_encode(self._h, _ptr(patches), _ptr(out)))
        return out

    def dispatches(self) -> int:
        v = ctypes.c_int()
        _check(library().tgx_encoder_dispatches(self._h, ctypes.byref(v)))
        return v.value

    def close(self) -> None:
        if self._h:
            library().tgx_encoder_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


class PatchStep:
    """patch::PatchStep (crates/graph/src/patch.rs:98-166, 356-415) over an encoder, an LM side and
    a sampler made alike: each step embeds the patches before, steps the LM side on them and
    samples on its mu, on the device throughout. The three must outlive it."""

    def __init__(self, encoder: Encoder, side: "LmSide", sampler: Sampler):
        self.encoder, self.side, self.sampler = encoder, side, sampler
        self.ctx = side.ctx
        self._h = ctypes.c_void_p()
        _check(library().tgx_patch_step_create(encoder._h, side._h, sampler._h, ctypes.byref(self._h)))
        _opened(self)

    def run_rows(self, rows: Sequence[Optional[Row]], cond, noise, sampling):
        """PatchStep::run_rows (patch.rs:356-415): up to the step's rows, run on its program of the
        fewest rows that holds them -> (patches [rows][feat_dim][patch_size], stop logits
        [rows][2])."""
        P = self.sampler.patch
        n = len(rows)
        cond = np.ascontiguousarray(cond, dtype=np.float32).reshape(n, P.feat_dim, P.patch_size)
        noise = np.ascontiguousarray(noise, dtype=np.float32).reshape(n, P.feat_dim, P.patch_size)
        sampling = np.ascontiguousarray(sampling, dtype=np.float32).reshape(n, 2)
        patch = np.empty_like(noise)
        stop = np.empty((n, 2), dtype=np.float32)
        _check(library().tgx_patch_step_run(self._h, self.side._rows(rows), len(rows), _ptr(cond), _ptr(noise),
                                            _ptr(sampling), _ptr(patch), _ptr(stop)))
        return patch, stop

    def launch(self, times: int = 1, advance: bool = True) -> None:
        _check(library().tgx_patch_step_launch(self._h, times, 1 if advance else 0))

    def wait(self) -> None:
        _check(library().tgx_patch_step_wait(self._h))

    def elapsed_ms(self) -> float:
        v = ctypes.c_float()
        _check(library().tgx_patch_step_elapsed_ms(self._h, ctypes.byref(v)))
        return v.value

    def close(self) -> None:
        if self._h:
            library().tgx_patch_step_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass
