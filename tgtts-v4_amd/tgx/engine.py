"""The engine the service's GPU thread drives (crates/tgtts/src/rt.rs:92-111 Engine,
crates/graph/src/generator.rs Generator) through libtgx's tgx_engine_*: requests in slots, each
started from its prompt, a patch of every request under way sampled in one patch step until its
stop head says to stop or its most patches are sampled. Latent frames come back where the
reference decodes audio: the audio VAE is not part of the path."""

from __future__ import annotations

import ctypes
import sys
from dataclasses import dataclass
from typing import Optional

import numpy as np

from . import Context, Shape, _check, _HeadsShape, _opened, _ptr, _shape_struct, library
from .patch import HeadsShape


class _Settings(ctypes.Structure):
    _fields_ = [("slots", ctypes.c_int), ("capacity", ctypes.c_int), ("max_rows", ctypes.c_int),
                ("timesteps", ctypes.c_int), ("prompt_cache_bytes", ctypes.c_size_t)]


class _Outcome(ctypes.Structure):
    _fields_ = [("slot", ctypes.c_int), ("status", ctypes.c_int), ("last", ctypes.c_int),
                ("stop_logits", ctypes.c_float * 2)]


@dataclass
class Settings:
    """generator::Settings (generator.rs:35-56)."""

    slots: int = 16
    capacity: int = 2048
    max_rows: int = 512
    timesteps: int = 10
    prompt_cache_bytes: int = 1 << 30


@dataclass
class Outcome:
    """generator::Outcome (generator.rs:76): the patch [patch_size][feat_dim] or the status that
    ended the request."""

    slot: int
    status: int
    last: bool
    stop_logits: tuple
    frames: Optional[np.ndarray]


class Engine:
    """Generator::new (generator.rs:130-193) over explicit shapes and a checkpoint."""

    def __init__(self, ctx: Context, checkpoint, base: Shape, residual: Shape, heads: HeadsShape, encoder: Shape,
                 dit: Shape, feat_dim: int, patch_size: int, settings: Settings = Settings()):
        self.ctx = ctx
        self.checkpoint = checkpoint  # read for token embeddings: kept alive beside the engine
        self.feat_dim, self.patch_size, self.latent = feat_dim, patch_size, heads.latent
        self.settings = settings
        structs = [_shape_struct(s) for s in (base, residual, encoder, dit)]
        self._keep = structs
        hs = _HeadsShape(heads.encoder, heads.dit, heads.latent, heads.levels)
        st = _Settings(settings.slots, settings.capacity, settings.max_rows, settings.timesteps, settings.prompt_cache_bytes)
        self._h = ctypes.c_void_p()
        b, r, e, d = (ctypes.byref(s[0]) for s in structs)
        _check(library().tgx_engine_create(ctx._h, checkpoint._h, b, r, ctypes.byref(hs), e, d, feat_dim, patch_size,
                                           ctypes.byref(st), ctypes.byref(self._h)))
        _opened(self)

    @classmethod
    def from_config(cls, ctx: Context, config, checkpoint, settings: Settings = Settings(),
                    base_layers: Optional[int] = None) -> "Engine":
        """From a tgx.config.Config as Generator::new reads config.json: the stacks derived from the
        base LM's, the heads' widths from the config."""
        from .config import shape

        base = shape(config.lm_config, base_layers, settings.capacity)
        residual = shape(config.residual_lm(), None, settings.capacity)
        encoder = shape(config.local_encoder(), None, 16)
        dit = shape(config.local_dit(), None, 16)
        heads = HeadsShape(config.encoder_config.hidden_dim, config.dit_config.hidden_dim,
                           config.scalar_quantization_latent_dim, config.scalar_quantization_scale)
        return cls(ctx, checkpoint, base, residual, heads, encoder, dit, config.feat_dim, config.patch_size, settings)

    def slots(self) -> int:
        v = ctypes.c_int()
        _check(library().tgx_engine_slots(self._h, ctypes.byref(v)))
        return v.value

    def start(self, slot: int, prompt, voice, max_patches: int, temperature: float = 1.0, cfg: float = 2.0) -> int:
        """Engine::start (rt.rs:98-100): the prompt's positions that ran through the LMs."""
        s = prompt._struct()
        v = np.ascontiguousarray(voice, dtype=np.float32)
        n = ctypes.c_int()
        _check(library().tgx_engine_start(self._h, slot, ctypes.byref(s), _ptr(v), v.size, max_patches, temperature, cfg,
                                          ctypes.byref(n)))
        return n.value

    def sample_after(self, slot: int, frames) -> None:
        f = np.ascontiguousarray(frames, dtype=np.float32)
        _check(library().tgx_engine_sample_after(self._h, slot, _ptr(f)))

    def step(self, noise) -> list:
        """Engine::step (rt.rs:102-104): noise [slots][feat_dim][patch_size]; an Outcome for each
        request under way."""
        S = self.settings.slots
        nz = np.ascontiguousarray(noise, dtype=np.float32).reshape(S, self.feat_dim, self.patch_size)
        outcomes = (_Outcome * S)()
        frames = np.zeros((S, self.patch_size, self.feat_dim), dtype=np.float32)
        n = ctypes.c_int()
        _check(library().tgx_engine_step(self._h, _ptr(nz), outcomes, _ptr(frames), ctypes.byref(n)))
        out = []
        for i in range(n.value):
            o = outcomes[i]
            out.append(Outcome(o.slot, o.status, bool(o.last), (o.stop_logits[0], o.stop_logits[1]),
                               frames[o.slot].copy() if o.status == 0 else None))
        return out

    def levels(self, slot: int) -> np.ndarray:
        out = np.empty(self.latent, dtype=np.float32)
        _check(library().tgx_engine_levels(self._h, slot, _ptr(out)))
        return out

    def _frames(self, fn, slot: int, max_frames: int) -> np.ndarray:
        out = np.empty((max_frames, self.feat_dim), dtype=np.float32)
        n = ctypes.c_int()
        _check(fn(self._h, slot, _ptr(out), max_frames, ctypes.byref(n)))
        return out[: n.value]

    def take_frames(self, slot: int, max_frames: int = 4096) -> np.ndarray:
        return self._frames(library().tgx_engine_take_frames, slot, max_frames)

    def finish(self, slot: int, max_frames: int = 4096) -> np.ndarray:
        """Engine::finish (rt.rs:106-107): the frames not yet taken."""
        return self._frames(library().tgx_engine_finish, slot, max_frames)

    def prompt_cache(self):
        b, v = ctypes.c_size_t(), ctypes.c_int()
        _check(library().tgx_engine_prompt_cache(self._h, ctypes.byref(b), ctypes.byref(v)))
        return b.value, v.value

    def close(self) -> None:
        if self._h:
            library().tgx_engine_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass
