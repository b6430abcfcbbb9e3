"""graph::prompt (crates/graph/src/prompt.rs): a prompt run into a slot of a patch step's caches, and
the PromptCache that keeps, for each voice, what its next prompts share — through libtgx
(tgx_prompter_*, tgx_prompt_cache_*)."""

from __future__ import annotations

import ctypes
import sys
from dataclasses import dataclass
import numpy as np

from . import Context, _check, _opened, _ptr, _Row, library


class _Prompt(ctypes.Structure):
    _fields_ = [("tokens", ctypes.c_void_p), ("patches", ctypes.c_void_p), ("audio", ctypes.c_void_p),
                ("len", ctypes.c_int)]


@dataclass
class Prompt:
    """prompt::Prompt (prompt.rs:322-332): each position's token (read where it is text), patch
    ([patch_size][feat_dim], read where it is audio) and whether it is audio."""

    tokens: np.ndarray
    patches: np.ndarray
    audio: np.ndarray

    def _struct(self):
        self._keep = (np.ascontiguousarray(self.tokens, dtype=np.uint32),
                      np.ascontiguousarray(self.patches, dtype=np.float32),
                      np.ascontiguousarray(self.audio, dtype=np.uint8))
        t, p, a = self._keep
        return _Prompt(t.ctypes.data, p.ctypes.data, a.ctypes.data, len(t))

    def __len__(self):
        return len(self.tokens)


class PromptCache:
    """PromptCache::new (prompt.rs:414-424): at most `budget` bytes, host and device together."""

    def __init__(self, ctx: Context, budget: int):
        self.ctx = ctx
        self._h = ctypes.c_void_p()
        _check(library().tgx_prompt_cache_create(ctx._h, budget, ctypes.byref(self._h)))
        _opened(self)

    def bytes(self) -> int:
        v = ctypes.c_size_t()
        _check(library().tgx_prompt_cache_bytes(self._h, ctypes.byref(v)))
        return v.value

    def voices(self) -> int:
        v = ctypes.c_int()
        _check(library().tgx_prompt_cache_voices(self._h, ctypes.byref(v)))
        return v.value

    def close(self) -> None:
        if self._h:
            library().tgx_prompt_cache_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass


class Prompter:
    """Prompter::new (prompt.rs:527-552) over a patch step's encoder and LM side: runs of up to
    `max_rows` positions at a time. The patch step must outlive it."""

    TENSORS = {"base_out": "hidden", "levels": "latent", "quantized": "hidden", "lm_hidden": "hidden",
               "residual_in": "hidden", "residual_out": "hidden"}

    def __init__(self, step, max_rows: int = 256):
        self.step = step
        self.ctx = step.side.ctx
        self._h = ctypes.c_void_p()
        _check(library().tgx_prompter_create(step._h, max_rows, ctypes.byref(self._h)))
        _opened(self)
        self.hidden = step.side.base_shape.hidden
        self.latent = step.side.heads.latent

    def max_rows(self) -> int:
        v = ctypes.c_int()
        _check(library().tgx_prompter_max_rows(self._h, ctypes.byref(v)))
        return v.value

    def embed(self, patch) -> np.ndarray:
        """Prompter::embed (prompt.rs:559-566): [patch_size][feat_dim] -> [hidden]."""
        p = np.ascontiguousarray(patch, dtype=np.float32)
        out = np.empty(self.hidden, dtype=np.float32)
        _check(library().tgx_prompter_embed(self._h, _ptr(p), _ptr(out)))
        return out

    def embeddings(self, checkpoint, prompt: Prompt):
        """Prompter::embeddings (prompt.rs:636-648): (x, audio_x), [len - 1][hidden] each."""
        n = max(len(prompt) - 1, 0)
        x = np.empty((n, self.hidden), dtype=np.float32)
        ax = np.empty((n, self.hidden), dtype=np.float32)
        s = prompt._struct()
        _check(library().tgx_prompter_embeddings(self._h, checkpoint._h, ctypes.byref(s), _ptr(x), _ptr(ax)))
        return x, ax

    def run_rows(self, position: int, slot: int, x, audio_x, audio) -> None:
        """Prompter::run_rows (prompt.rs:692-752)."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        ax = np.ascontiguousarray(audio_x, dtype=np.float32)
        a = np.ascontiguousarray(audio, dtype=np.uint8)
        _check(library().tgx_prompter_run_rows(self._h, _Row(position, slot), _ptr(x), _ptr(ax), _ptr(a), len(a)))

    def run(self, slot: int, checkpoint, prompt: Prompt) -> None:
        """Prompter::run (prompt.rs:568-583): every position but the last, from position 0."""
        s = prompt._struct()
        _check(library().tgx_prompter_run(self._h, slot, checkpoint._h, ctypes.byref(s)))

    def run_cached(self, slot: int, checkpoint, prompt: Prompt, voice, cache: PromptCache) -> int:
        """Prompter::run_cached (prompt.rs:585-641): the positions that ran through the LMs."""
        s = prompt._struct()
        v = np.ascontiguousarray(voice, dtype=np.float32)
        ran = ctypes.c_int()
        _check(library().tgx_prompter_run_cached(self._h, slot, checkpoint._h, ctypes.byref(s), _ptr(v), v.size,
                                                 cache._h, ctypes.byref(ran)))
        return ran.value

    def read(self, tensor: str, rows: int) -> np.ndarray:
        """The last run's last piece of `rows` rows: one of TENSORS."""
        width = self.hidden if self.TENSORS[tensor] == "hidden" else self.latent
        out = np.empty((rows, width), dtype=np.float32)
        _check(library().tgx_prompter_read(self._h, tensor.encode(), _ptr(out), out.size))
        return out

    def close(self) -> None:
        if self._h:
            library().tgx_prompter_destroy(self._h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        if sys.is_finalizing():
            return
        try:
            self.close()
        except Exception:
            pass
