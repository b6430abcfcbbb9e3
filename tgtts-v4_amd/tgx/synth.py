"""Seeded synthetic inputs: one stream of standard normals per tensor name, and the MiniCPM-4
stacks' weights drawn from them (no checkpoint is available offline).

A tensor's values depend only on (seed, name, count): the stream is numpy's PCG64 seeded with
splitmix64(seed xor fnv1a64(name)), drawing standard normals (numpy's ziggurat) in float64.
"""

from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache

import numpy as np

GOLDEN = np.uint64(0x9E3779B97F4A7C15)
M1 = np.uint64(0xBF58476D1CE4E5B9)
M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * M1
        z = (z ^ (z >> np.uint64(27))) * M2
        return z ^ (z >> np.uint64(31))


def fnv1a64(name: str) -> int:
    h = 0xCBF29CE484222325
    for byte in name.encode():
        h ^= byte
        h = (h * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def stream_seed(seed: int, name: str) -> int:
    s = np.array([(seed ^ fnv1a64(name)) & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64)
    with np.errstate(over="ignore"):
        return int(_mix(s + GOLDEN)[0])


def normal(seed: int, name: str, n: int, dtype=np.float64) -> np.ndarray:
    """n standard normals from the stream of (seed, name)."""
    gen = np.random.Generator(np.random.PCG64(stream_seed(seed, name)))
    return gen.standard_normal(n, dtype=dtype)


def bf16_round(a: np.ndarray) -> np.ndarray:
    """float32 values rounded to the nearest bf16 (ties to even), as float32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    u = a.view(np.uint32)
    r = (u >> np.uint32(16)) & np.uint32(1)
    r += np.uint32(0x7FFF)
    r += u
    r &= np.uint32(0xFFFF0000)
    out = r.view(np.float32)
    nan = np.isnan(a)
    if nan.any():
        out[nan] = np.float32(np.nan)
    return out


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """The bf16 bits (uint16) of bf16_round(a)."""
    return (bf16_round(a).view(np.uint32) >> np.uint32(16)).astype(np.uint16)


@dataclass(frozen=True)
class StackSpec:
    """A MiniCPM-4 stack's shape and how its weights are drawn."""

    hidden: int = 1024
    inner: int = 4096
    heads: int = 16
    kv_heads: int = 2
    head_dim: int = 64
    layers: int = 24
    eps: float = 1e-5
    rope_theta: float = 10000.0
    std: float = 0.02
    # Norm gains: 1 + gain_std * N(0, 1). Gains drawn N(0, 0.02) as the projections are would
    # shrink every activation fifty-fold per norm.
    gain_std: float = 0.02
    seed: int = 0
    # "f32": weights as drawn (in float32); "bf16": rounded to bf16.
    dtype: str = "bf16"

    @property
    def qkv_rows(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim


def layer_names(l: int) -> list[str]:
    return [
        f"layers.{l}.input_layernorm",
        f"layers.{l}.qkv_proj",
        f"layers.{l}.o_proj",
        f"layers.{l}.post_attention_layernorm",
        f"layers.{l}.gate_up_proj",
        f"layers.{l}.down_proj",
    ]


def tensor_shape(spec: StackSpec, name: str) -> tuple[int, ...]:
    h, i = spec.hidden, spec.inner
    if name == "norm" or name.endswith("layernorm"):
        return (h,)
    if name.endswith("qkv_proj"):
        return (spec.qkv_rows, h)
    if name.endswith("o_proj"):
        return (h, spec.heads * spec.head_dim)
    if name.endswith("gate_up_proj"):
        return (2 * i, h)
    if name.endswith("down_proj"):
        return (h, i)
    raise KeyError(name)


def weight(spec: StackSpec, name: str) -> np.ndarray:
    """The float32 values of one tensor (bf16-rounded when spec.dtype is "bf16")."""
    shape = tensor_shape(spec, name)
    n = int(np.prod(shape))
    z = normal(spec.seed, name, n, np.float32)
    if len(shape) == 1:
        v = np.float32(1.0) + np.float32(spec.gain_std) * z
    else:
        v = np.float32(spec.std) * z
    v = v.astype(np.float32).reshape(shape)
    if spec.dtype == "bf16":
        v = bf16_round(v)
    return v


@lru_cache(maxsize=4)
def stack_weights(spec: StackSpec) -> dict:
    """Every tensor of the stack by name, as Decoder.load takes them (float32 arrays)."""
    out = {}
    for l in range(spec.layers):
        for name in layer_names(l):
            out[name] = weight(spec, name)
    out["norm"] = weight(spec, "norm")
    return out


def embeddings(seed: int, name: str, rows: int, hidden: int) -> np.ndarray:
    """Seeded N(0, 1) hidden states [rows][hidden] in float32."""
    return normal(seed, name, rows * hidden).astype(np.float32).reshape(rows, hidden)


def linear_layer(seed: int, name: str, n: int, k: int, std: float = 0.02, bias: bool = True, dtype: str = "bf16") -> dict:
    """A linear layer's weight [n][k] and bias [n], N(0, std), bf16-rounded when dtype is "bf16"."""
    out = {}
    w = (np.float32(std) * normal(seed, f"{name}.weight", n * k, np.float32)).astype(np.float32).reshape(n, k)
    out[f"{name}.weight"] = bf16_round(w) if dtype == "bf16" else w
    if bias:
        b = (np.float32(std) * normal(seed, f"{name}.bias", n, np.float32)).astype(np.float32)
        out[f"{name}.bias"] = bf16_round(b) if dtype == "bf16" else b
    return out


@lru_cache(maxsize=4)
def sampler_weights(stack: StackSpec, feat_dim: int = 64) -> dict:
    """The local DiT's tensors by the names Sampler.load takes: the stack's, in_proj and cond_proj
    ([hidden][feat_dim]), out_proj ([feat_dim][hidden]) and the two time MLPs."""
    out = dict(stack_weights(stack))
    h, s = stack.hidden, stack.seed
    out.update(linear_layer(s, "in_proj", h, feat_dim, dtype=stack.dtype))
    out.update(linear_layer(s, "cond_proj", h, feat_dim, dtype=stack.dtype))
    out.update(linear_layer(s, "out_proj", feat_dim, h, dtype=stack.dtype))
    for m in ("time_mlp", "delta_time_mlp"):
        out.update(linear_layer(s, f"{m}.linear_1", h, h, dtype=stack.dtype))
        out.update(linear_layer(s, f"{m}.linear_2", h, h, dtype=stack.dtype))
    return out


def encoder_weights(stack: StackSpec, feat_dim: int = 64) -> dict:
    """The local encoder's tensors by the names Encoder.load takes: the stack's, the learned token
    ("special_token" [hidden], N(0, 1)) and in_proj ([hidden][feat_dim])."""
    out = dict(stack_weights(stack))
    h, s = stack.hidden, stack.seed
    out.update(linear_layer(s, "in_proj", h, feat_dim, dtype=stack.dtype))
    special = normal(s, "special_token", h, np.float32).astype(np.float32)
    out["special_token"] = bf16_round(special) if stack.dtype == "bf16" else special
    return out


HEADS = (
    # name, out, in (as multiples of: h hidden, e encoder, d dit, l latent), bias
    ("enc_to_lm_proj", "h", "e", True),
    ("fsq_layer.in_proj", "l", "h", True),
    ("fsq_layer.out_proj", "h", "l", True),
    ("fusion_concat_proj", "h", "2h", True),
    ("lm_to_dit_proj", "d", "h", True),
    ("res_to_dit_proj", "d", "h", True),
    ("stop_proj", "h", "h", True),
    ("stop_head", "2", "h", False),
)


def heads_weights(seed: int, hidden: int, encoder: int, dit: int, latent: int, dtype: str = "bf16") -> dict:
    """The layers between the LMs (lm_side.rs:113-141), N(0, 0.02)."""
    size = {"h": hidden, "e": encoder, "d": dit, "l": latent, "2h": 2 * hidden, "2": 2}
    out = {}
    for name, n, k, bias in HEADS:
        out.update(linear_layer(seed, name, size[n], size[k], bias=bias, dtype=dtype))
    return out


def lm_side_weights(base: StackSpec, residual: StackSpec, encoder: int, dit: int, latent: int) -> dict:
    """Every tensor of the LM side by the names LmSide.load takes."""
    out = {f"base_lm.{k}": v for k, v in stack_weights(base).items()}
    out.update({f"residual_lm.{k}": v for k, v in stack_weights(residual).items()})
    out.update(heads_weights(base.seed + 7, base.hidden, encoder, dit, latent, base.dtype))
    return out
