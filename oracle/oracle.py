"""TEST INFRASTRUCTURE ONLY — ctypes bindings of the oracle (liboracle.so, oracle.c).

Only tests/, the smoke check and the benchmark's CPU-baseline leg import this, to hold results
against or as the CPU path timed beside the GPU; the GPU library never does.
"""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "liboracle.so"

_lib = None


def library() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        lib = ctypes.CDLL(str(LIB))
        P = ctypes.c_void_p
        lib.orc_rope_tables.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_float, P, P, P]
        lib.orc_rope_tables.restype = None
        lib.orc_rmsnorm_f64.argtypes = [P, P, ctypes.c_int, ctypes.c_double, P]
        lib.orc_rmsnorm_f64.restype = None
        lib.orc_rmsnorm_f32.argtypes = [P, P, ctypes.c_int, ctypes.c_float, P]
        lib.orc_rmsnorm_f32.restype = None
        lib.orc_attention_f64.argtypes = [P, P, P] + [ctypes.c_int] * 5 + [P]
        lib.orc_attention_f64.restype = None
        for name in ("orc_decode_f64", "orc_decode_f32"):
            fn = getattr(lib, name)
            fn.argtypes = [P, P, P, P, P, ctypes.c_int, P, P]
            fn.restype = ctypes.c_int
        for name in ("orc_prefill_f64", "orc_prefill_f32"):
            fn = getattr(lib, name)
            fn.argtypes = [P, P, P, P, P, ctypes.c_int, ctypes.c_int, P, P]
            fn.restype = ctypes.c_int
        lib.orc_set_threads.argtypes = [ctypes.c_int]
        lib.orc_set_threads.restype = None
        lib.orc_threads.restype = ctypes.c_int
        _lib = lib
    return _lib


def _p(a: np.ndarray) -> ctypes.c_void_p:
    return ctypes.c_void_p(a.ctypes.data)


class _Shape(ctypes.Structure):
    _fields_ = [
        ("hidden", ctypes.c_int),
        ("inner", ctypes.c_int),
        ("heads", ctypes.c_int),
        ("kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("layers", ctypes.c_int),
        ("capacity", ctypes.c_int),
        ("eps", ctypes.c_double),
        ("rope", ctypes.c_int),
        ("cos", ctypes.c_void_p),
        ("sin", ctypes.c_void_p),
    ]


class _Layer(ctypes.Structure):
    _fields_ = [(n, ctypes.c_void_p) for n in ("input_norm", "qkv", "o", "post_norm", "gate_up", "down")]


def rope_tables(capacity: int, head_dim: int, theta: float = 10000.0, factors=None):
    cos = np.empty((capacity, head_dim // 2), dtype=np.float32)
    sin = np.empty_like(cos)
    f = None
    if factors is not None:
        f = np.ascontiguousarray(factors, dtype=np.float64)
    library().orc_rope_tables(capacity, head_dim, theta, _p(f) if f is not None else None, _p(cos), _p(sin))
    return cos, sin


def rmsnorm(x: np.ndarray, g: np.ndarray, eps: float, precision: str = "f64") -> np.ndarray:
    g = np.ascontiguousarray(g, dtype=np.float32)
    if precision == "f64":
        x = np.ascontiguousarray(x, dtype=np.float64)
        out = np.empty_like(x)
        library().orc_rmsnorm_f64(_p(x), _p(g), x.size, eps, _p(out))
    else:
        x = np.ascontiguousarray(x, dtype=np.float32)
        out = np.empty_like(x)
        library().orc_rmsnorm_f32(_p(x), _p(g), x.size, eps, _p(out))
    return out


def attention(q, k_cache, v_cache, heads, kv_heads, head_dim, position) -> np.ndarray:
    """q [heads][d], caches [kv_heads][capacity][d] (float64) -> [heads][d]."""
    q = np.ascontiguousarray(q, dtype=np.float64)
    kc = np.ascontiguousarray(k_cache, dtype=np.float64)
    vc = np.ascontiguousarray(v_cache, dtype=np.float64)
    capacity = kc.shape[1]
    out = np.empty((heads, head_dim), dtype=np.float64)
    library().orc_attention_f64(_p(q), _p(kc), _p(vc), heads, kv_heads, head_dim, capacity, position, _p(out))
    return out


class Stack:
    """A MiniCPM-4 stack on the CPU with one request's cache: `decode(position, x)` and
    `prefill(start, x)` as the GPU's, in float64 ("f64") or float32 ("f32")."""

    def __init__(self, spec, weights: dict, capacity: int, precision: str = "f64", rope: bool = True,
                 rope_factors=None, shift: int = 0):
        self.spec = spec
        self.precision = precision
        self.capacity = capacity
        self.dt = np.float64 if precision == "f64" else np.float32
        self.w = {k: np.ascontiguousarray(v, dtype=np.float32) for k, v in weights.items()}
        # A planted defect for the tests: the tables read `shift` positions on.
        self.cos, self.sin = rope_tables(capacity + shift, spec.head_dim, spec.rope_theta, rope_factors)
        self.cos = np.ascontiguousarray(self.cos[shift:])
        self.sin = np.ascontiguousarray(self.sin[shift:])
        self.shape = _Shape(spec.hidden, spec.inner, spec.heads, spec.kv_heads, spec.head_dim, spec.layers,
                            capacity, spec.eps, 1 if rope else 0, self.cos.ctypes.data, self.sin.ctypes.data)
        self.layers = (_Layer * max(1, spec.layers))()
        for l in range(spec.layers):
            L = self.layers[l]
            L.input_norm = self.w[f"layers.{l}.input_layernorm"].ctypes.data
            L.qkv = self.w[f"layers.{l}.qkv_proj"].ctypes.data
            L.o = self.w[f"layers.{l}.o_proj"].ctypes.data
            L.post_norm = self.w[f"layers.{l}.post_attention_layernorm"].ctypes.data
            L.gate_up = self.w[f"layers.{l}.gate_up_proj"].ctypes.data
            L.down = self.w[f"layers.{l}.down_proj"].ctypes.data
        self.norm = self.w["norm"]
        cache = (spec.layers, spec.kv_heads, capacity, spec.head_dim)
        self.k = np.zeros(cache, dtype=self.dt)
        self.v = np.zeros(cache, dtype=self.dt)

    def decode(self, position: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=self.dt).reshape(-1)
        out = np.empty(self.spec.hidden, dtype=self.dt)
        fn = library().orc_decode_f64 if self.precision == "f64" else library().orc_decode_f32
        rc = fn(ctypes.byref(self.shape), self.layers, _p(self.norm), _p(self.k), _p(self.v), position, _p(x), _p(out))
        if rc != 0:
            raise ValueError(f"oracle decode at {position} of {self.capacity}")
        return out

    def prefill(self, start: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=self.dt)
        out = np.empty_like(x)
        fn = library().orc_prefill_f64 if self.precision == "f64" else library().orc_prefill_f32
        rc = fn(ctypes.byref(self.shape), self.layers, _p(self.norm), _p(self.k), _p(self.v), start, x.shape[0], _p(x), _p(out))
        if rc != 0:
            raise ValueError(f"oracle prefill of {x.shape[0]} from {start} in {self.capacity}")
        return out

    def prefill_rows(self, start: int, x: np.ndarray) -> np.ndarray:
        """`prefill` restated layer by layer over all the run's positions at once, with numpy's
        float64 matrix products (prefill.rs:137-504 runs the same op order a layer at a time):
        thousands of positions in seconds where position by position takes minutes. The products
        sum in BLAS's order, so it agrees with `prefill` to float64 rounding, not bit for bit
        (tests/test_oracle.py pins it there). Runs in the stack's precision (float32 for "f32", the
        CPU baseline's); writes the caches as `prefill`."""
        dt = self.dt
        s = self.spec
        x = np.asarray(x, dtype=dt)
        n = x.shape[0]
        if start < 0 or n <= 0 or start + n > self.capacity:
            raise ValueError(f"oracle prefill of {n} from {start} in {self.capacity}")
        H, KV, d, I = s.heads, s.kv_heads, s.head_dim, s.inner
        group, half, end = H // KV, d // 2, start + n
        pos = np.arange(start, end)
        co = self.cos[pos].astype(dt)[:, None, :]  # [n][1][d/2]
        si = self.sin[pos].astype(dt)[:, None, :]
        rope = self.shape.rope != 0
        scale = dt(1.0 / np.sqrt(float(d)))
        future = np.arange(end)[None, :] > pos[:, None]  # [n][end]: keys past each position

        def norm(v, g):
            return v / np.sqrt(np.mean(v * v, axis=-1, keepdims=True) + dt(s.eps)) * g.astype(dt)

        def rotate(v):  # [n][heads][d]: a' = a cos - c sin, c' = c cos + a sin
            a, c = v[..., :half], v[..., half:]
            return np.concatenate([a * co - c * si, c * co + a * si], axis=-1)

        hs = x.copy()
        for l in range(s.layers):
            W = lambda name: self.w[f"layers.{l}.{name}"].astype(dt)
            qkv = norm(hs, self.w[f"layers.{l}.input_layernorm"]) @ W("qkv_proj").T
            q = qkv[:, : H * d].reshape(n, H, d)
            k = qkv[:, H * d : (H + KV) * d].reshape(n, KV, d)
            v = qkv[:, (H + KV) * d :].reshape(n, KV, d)
            if rope:
                q, k = rotate(q), rotate(k)
            self.k[l, :, start:end] = k.transpose(1, 0, 2)
            self.v[l, :, start:end] = v.transpose(1, 0, 2)
            att = np.empty((n, H, d), dtype=dt)
            for h in range(H):
                keys, values = self.k[l, h // group, :end], self.v[l, h // group, :end]
                sc = (q[:, h] @ keys.T) * scale
                sc[future] = -np.inf
                sc -= sc.max(axis=1, keepdims=True)
                p = np.exp(sc)
                att[:, h] = (p @ values) / p.sum(axis=1, keepdims=True)
            hs = hs + att.reshape(n, H * d) @ W("o_proj").T
            gu = norm(hs, self.w[f"layers.{l}.post_attention_layernorm"]) @ W("gate_up_proj").T
            gate, up = gu[:, :I], gu[:, I:]
            hs = hs + (gate / (dt(1.0) + np.exp(-gate)) * up) @ W("down_proj").T
        return norm(hs, self.norm)


def set_threads(n: int) -> None:
    library().orc_set_threads(n)


def threads() -> int:
    return library().orc_threads()
