"""TEST INFRASTRUCTURE ONLY — the oracle of the patch sampler and the LM side, in numpy float64.

A CPU restatement of what runs around the LMs for each patch:

  schedule, euler_steps   crates/graph/src/local/dit.rs:44-79, in float32 with libm's cosf, as
                          the reference computes them on the host
  time_embedding          dit.rs:367-381 (float32 recipe with libm's expf/sinf/cosf)
  time_mlp                dit.rs:390-422, linear_2(SiLU(linear_1(x))) in float64
  encode                  crates/graph/src/local/encoder.rs:42-128: the learned token and
                          in_proj of the patch's frames through the local stack, the learned
                          token's output
  local_stack             crates/graph/src/local/mod.rs:549-656 with local_{norm,qkv_rope,
                          attention,partial,add_norm,gate_up}.comp: a bidirectional MiniCPM-4
                          stack over sequences of T tokens, RoPE at each token's place m % T
  sample                  dit.rs:178-258 with local_embed.comp, cfm_noise.comp:14-18 and
                          dit_euler.comp:81-110 (CFG-Zero* guidance, the Euler step)
  quantize, linear        gemv_linear.comp:40-61 (none / SiLU / the scalar quantizer)
  lm_side_step            crates/graph/src/lm_side.rs:385-478: enc_to_lm_proj, the base LM,
                          fsq in/out, fusion_concat_proj, lm_to_dit / res_to_dit, stop head

Only tests/, the smoke check and the benchmark's CPU-baseline leg import this, to hold results
against; the GPU library never does.

Pinning (tests/test_patch_oracle.py): the schedule's closed-form ends (t_span[0] = 1,
t_span[n] = 0), its 9 evaluations for 10 steps and the zero-init count for other step counts;
the time embedding's t = 0 closed form; CFG-Zero*'s reductions (guidance 1 gives the conditional
velocity, equal velocities give it back, a zero unconditional velocity gives cfg v_c); the
quantizer's special cases (0, saturation, ties to even, levels on the 1/L grid); the local
stack against an independent torch float64 model built from library ops
(scaled_dot_product_attention without a mask, silu, rms_norm by hand); time_mlp and the layers
between the LMs against torch's linear and silu (a transposed weight must fail); the whole
sampler against the closed form it takes when out_proj reads nothing; and the DiT's sequence
(mu 0..1 in the conditional sequence only, time 2, cond 3..6, x 7..10, the velocity read from x):
one Euler step against the sequence assembled by hand through the torch model, the velocity of
x alone when the stack is made per-token, mu moving v_c and not v_u; planted layouts (cond and x
traded, the velocity read from cond, mu in both sequences) fail them.
"""

from __future__ import annotations

import ctypes
import ctypes.util
from dataclasses import dataclass

import numpy as np

import oracle

MU_TOKENS = 2
TIME_AT = MU_TOKENS
COND_AT = TIME_AT + 1

_libm = ctypes.CDLL(ctypes.util.find_library("m"))
for _f in ("cosf", "sinf", "expf"):
    getattr(_libm, _f).argtypes = [ctypes.c_float]
    getattr(_libm, _f).restype = ctypes.c_float


def _f32(v) -> np.float32:
    return np.float32(v)


def schedule(timesteps: int) -> np.ndarray:
    """t_span (dit.rs:44-58): linspace(1, 0, n + 1) as torch builds it in float32 (the first half
    from 1, the second from 0), then t + (cos(pi t / 2) - 1 + t), in float32."""
    steps = timesteps + 1
    step = _f32(_f32(0.0 - 1.0) / _f32(timesteps))
    out = np.empty(steps, dtype=np.float32)
    half_pi = _f32(np.pi / 2)
    for i in range(steps):
        if i < steps // 2:
            t = _f32(_f32(1.0) + _f32(step * _f32(i)))
        else:
            t = _f32(_f32(0.0) - _f32(step * _f32(steps - i - 1)))
        c = _f32(_libm.cosf(float(_f32(half_pi * t))))
        out[i] = _f32(t + _f32(_f32(c - _f32(1.0)) + t))
    return out


def euler_steps(timesteps: int) -> list:
    """(t, dt) of each DiT evaluation (dit.rs:61-79): the first max(1, floor(0.04 len)) steps
    run nothing; t -= dt and dt = t - t_span[step + 1] in float32."""
    span = schedule(max(timesteps, 1))
    zero_init = max(1, int(len(span) * 0.04))
    t, dt = span[0], _f32(span[0] - span[1])
    out = []
    for step in range(1, len(span)):
        if step > zero_init:
            out.append((float(t), float(dt)))
        t = _f32(t - dt)
        if step < len(span) - 1:
            dt = _f32(t - span[step + 1])
    return out


def time_embedding(t: float, hidden: int) -> np.ndarray:
    """SinusoidalPosEmb at scale 1000 in float32 (dit.rs:367-381): sines then cosines."""
    half = hidden // 2
    rate = _f32(-(np.log(10000.0) / (half - 1)))
    scaled = _f32(_f32(t) * _f32(1000.0))
    out = np.empty(hidden, dtype=np.float64)
    for i in range(half):
        angle = _f32(scaled * _f32(_libm.expf(float(_f32(_f32(i) * rate)))))
        out[i] = float(_libm.sinf(float(angle)))
        out[half + i] = float(_libm.cosf(float(angle)))
    return out


def time_mlp(w: dict, prefix: str, x: np.ndarray) -> np.ndarray:
    """linear_2(SiLU(linear_1(x))) in float64 (dit.rs:409-421)."""
    g = lambda n: np.asarray(w[f"{prefix}.{n}"], dtype=np.float64)
    inner = g("linear_1.weight") @ x + g("linear_1.bias")
    inner = inner / (1.0 + np.exp(-inner))
    return g("linear_2.weight") @ inner + g("linear_2.bias")


def time_tokens(w: dict, timesteps: int, hidden: int) -> np.ndarray:
    """Each evaluation's time token: time_mlp(emb(t)) + delta_time_mlp(emb(0)) (dit.rs:351-364)."""
    const = time_mlp(w, "delta_time_mlp", time_embedding(0.0, hidden))
    return np.stack([time_mlp(w, "time_mlp", time_embedding(t, hidden)) + const for t, _ in euler_steps(timesteps)])


def rmsnorm(x: np.ndarray, g: np.ndarray, eps: float) -> np.ndarray:
    return x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps) * np.asarray(g, dtype=np.float64)


def rope(v: np.ndarray, cos: np.ndarray, sin: np.ndarray) -> np.ndarray:
    """Rotate-half RoPE of [..., T, heads, d] at the rows' places (cos/sin [T][d/2])."""
    half = v.shape[-1] // 2
    a, c = v[..., :half], v[..., half:]
    co = cos[:, None, :].astype(np.float64)
    si = sin[:, None, :].astype(np.float64)
    return np.concatenate([a * co - c * si, c * co + a * si], axis=-1)


@dataclass
class StackShape:
    hidden: int = 1024
    inner: int = 4096
    heads: int = 16
    kv_heads: int = 2
    head_dim: int = 64
    layers: int = 4
    eps: float = 1e-5
    rope_theta: float = 10000.0


def local_stack(w: dict, s, x: np.ndarray, T: int, rope_on: bool = True) -> np.ndarray:
    """The local stack over x [seqs * T][hidden] (float64), every token attending to its whole
    sequence; returns the last layer's output after the final norm."""
    M, h = x.shape
    seqs = M // T
    H, KV, d = s.heads, s.kv_heads, s.head_dim
    cos, sin = oracle.rope_tables(T, d, s.rope_theta)
    x = np.asarray(x, dtype=np.float64)
    W = lambda n: np.asarray(w[n], dtype=np.float64)
    for l in range(s.layers):
        n = rmsnorm(x, w[f"layers.{l}.input_layernorm"], s.eps)
        qkv = n @ W(f"layers.{l}.qkv_proj").T
        q = qkv[:, : H * d].reshape(seqs, T, H, d)
        k = qkv[:, H * d : (H + KV) * d].reshape(seqs, T, KV, d)
        v = qkv[:, (H + KV) * d :].reshape(seqs, T, KV, d)
        if rope_on:
            q, k = rope(q, cos, sin), rope(k, cos, sin)
        group = H // KV
        kk = np.repeat(k, group, axis=2)  # [seqs][T][H][d]
        vv = np.repeat(v, group, axis=2)
        scores = np.einsum("sthd,sjhd->shtj", q, kk) / np.sqrt(d)
        scores -= scores.max(axis=-1, keepdims=True)
        p = np.exp(scores)
        p /= p.sum(axis=-1, keepdims=True)
        att = np.einsum("shtj,sjhd->sthd", p, vv).reshape(M, H * d)
        x = x + att @ W(f"layers.{l}.o_proj").T
        n = rmsnorm(x, w[f"layers.{l}.post_attention_layernorm"], s.eps)
        gu = n @ W(f"layers.{l}.gate_up_proj").T
        gate, up = gu[:, : s.inner], gu[:, s.inner :]
        x = x + (gate / (1.0 + np.exp(-gate)) * up) @ W(f"layers.{l}.down_proj").T
    return rmsnorm(x, w["norm"], s.eps)


def encode(w: dict, s, feat: int, frames: int, patches) -> np.ndarray:
    """VoxCPMLocEnc for each row (crates/graph/src/local/encoder.rs:42-128): the learned token,
    then in_proj of the patch's frames, through the local stack (a sequence of 1 + frames tokens
    to a row); the learned token's output after the final norm, [rows][hidden] float64."""
    patches = np.asarray(patches, dtype=np.float64).reshape(-1, feat, frames)
    rows, h = patches.shape[0], s.hidden
    W = lambda n: np.asarray(w[n], dtype=np.float64)
    tokens = np.zeros((rows, 1 + frames, h))
    tokens[:, 0] = W("special_token")
    tokens[:, 1:] = (W("in_proj.weight") @ patches).transpose(0, 2, 1) + W("in_proj.bias")
    out = local_stack(w, s, tokens.reshape(rows * (1 + frames), h), 1 + frames).reshape(rows, 1 + frames, h)
    return out[:, 0]


def cfg_zero_star(v_c: np.ndarray, v_u: np.ndarray, cfg: float) -> np.ndarray:
    """dit_euler.comp:81-110: alpha = <v_c, v_u> / (|v_u|^2 + 1e-8), guided = alpha v_u +
    cfg (v_c - alpha v_u)."""
    alpha = np.sum(v_c * v_u) / (np.sum(v_u * v_u) + 1e-8)
    scaled = v_u * alpha
    return scaled + cfg * (v_c - scaled)


def layout(frames: int) -> dict:
    """Where each part of the DiT's sequence sits (dit.rs:36-41): mu at tokens 0..1 (in the
    conditional sequence only), the time token at 2, the patch before (cond) at 3..3 + frames - 1,
    the state x after it; the velocity is read from x's tokens."""
    x_at = COND_AT + frames
    return {"mu": 0, "time": TIME_AT, "cond": COND_AT, "x": x_at, "read": x_at}


def sample(w: dict, s, feat: int, frames: int, timesteps: int, mu, cond, noise, sampling, rope_on: bool = True,
           places: dict | None = None, velocities: bool = False):
    """Sampler::sample (dit.rs:178-258, 294-309) for every row: returns (x0, patch), each
    [rows][feat][frames] float64, x0 the starting point temperature * noise; with `velocities`
    also each evaluation's (v_c, v_u), [evaluations][rows][2][feat][frames]. `places` overrides
    `layout` (the tests plant a misplaced sequence with it; "mu_both" puts mu in both sequences)."""
    rows = noise.shape[0]
    T = COND_AT + 2 * frames
    h = s.hidden
    at = places or layout(frames)
    W = lambda n: np.asarray(w[n], dtype=np.float64)
    mu = np.asarray(mu, dtype=np.float64).reshape(rows, MU_TOKENS, h)
    cond = np.asarray(cond, dtype=np.float64).reshape(rows, feat, frames)
    state = np.asarray(sampling, dtype=np.float64).reshape(rows, 2)[:, 0][:, None, None] * np.asarray(noise, np.float64)
    x0 = state.copy()
    tokens = np.zeros((rows, 2, T, h))
    cond_tok = (W("cond_proj.weight") @ cond).transpose(0, 2, 1) + W("cond_proj.bias")  # [rows][frames][h]
    for s_ in range(2):
        tokens[:, s_, at["cond"] : at["cond"] + frames] = cond_tok
    seqs_with_mu = slice(None) if at.get("mu_both") else 0  # zero in the unconditional sequence
    tokens[:, seqs_with_mu, at["mu"] : at["mu"] + MU_TOKENS] = mu[:, None] if at.get("mu_both") else mu
    times = time_tokens(w, timesteps, h)
    vs = []
    for i, (t, dt) in enumerate(euler_steps(timesteps)):
        tokens[:, :, at["time"]] = times[i]
        x_tok = (W("in_proj.weight") @ state).transpose(0, 2, 1) + W("in_proj.bias")
        tokens[:, :, at["x"] : at["x"] + frames] = x_tok[:, None]
        out = local_stack(w, s, tokens.reshape(rows * 2 * T, h), T, rope_on).reshape(rows, 2, T, h)
        vel = out[:, :, at["read"] : at["read"] + frames] @ W("out_proj.weight").T + W("out_proj.bias")  # [rows][2][frames][feat]
        vel = vel.transpose(0, 1, 3, 2)  # [rows][2][feat][frames]
        vs.append(vel)
        for r in range(rows):
            g = cfg_zero_star(vel[r, 0], vel[r, 1], float(sampling[r][1]))
            state[r] -= dt * g
    if velocities:
        return x0, state, np.stack(vs) if vs else np.zeros((0, rows, 2, feat, frames))
    return x0, state


def quantize(v: np.ndarray, levels: int) -> np.ndarray:
    """The scalar quantizer (gemv_linear.comp:54-59): roundEven(sign(v) tanh|v| L) / L."""
    return np.rint(np.sign(v) * np.tanh(np.abs(v)) * levels) / levels


def linear(w: dict, name: str, x: np.ndarray, bias: bool = True) -> np.ndarray:
    y = np.asarray(x, np.float64) @ np.asarray(w[f"{name}.weight"], np.float64).T
    if bias:
        y = y + np.asarray(w[f"{name}.bias"], np.float64)
    return y


def quantizer(w: dict, base_out: np.ndarray, levels: int):
    """fsq_layer.in_proj of the base LM's output and its rounding (lm_side.rs:405-412): the
    preactivation and the levels."""
    pre = linear(w, "fsq_layer.in_proj", base_out)
    return pre, quantize(pre, levels)


def heads_after_levels(w: dict, lv: np.ndarray, embed: np.ndarray):
    """From the levels: lm_hidden, the residual LM's input, lm_to_dit_proj's half of mu, the stop
    head's hidden state and its logits (lm_side.rs:413-460)."""
    lm_hidden = linear(w, "fsq_layer.out_proj", lv)
    residual_in = linear(w, "fusion_concat_proj", np.concatenate([lm_hidden, embed], axis=-1))
    to_dit = linear(w, "lm_to_dit_proj", lm_hidden)
    stop_pre = linear(w, "stop_proj", lm_hidden)
    stop_hidden = stop_pre / (1.0 + np.exp(-stop_pre))
    stop_logits = linear(w, "stop_head", stop_hidden, bias=False)
    return lm_hidden, residual_in, to_dit, stop_hidden, stop_logits
