"""The patch oracle pinned on the CPU: the Euler schedule's ends and step counts
(crates/graph/src/local/dit.rs:44-79), the time embedding's closed form (dit.rs:367-381),
CFG-Zero*'s reductions (dit_euler.comp:81-110), the scalar quantizer's special cases
(gemv_linear.comp:54-59), the local stack against an independent torch float64 model, and the
whole sampler against the closed form it takes when out_proj reads nothing. The library's own
schedule (host code, no GPU) must agree with the oracle's bit for bit."""

import math

import numpy as np
import pytest

import patch_oracle as po


def test_ten_steps_run_the_dit_nine_times_from_one_towards_zero():
    span = po.schedule(10)
    assert span[0] == np.float32(1.0) and span[-1] == np.float32(0.0)
    assert np.all(np.diff(span) < 0)
    steps = po.euler_steps(10)
    assert len(steps) == 9
    # The first evaluation is at t_span[1], each dt the gap to the next time.
    assert steps[0][0] == pytest.approx(float(span[1]), abs=1e-7)
    for (t, dt), nxt in zip(steps, span[2:]):
        assert t - dt == pytest.approx(float(nxt), abs=2e-7)
    assert sum(dt for _, dt in steps) == pytest.approx(float(span[1]), abs=1e-6)


@pytest.mark.parametrize("n, evaluations", [(1, 0), (2, 1), (10, 9), (24, 23), (25, 24), (49, 47), (50, 48)])
def test_the_zero_init_steps_are_four_percent_but_at_least_one(n, evaluations):
    assert len(po.euler_steps(n)) == evaluations


def test_the_sway_is_the_closed_form_in_float64_to_float32_precision():
    span = po.schedule(16)
    t = np.linspace(1.0, 0.0, 17)
    want = t + (np.cos(np.pi / 2 * t) - 1.0 + t)
    assert np.max(np.abs(span - want)) < 4e-7


@pytest.mark.parametrize("n", [1, 2, 5, 10, 25, 50])
def test_the_library_schedule_is_the_oracles_bit_for_bit(n):
    from tgx.patch import euler_steps

    got = euler_steps(n)
    want = po.euler_steps(n)
    assert len(got) == len(want)
    for (gt, gdt), (wt, wdt) in zip(got, want):
        assert np.float32(gt) == np.float32(wt) and np.float32(gdt) == np.float32(wdt)


def test_the_time_embedding_at_zero_is_sines_zero_then_cosines_one():
    e = po.time_embedding(0.0, 1024)
    assert np.all(e[:512] == 0.0) and np.all(e[512:] == 1.0)


def test_the_time_embedding_follows_the_float64_closed_form():
    h = 1024
    e = po.time_embedding(0.37, h)
    freqs = np.exp(np.arange(h // 2) * -(math.log(10000.0) / (h // 2 - 1)))
    a = 370.0 * freqs
    # f32 angles of magnitude up to 370: an ulp of 3e-5 there.
    assert np.max(np.abs(e - np.concatenate([np.sin(a), np.cos(a)]))) < 1e-4


def test_cfg_zero_star_reduces_as_its_algebra_says():
    rng = np.random.default_rng(0)
    vc, vu = rng.standard_normal(256), rng.standard_normal(256)
    assert np.allclose(po.cfg_zero_star(vc, vu, 1.0), vc, atol=1e-12)
    g = po.cfg_zero_star(vu, vu, 2.0)
    alpha = vu @ vu / (vu @ vu + 1e-8)
    assert np.allclose(g, vu * (alpha + 2.0 * (1 - alpha)), atol=1e-12)
    assert np.allclose(po.cfg_zero_star(vc, np.zeros(256), 2.0), 2.0 * vc)
    # A planted defect: guidance applied to the raw unconditional velocity differs.
    plain = vu + 2.0 * (vc - vu)
    assert not np.allclose(po.cfg_zero_star(vc, vu, 2.0), plain)


def test_the_quantizer_rounds_tanh_to_its_levels_ties_to_even():
    L = 9
    assert po.quantize(np.array([0.0]), L)[0] == 0.0
    assert np.all(po.quantize(np.array([40.0, -40.0]), L) == [1.0, -1.0])
    v = np.linspace(-3, 3, 10001)
    q = po.quantize(v, L)
    assert np.allclose(q * L, np.rint(q * L))
    assert np.max(np.abs(q - np.tanh(v))) <= 0.5 / L + 1e-12
    assert np.all(np.diff(q) >= 0)
    # Ties: tanh(v) L = k + 1/2 rounds to the even k.
    for k in (0, 1, 2, 7):
        tie = math.atanh((k + 0.5) / L)
        got = po.quantize(np.array([tie]), L)[0] * L
        assert round(got) in (k, k + 1)
    assert np.rint(2.5) == 2.0 and np.rint(3.5) == 4.0


def _torch_local_stack(w, s, x, T):
    """An independent float64 model of the local stack from torch library ops."""
    import torch
    import torch.nn.functional as F

    def t(n):
        return torch.tensor(np.asarray(w[n], dtype=np.float64))

    def norm(v, g):
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + s.eps) * g

    import oracle

    cos, sin = (torch.tensor(a.astype(np.float64)) for a in oracle.rope_tables(T, s.head_dim, s.rope_theta))
    cos = torch.cat([cos, cos], -1)
    sin = torch.cat([sin, sin], -1)

    def rot(v):  # [seqs][heads][T][d]
        half = v.shape[-1] // 2
        return v * cos + torch.cat([-v[..., half:], v[..., :half]], -1) * sin

    H, KV, d = s.heads, s.kv_heads, s.head_dim
    xt = torch.tensor(x)
    seqs = xt.shape[0] // T
    for l in range(s.layers):
        n = norm(xt, t(f"layers.{l}.input_layernorm"))
        qkv = n @ t(f"layers.{l}.qkv_proj").T
        q = qkv[:, : H * d].reshape(seqs, T, H, d).transpose(1, 2)
        k = qkv[:, H * d : (H + KV) * d].reshape(seqs, T, KV, d).transpose(1, 2)
        v = qkv[:, (H + KV) * d :].reshape(seqs, T, KV, d).transpose(1, 2)
        q, k = rot(q), rot(k)
        k = k.repeat_interleave(H // KV, dim=1)
        v = v.repeat_interleave(H // KV, dim=1)
        a = F.scaled_dot_product_attention(q, k, v).transpose(1, 2).reshape(-1, H * d)
        xt = xt + a @ t(f"layers.{l}.o_proj").T
        n = norm(xt, t(f"layers.{l}.post_attention_layernorm"))
        gate, up = (n @ t(f"layers.{l}.gate_up_proj").T).split(s.inner, -1)
        xt = xt + (F.silu(gate) * up) @ t(f"layers.{l}.down_proj").T
    return norm(xt, t("norm")).numpy()


def _small_dit(layers=2):
    from tgx.synth import StackSpec, sampler_weights

    spec = StackSpec(layers=layers, hidden=1024, inner=1024, dtype="f32", seed=3)
    return spec, sampler_weights(spec, 64)


def test_the_local_stack_matches_an_independent_torch_model():
    spec, w = _small_dit(2)
    s = po.StackShape(hidden=spec.hidden, inner=spec.inner, layers=spec.layers)
    T = 11
    x = np.random.default_rng(1).standard_normal((2 * T, spec.hidden))
    got = po.local_stack(w, s, x, T)
    want = _torch_local_stack(w, s, x, T)
    assert np.max(np.abs(got - want)) < 1e-9
    # Planted defects: RoPE left out, or positions counted across sequences, must show.
    assert np.max(np.abs(po.local_stack(w, s, x, T, rope_on=False) - want)) > 1e-3


def test_sequences_do_not_see_each_other():
    spec, w = _small_dit(1)
    s = po.StackShape(hidden=spec.hidden, inner=spec.inner, layers=spec.layers)
    T = 11
    x = np.random.default_rng(2).standard_normal((3 * T, spec.hidden))
    both = po.local_stack(w, s, x, T)
    alone = po.local_stack(w, s, x[T : 2 * T], T)
    assert np.allclose(both[T : 2 * T], alone, atol=1e-12)


def test_the_sampler_is_the_euler_closed_form_when_out_proj_reads_nothing():
    """out_proj.weight = 0: both velocities are the bias b, guided = (alpha + cfg (1 - alpha)) b,
    and the patch is x0 - (sum of dt) guided whatever the DiT computes."""
    spec, w = _small_dit(1)
    w = dict(w)
    w["out_proj.weight"] = np.zeros_like(w["out_proj.weight"])
    s = po.StackShape(hidden=spec.hidden, inner=spec.inner, layers=spec.layers)
    rows, feat, frames, n = 2, 64, 4, 10
    rng = np.random.default_rng(3)
    mu = rng.standard_normal((rows, 2, spec.hidden))
    cond = rng.standard_normal((rows, feat, frames))
    noise = rng.standard_normal((rows, feat, frames))
    sampling = np.array([[0.8, 2.0], [1.0, 1.5]])
    x0, patch = po.sample(w, s, feat, frames, n, mu, cond, noise, sampling)
    b = np.asarray(w["out_proj.bias"], np.float64)[None, :, None] * np.ones((1, 1, frames))
    total = sum(dt for _, dt in po.euler_steps(n))
    for r in range(rows):
        g = po.cfg_zero_star(b[0], b[0], sampling[r, 1])
        assert np.allclose(patch[r], x0[r] - total * g, atol=1e-12)
        assert np.allclose(x0[r], sampling[r, 0] * noise[r])


def test_the_time_mlp_and_the_heads_match_torch_library_ops():
    """time_mlp (dit.rs:409-421) and the layers between the LMs (lm_side.rs:405-460) against
    torch's linear and silu in float64: the weights' orientation (y = x W^T + b), the bias and the
    SiLU are the library's. A planted defect (W taken transposed) must show."""
    import torch
    import torch.nn.functional as F

    from tgx.synth import heads_weights

    _, w = _small_dit(1)
    t = lambda a: torch.as_tensor(np.asarray(a, np.float64))
    x = po.time_embedding(0.37, 1024).astype(np.float64)
    want = F.linear(F.silu(F.linear(t(x), t(w["time_mlp.linear_1.weight"]), t(w["time_mlp.linear_1.bias"]))),
                    t(w["time_mlp.linear_2.weight"]), t(w["time_mlp.linear_2.bias"])).numpy()
    assert np.max(np.abs(po.time_mlp(w, "time_mlp", x) - want)) < 1e-12

    h = heads_weights(5, 1024, 1024, 256, 64, dtype="f32")
    rng = np.random.default_rng(4)
    lv = rng.standard_normal((3, 64))
    embed = rng.standard_normal((3, 1024))
    got = po.heads_after_levels(h, lv, embed)
    lin = lambda name, v, bias=True: F.linear(v, t(h[f"{name}.weight"]), t(h[f"{name}.bias"]) if bias else None)
    lm_hidden = lin("fsq_layer.out_proj", t(lv))
    stop_hidden = F.silu(lin("stop_proj", lm_hidden))
    want = (lm_hidden, lin("fusion_concat_proj", torch.cat([lm_hidden, t(embed)], dim=-1)),
            lin("lm_to_dit_proj", lm_hidden), stop_hidden, lin("stop_head", stop_hidden, bias=False))
    for g_, w_ in zip(got, want):
        assert np.max(np.abs(g_ - w_.numpy())) < 1e-12
    wrong = dict(h)
    wrong["stop_proj.weight"] = np.ascontiguousarray(h["stop_proj.weight"].T)
    assert np.max(np.abs(po.heads_after_levels(wrong, lv, embed)[3] - want[3].numpy())) > 1e-3


def test_the_encoder_matches_an_independent_torch_model():
    """encode (crates/graph/src/local/encoder.rs:42-128) against the torch stack model fed
    [special; in_proj(frames)] built with torch's linear; a row's embedding is its own alone; the
    frames reversed, which only RoPE tells apart, must change it (the reference's defect check,
    crates/graph/tests/local.rs:496-505)."""
    import torch
    import torch.nn.functional as F

    from tgx.synth import StackSpec, encoder_weights

    spec = StackSpec(layers=2, hidden=1024, inner=1024, dtype="f32", seed=6)
    w = encoder_weights(spec, 64)
    s = po.StackShape(hidden=spec.hidden, inner=spec.inner, layers=spec.layers)
    rng = np.random.default_rng(12)
    patches = rng.standard_normal((3, 64, 4))
    got = po.encode(w, s, 64, 4, patches)
    t = lambda a: torch.as_tensor(np.asarray(a, np.float64))
    frames = F.linear(t(patches).transpose(1, 2), t(w["in_proj.weight"]), t(w["in_proj.bias"]))  # [rows][4][h]
    tokens = torch.cat([t(w["special_token"]).expand(3, 1, -1), frames], dim=1).reshape(15, -1).numpy()
    want = _torch_local_stack(w, s, tokens, 5).reshape(3, 5, -1)[:, 0]
    assert np.max(np.abs(got - want)) < 1e-9
    alone = po.encode(w, s, 64, 4, patches[1:2])
    assert np.allclose(alone[0], got[1], atol=1e-12)
    reversed_ = po.encode(w, s, 64, 4, patches[:, :, ::-1])
    assert np.max(np.abs(reversed_ - got)) > 1e-3


# ---- the DiT's sequence: where mu, the time, the patch before and the state sit -----------------

# Planted defects: the patch before (cond) and the state x trading places, the velocity read where
# x now sits (a layout consistent with itself, which only the positions RoPE sees tell apart); and
# the same trade with the velocity read at x's proper place, that is from cond's outputs.
SWAPPED = {"mu": 0, "time": 2, "cond": 7, "x": 3, "read": 3}
MISREAD = {"mu": 0, "time": 2, "cond": 7, "x": 3, "read": 7}


def _dit_case(rows=2, seed=21, hidden=1024):
    rng = np.random.default_rng(seed)
    mu = rng.standard_normal((rows, 2, hidden))
    cond = rng.standard_normal((rows, 64, 4))
    noise = rng.standard_normal((rows, 64, 4))
    sampling = np.array([[0.9, 2.0], [1.0, 1.5], [0.7, 3.0]])[:rows]
    return mu, cond, noise, sampling


def _shape(spec):
    return po.StackShape(hidden=spec.hidden, inner=spec.inner, layers=spec.layers)


def test_the_dit_sequence_assembled_by_hand_gives_the_oracles_euler_step():
    """crates/graph/src/local/dit.rs:36-41, 178-258: each row's conditional sequence is
    [mu_0, mu_1, time, cond_0..3, x_0..3] and its unconditional one the same with mu zero, the
    velocity out_proj of x's four outputs. Assembled here token by token with torch's linear,
    through the independent torch float64 model of the local stack, CFG-Zero* and one Euler step
    by their formulas (dit_euler.comp:81-110): with 2 timesteps the DiT runs once. A sequence
    with cond and x trading places (read where x sits) must fail it."""
    import torch
    import torch.nn.functional as F

    spec, w = _small_dit(2)
    s = _shape(spec)
    h, rows = spec.hidden, 2
    mu, cond, noise, sampling = _dit_case(rows)
    ((t, dt),) = po.euler_steps(2)
    time_token = po.time_tokens(w, 2, h)[0]  # pinned above: the embedding's closed form, time_mlp
    tt = lambda a: torch.as_tensor(np.asarray(a, np.float64))
    x0 = sampling[:, 0][:, None, None] * noise
    seqs = []
    for r in range(rows):
        cond_tokens = F.linear(tt(cond[r]).T, tt(w["cond_proj.weight"]), tt(w["cond_proj.bias"]))  # [4][h]
        x_tokens = F.linear(tt(x0[r]).T, tt(w["in_proj.weight"]), tt(w["in_proj.bias"]))
        for conditional in (True, False):
            m = tt(mu[r]) if conditional else torch.zeros(2, h, dtype=torch.float64)
            seqs.append(torch.cat([m, tt(time_token)[None], cond_tokens, x_tokens]))
    assert seqs[0].shape == (11, h)
    out = _torch_local_stack(w, s, torch.cat(seqs).numpy(), 11).reshape(rows, 2, 11, h)
    vel = F.linear(tt(out[:, :, 7:11]), tt(w["out_proj.weight"]), tt(w["out_proj.bias"])).numpy().transpose(0, 1, 3, 2)
    want = np.empty_like(x0)
    for r in range(rows):
        vc, vu = vel[r, 0], vel[r, 1]
        alpha = np.sum(vc * vu) / (np.sum(vu * vu) + 1e-8)
        want[r] = x0[r] - dt * (alpha * vu + sampling[r, 1] * (vc - alpha * vu))
    _, got = po.sample(w, s, 64, 4, 2, mu, cond, noise, sampling)
    scale = np.max(np.abs(want - x0))
    assert np.max(np.abs(got - want)) <= 1e-9 * scale
    _, wrong = po.sample(w, s, 64, 4, 2, mu, cond, noise, sampling, places=SWAPPED)
    assert np.max(np.abs(wrong - want)) > 1e-4 * scale


def _per_token_dit(spec, w):
    """The DiT with every layer's o_proj and down_proj zero: attention and MLP add nothing, so the
    stack maps each token alone through the final norm."""
    w = dict(w)
    for l in range(spec.layers):
        for name in ("o_proj", "down_proj"):
            w[f"layers.{l}.{name}"] = np.zeros_like(w[f"layers.{l}.{name}"])
    return w


def test_with_the_stack_per_token_the_velocity_is_x_alone():
    """With the stack per token, each evaluation's velocities are
    out_proj(norm(in_proj(x) + b)) + b of the state x alone, the same in both sequences, and mu,
    the patch before and the time do not move them. Reading the velocity from cond's outputs
    (MISREAD) must fail it."""
    spec, w = _small_dit(2)
    w = _per_token_dit(spec, w)
    s = _shape(spec)
    mu, cond, noise, sampling = _dit_case(2)
    x0, _, vs = po.sample(w, s, 64, 4, 10, mu, cond, noise, sampling, velocities=True)
    W = lambda n: np.asarray(w[n], np.float64)
    tokens = (W("in_proj.weight") @ x0).transpose(0, 2, 1) + W("in_proj.bias")  # [rows][4][h]
    normed = tokens / np.sqrt(np.mean(tokens * tokens, axis=-1, keepdims=True) + spec.eps) * W("norm")
    want = (normed @ W("out_proj.weight").T + W("out_proj.bias")).transpose(0, 2, 1)  # [rows][feat][4]
    for c in (0, 1):
        assert np.max(np.abs(vs[0][:, c] - want)) <= 1e-10 * np.max(np.abs(want))
    rng = np.random.default_rng(5)
    _, _, moved = po.sample(w, s, 64, 4, 10, rng.standard_normal(mu.shape), rng.standard_normal(cond.shape), noise,
                            sampling, velocities=True)
    assert np.allclose(moved, vs, rtol=0, atol=1e-12)
    _, _, misread = po.sample(w, s, 64, 4, 10, mu, cond, noise, sampling, places=MISREAD, velocities=True)
    assert np.max(np.abs(misread[0][:, 0] - want)) > 1e-3 * np.max(np.abs(want))


def test_mu_reaches_the_conditional_sequence_only():
    """mu tokens sit in the conditional sequence and are zero in the unconditional one
    (dit.rs:36-41): at the first evaluation (the state x0 the same either way) another mu leaves
    v_u exactly as it was and moves v_c. With mu zero the two sequences are the same, so v_c = v_u
    at every evaluation and each Euler step moves x by dt (alpha + cfg (1 - alpha)) v_c."""
    spec, w = _small_dit(2)
    s = _shape(spec)
    mu, cond, noise, sampling = _dit_case(2)
    _, _, vs = po.sample(w, s, 64, 4, 10, mu, cond, noise, sampling, velocities=True)
    _, _, other = po.sample(w, s, 64, 4, 10, 3.0 * mu[::-1], cond, noise, sampling, velocities=True)
    assert np.allclose(other[0][:, 1], vs[0][:, 1], rtol=0, atol=1e-12)
    assert np.max(np.abs(other[0][:, 0] - vs[0][:, 0])) > 1e-3 * np.max(np.abs(vs[0][:, 0]))
    x0, patch, zero = po.sample(w, s, 64, 4, 10, np.zeros_like(mu), cond, noise, sampling, velocities=True)
    assert np.allclose(zero[:, :, 0], zero[:, :, 1], rtol=0, atol=1e-12)
    x = x0.copy()
    for (t, dt), v in zip(po.euler_steps(10), zero):
        for r in range(2):
            vc = v[r, 0]
            alpha = np.sum(vc * vc) / (np.sum(vc * vc) + 1e-8)
            x[r] -= dt * (alpha + sampling[r, 1] * (1 - alpha)) * vc
    assert np.max(np.abs(patch - x)) <= 1e-12 * np.max(np.abs(x))
    # Planted: mu written into both sequences must break the first check.
    both = {**po.layout(4), "mu_both": True}
    _, _, a = po.sample(w, s, 64, 4, 10, mu, cond, noise, sampling, places=both, velocities=True)
    _, _, b = po.sample(w, s, 64, 4, 10, 3.0 * mu[::-1], cond, noise, sampling, places=both, velocities=True)
    assert np.max(np.abs(a[0][:, 1] - b[0][:, 1])) > 1e-3 * np.max(np.abs(a[0][:, 1]))
