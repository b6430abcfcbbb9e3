"""The oracle pinned before it is trusted: against the reference's own known-answer fixture
(crates/testkit/tests/fixtures/testkit.safetensors, copied to tests/golden/), the reference's
unit-test facts, closed forms, an independent float64 model built from torch library ops, and
planted defects that must fail. CPU only."""

import math
from pathlib import Path

import numpy as np
import pytest

GOLDEN = Path(__file__).resolve().parent / "golden"


def load_testkit():
    from safetensors.torch import load_file

    return load_file(str(GOLDEN / "testkit.safetensors"))


# ---- RMSNorm ------------------------------------------------------------------------------------


def test_rmsnorm_matches_upstream_rms_layernorm_known_answer():
    """fixtures/testkit.py:15-17: upstream's rms_layernorm([[3, 4]], [1, 2], eps=0) as torch
    computed it, and crates/testkit/tests/testkit.rs:58-70's closed form [3/sqrt(12.5), 8/sqrt(12.5)]."""
    import oracle

    want = load_testkit()["rms_layernorm"].numpy().ravel()
    got = oracle.rmsnorm(np.array([3.0, 4.0]), np.array([1.0, 2.0], dtype=np.float32), 0.0)
    rms = np.sqrt(12.5)
    assert np.allclose(got, [3 / rms, 8 / rms], rtol=0, atol=1e-15)
    assert np.allclose(got, want, rtol=1e-6, atol=1e-6)
    got32 = oracle.rmsnorm(np.array([3.0, 4.0]), np.array([1.0, 2.0], dtype=np.float32), 0.0, "f32")
    assert np.allclose(got32, want, rtol=1e-6, atol=1e-6)


def test_rmsnorm_closed_form_and_a_missing_gain_fails():
    import oracle

    rng = np.random.default_rng(3)
    x = rng.uniform(-2, 2, 2048)
    g = (1 + rng.uniform(-1, 1, 2048) / 4).astype(np.float32)
    eps = 1e-5
    want = x / np.sqrt(np.mean(x * x) + eps) * g.astype(np.float64)
    got = oracle.rmsnorm(x, g, eps)
    assert np.max(np.abs(got - want)) <= 1e-12 * np.max(np.abs(want))
    # Defect (crates/vulkan/tests/glsl.rs:235-236): the gain left out.
    ungained = x / np.sqrt(np.mean(x * x) + eps)
    assert np.sum(np.abs(got - ungained) > 1e-3) > 1024


# ---- half-precision conversions -----------------------------------------------------------------


def test_bf16_rounding_matches_torchs_bits():
    """testkit.rs:30-55: torch rounds [1.0, -2.5, 0.1, 3.14159] to bf16 bits 3f80 c020 3dcd 4049."""
    from tgx.synth import bf16_bits

    want = load_testkit()["bf16"].view(dtype=__import__("torch").int16).numpy().view(np.uint16)
    got = bf16_bits(np.array([1.0, -2.5, 0.1, 3.14159], dtype=np.float32))
    assert list(got) == [0x3F80, 0xC020, 0x3DCD, 0x4049]
    assert np.array_equal(got, want)
    # Ties go to even: 1 + 2^-8 is halfway between 1 and 1 + 2^-7.
    assert bf16_bits(np.array([1 + 2**-8], dtype=np.float32))[0] == 0x3F80
    assert bf16_bits(np.array([1 + 3 * 2**-8], dtype=np.float32))[0] == 0x3F82


def test_f16_fixture_widens_exactly():
    """testkit.rs:38-43: f16 [0.1, -65504, 6e-8] widen to 0.099975586, -65504, 5.9604645e-8."""
    f16 = load_testkit()["f16"].numpy()
    assert list(f16.astype(np.float32)) == [np.float32(0.099975586), np.float32(-65504.0), np.float32(5.9604645e-8)]


# ---- RoPE tables --------------------------------------------------------------------------------


def test_rope_tables_start_at_the_identity_and_turn_at_each_rate():
    """decode.rs:1232-1242: cos 1 and sin 0 at position 0; at position 1, frequency 0 turns one
    radian, cos(1f32) and sin(1f32) exactly."""
    import oracle

    cos, sin = oracle.rope_tables(64, 128)
    assert cos.shape == (64, 64)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    # f32's cos(1) and sin(1): the double values rounded once to f32.
    assert cos[1, 0] == np.float32(math.cos(1.0))
    assert sin[1, 0] == np.float32(math.sin(1.0))


def test_rope_tables_follow_the_f32_recipe():
    """decode.rs:146-168 restated here with libm's own f32 functions, one value at a time:
    inv = 1 / powf(theta, i / d), r = 1 / (f32)factor, angle = (t * r) * inv; bit-exact."""
    import ctypes

    import oracle

    libm = ctypes.CDLL("libm.so.6")
    for name in ("powf", "cosf", "sinf"):
        getattr(libm, name).restype = ctypes.c_float
    libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]
    libm.cosf.argtypes = [ctypes.c_float]
    libm.sinf.argtypes = [ctypes.c_float]
    d = 64
    factors = 1.0 + np.arange(d // 2) * 0.47
    cos, sin = oracle.rope_tables(300, d, 10000.0, factors)
    f32 = np.float32
    for t in (0, 1, 2, 37, 255, 299):
        for j in (0, 1, 7, 31):
            inv = f32(1.0) / f32(libm.powf(10000.0, float(f32(2 * j) / f32(d))))
            r = f32(1.0) / f32(factors[j])
            angle = (f32(t) * r) * inv
            assert cos[t, j] == f32(libm.cosf(float(angle))), (t, j)
            assert sin[t, j] == f32(libm.sinf(float(angle))), (t, j)
    # A recipe in f64 differs from it somewhere.
    inv64 = 1.0 / np.power(10000.0, np.arange(0, d, 2) / d)
    angle64 = np.arange(300)[:, None] / factors[None, :] * inv64[None, :]
    assert np.any(np.cos(angle64).astype(np.float32) != cos)


# ---- attention ----------------------------------------------------------------------------------


def brute_attention(q, kc, vc, heads, kv_heads, position):
    group = heads // kv_heads
    d = q.shape[1]
    out = np.zeros_like(q)
    for h in range(heads):
        k = kc[h // group, : position + 1]
        v = vc[h // group, : position + 1]
        s = k @ q[h] / np.sqrt(d)
        w = np.exp(s - s.max())
        out[h] = (w / w.sum()) @ v
    return out


@pytest.mark.parametrize("position", [0, 5, 31, 32, 33, 100, 446, 511])
def test_attention_is_softmax_attention_up_to_the_position(position):
    """crates/vulkan/tests/glsl.rs:617-649, with what lies past the position NaN, which must not
    reach the output (glsl.rs:690-699)."""
    import oracle

    rng = np.random.default_rng(41)
    heads, kv, d, cap = 16, 2, 64, 512
    q = rng.uniform(-2, 2, (heads, d))
    kc = rng.uniform(-2, 2, (kv, cap, d))
    vc = rng.uniform(-1, 1, (kv, cap, d))
    want = brute_attention(q, kc, vc, heads, kv, position)
    kc[:, position + 1 :] = np.nan
    vc[:, position + 1 :] = np.nan
    got = oracle.attention(q, kc, vc, heads, kv, d, position)
    assert np.all(np.isfinite(got))
    assert np.max(np.abs(got - want)) <= 1e-12


def test_attention_over_one_position_returns_its_value():
    import oracle

    rng = np.random.default_rng(5)
    q = rng.normal(size=(8, 64))
    kc = rng.normal(size=(1, 4, 64))
    vc = rng.normal(size=(1, 4, 64))
    got = oracle.attention(q, kc, vc, 8, 1, 64, 0)
    assert np.allclose(got, np.repeat(vc[0, :1], 8, axis=0), atol=1e-15)


# ---- the whole stack against an independent float64 model --------------------------------------


def torch_stack(spec, weights, x, rope=True, start=0, causal=True, rope_dim=None, gqa_tiled=False):
    """MiniCPM-4 layers over a run of positions from library ops in float64: RMSNorm written out,
    RoPE by rotate_half, torch's scaled_dot_product_attention (causal, GQA by repeat), SiLU.
    rope_dim (a planted defect when not the head width): the width rotate_half pairs within.
    gqa_tiled (a planted defect): query head h reads KV head h % kv_heads, not h // group."""
    import torch
    import torch.nn.functional as F

    import oracle

    T = x.shape[0]
    h = torch.tensor(x, dtype=torch.float64)
    w = {k: torch.tensor(v, dtype=torch.float64) for k, v in weights.items()}
    H, KV, d = spec.heads, spec.kv_heads, spec.head_dim
    rd = rope_dim or d
    cos, sin = oracle.rope_tables(start + T, rd, spec.rope_theta)
    cos = torch.tensor(cos[start:], dtype=torch.float64)
    sin = torch.tensor(sin[start:], dtype=torch.float64)
    cos = torch.cat([cos, cos] * (d // rd), dim=-1)[:, None, :]
    sin = torch.cat([sin, sin] * (d // rd), dim=-1)[:, None, :]

    def norm(v, g):
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + spec.eps) * g

    def rotate_half(v):
        parts = []
        for j in range(0, d, rd):
            a, b = v[..., j : j + rd // 2], v[..., j + rd // 2 : j + rd]
            parts += [-b, a]
        return torch.cat(parts, dim=-1)

    for l in range(spec.layers):
        n = norm(h, w[f"layers.{l}.input_layernorm"])
        qkv = n @ w[f"layers.{l}.qkv_proj"].T
        q = qkv[:, : H * d].reshape(T, H, d)
        k = qkv[:, H * d : (H + KV) * d].reshape(T, KV, d)
        v = qkv[:, (H + KV) * d :].reshape(T, KV, d)
        if rope:
            q = q * cos + rotate_half(q) * sin
            k = k * cos + rotate_half(k) * sin
        if gqa_tiled:
            k, v = k.repeat(1, H // KV, 1), v.repeat(1, H // KV, 1)
        else:
            k = k.repeat_interleave(H // KV, dim=1)
            v = v.repeat_interleave(H // KV, dim=1)
        att = F.scaled_dot_product_attention(q.transpose(0, 1), k.transpose(0, 1), v.transpose(0, 1), is_causal=causal)
        att = att.transpose(0, 1).reshape(T, H * d)
        h = h + att @ w[f"layers.{l}.o_proj"].T
        n = norm(h, w[f"layers.{l}.post_attention_layernorm"])
        gu = n @ w[f"layers.{l}.gate_up_proj"].T
        gate, up = gu[:, : spec.inner], gu[:, spec.inner :]
        h = h + (F.silu(gate) * up) @ w[f"layers.{l}.down_proj"].T
    return norm(h, w["norm"]).numpy()


@pytest.fixture(scope="module")
def tiny():
    from tgx.synth import StackSpec, stack_weights

    spec = StackSpec(hidden=512, inner=1024, heads=8, kv_heads=2, layers=2, dtype="f32", seed=7)
    return spec, stack_weights(spec)


def test_heads_of_128_dimensions_match_the_model_and_a_rope_of_64_fails():
    """VoxCPM2's LMs take heads of 128 dimensions (crates/graph/src/decode.rs:919-933): decode
    steps, a prefill and the layer-by-layer prefill at head_dim 128 against the float64 torch
    model; the model rotating the pairs (i, i + 32) of each 64 dimensions instead of (i, i + 64)
    must disagree with the oracle."""
    import oracle
    from tgx.synth import StackSpec, embeddings, stack_weights

    spec = StackSpec(hidden=1024, inner=1536, heads=8, kv_heads=2, head_dim=128, layers=2, dtype="f32", seed=9)
    w = stack_weights(spec)
    x = embeddings(3, "x", 40, spec.hidden).astype(np.float64)
    want = torch_stack(spec, w, x)
    st = oracle.Stack(spec, w, 64)
    out = st.prefill(0, x[:24])
    steps = np.stack([st.decode(t, x[t]) for t in range(24, 40)])
    got = np.concatenate([out, steps])
    assert np.max(np.abs(got - want)) <= 1e-10 * np.max(np.abs(want))
    rows = oracle.Stack(spec, w, 64).prefill_rows(0, x)
    assert np.max(np.abs(rows - want)) <= 1e-9 * np.max(np.abs(want))
    wrong = torch_stack(spec, w, x, rope_dim=64)
    assert np.max(np.abs(got - wrong)) > 1e-3 * np.max(np.abs(want))


@pytest.mark.parametrize("heads,kv_heads", [(6, 2), (10, 2), (12, 2), (24, 2)])
def test_groups_that_do_not_divide_16_match_the_model_and_the_wrong_kv_head_fails(heads, kv_heads):
    """Groups of 3, 5, 6 and 12 query heads a KV head (the kernels take any group up to 16): a
    prefill and decode steps against the float64 torch model (GQA by repeat_interleave: head h reads
    KV head h // group); the model reading KV head h % kv_heads instead must disagree."""
    import oracle
    from tgx.synth import StackSpec, embeddings, stack_weights

    spec = StackSpec(hidden=384, inner=768, heads=heads, kv_heads=kv_heads, layers=2, dtype="f32", seed=heads)
    w = stack_weights(spec)
    x = embeddings(4, "x", 30, spec.hidden).astype(np.float64)
    want = torch_stack(spec, w, x)
    st = oracle.Stack(spec, w, 32)
    got = np.concatenate([st.prefill(0, x[:20]), np.stack([st.decode(t, x[t]) for t in range(20, 30)])])
    assert np.max(np.abs(got - want)) <= 1e-10 * np.max(np.abs(want))
    wrong = torch_stack(spec, w, x, gqa_tiled=True)
    assert np.max(np.abs(got - wrong)) > 1e-3 * np.max(np.abs(want))


def test_decode_steps_match_a_float64_model_of_library_ops(tiny):
    import oracle
    from tgx.synth import embeddings

    spec, w = tiny
    x = embeddings(1, "x", 40, spec.hidden).astype(np.float64)
    want = torch_stack(spec, w, x)
    st = oracle.Stack(spec, w, 64)
    got = np.stack([st.decode(t, x[t]) for t in range(40)])
    assert np.max(np.abs(got - want)) <= 1e-10 * np.max(np.abs(want))


def test_prefill_matches_the_model_and_decode_goes_on_from_its_cache(tiny):
    """prefill.rs:473-503 and crates/graph/tests/prefill.rs:255-258: a run's outputs, then decode
    steps from the cache the run wrote."""
    import oracle
    from tgx.synth import embeddings

    spec, w = tiny
    x = embeddings(2, "x", 48, spec.hidden).astype(np.float64)
    want = torch_stack(spec, w, x)
    st = oracle.Stack(spec, w, 64)
    out = st.prefill(0, x[:32])
    steps = np.stack([st.decode(t, x[t]) for t in range(32, 48)])
    got = np.concatenate([out, steps])
    assert np.max(np.abs(got - want)) <= 1e-10 * np.max(np.abs(want))


@pytest.mark.parametrize("rope", [True, False])
def test_the_layer_by_layer_prefill_is_the_position_by_position_one(tiny, rope):
    """prefill_rows (a layer over every position at once, numpy's float64 products) against the
    pinned position-by-position path and the torch model: a run from 0, then a second run from
    where it ended in the same cache; outputs and both caches to float64 rounding. Planted
    defects must show: the causal mask left out, and the second run placed one position on."""
    import oracle
    from tgx.synth import embeddings

    spec, w = tiny
    x = embeddings(5, "x", 56, spec.hidden).astype(np.float64)
    want = torch_stack(spec, w, x, rope=rope)
    scale = np.max(np.abs(want))
    steps = oracle.Stack(spec, w, 64, rope=rope)
    rows = oracle.Stack(spec, w, 64, rope=rope)
    a = np.concatenate([steps.prefill(0, x[:37]), steps.prefill(37, x[37:])])
    b = np.concatenate([rows.prefill_rows(0, x[:37]), rows.prefill_rows(37, x[37:])])
    assert np.max(np.abs(b - a)) <= 1e-12 * scale
    assert np.max(np.abs(b - want)) <= 1e-10 * scale
    for cache in ("k", "v"):
        ca, cb = getattr(steps, cache), getattr(rows, cache)
        assert np.max(np.abs(cb - ca)) <= 1e-12 * np.max(np.abs(ca)), cache
    # Defects the comparison must see: every key visible to every position (the causal mask left
    # out), and the second run written one position on.
    leaky = torch_stack(spec, w, x[:37], rope=rope, causal=False)
    assert np.max(np.abs(leaky - a[:37])) > 1e-3 * scale
    shifted = oracle.Stack(spec, w, 64, rope=rope)
    s = np.concatenate([shifted.prefill_rows(0, x[:37]), shifted.prefill_rows(38, x[37:55])])
    assert np.max(np.abs(s - want[:55])) > 1e-3 * scale


def test_the_layer_by_layer_prefill_in_float32_is_the_float32_path(tiny):
    """prefill_rows in float32 (the CPU baseline's prefill) against the position-by-position
    float32 path and the float64 one, to float32 rounding."""
    import oracle
    from tgx.synth import embeddings

    spec, w = tiny
    x = embeddings(6, "x", 40, spec.hidden)
    want = oracle.Stack(spec, w, 64, "f64").prefill(0, x.astype(np.float64))
    steps = oracle.Stack(spec, w, 64, "f32").prefill(0, x)
    rows = oracle.Stack(spec, w, 64, "f32")
    got = rows.prefill_rows(0, x)
    assert got.dtype == np.float32 and rows.k.dtype == np.float32
    scale = np.max(np.abs(want))
    assert np.max(np.abs(got - steps)) <= 1e-4 * scale
    assert np.max(np.abs(got - want)) <= 1e-4 * scale


def test_a_stack_without_rope_and_its_defects(tiny):
    import oracle
    from tgx.synth import embeddings

    spec, w = tiny
    x = embeddings(3, "x", 40, spec.hidden).astype(np.float64)
    want = torch_stack(spec, w, x, rope=False)
    plain = oracle.Stack(spec, w, 64, rope=False)
    got = np.stack([plain.decode(t, x[t]) for t in range(40)])
    assert np.max(np.abs(got - want)) <= 1e-10 * np.max(np.abs(want))
    # Defects that must show: the stack rotated, and positions rotated one on.
    rotated = oracle.Stack(spec, w, 64, rope=True)
    r = np.stack([rotated.decode(t, x[t]) for t in range(40)])
    assert np.max(np.abs(r - want)) > 1e-2 * np.max(np.abs(want))
    # Positions one slot on (crates/graph/tests/decode.rs:252-255): position 0 of the cache stays
    # empty and every query attends to its zero key and value as well.
    shifted = oracle.Stack(spec, w, 64, rope=True)
    rope_want = torch_stack(spec, w, x)
    s = np.stack([shifted.decode(t + 1, x[t]) for t in range(40)])
    assert np.max(np.abs(s - rope_want)) > 1e-2 * np.max(np.abs(rope_want))


def test_float32_path_agrees_with_float64(tiny):
    import oracle
    from tgx.synth import embeddings

    spec, w = tiny
    x = embeddings(4, "x", 24, spec.hidden)
    a = oracle.Stack(spec, w, 32, "f64")
    b = oracle.Stack(spec, w, 32, "f32")
    for t in range(24):
        ga, gb = a.decode(t, x[t]), b.decode(t, x[t])
        assert np.max(np.abs(ga - gb)) <= 1e-4 * np.max(np.abs(ga))


def test_positions_past_the_capacity_are_refused(tiny):
    import oracle

    spec, w = tiny
    st = oracle.Stack(spec, w, 8)
    with pytest.raises(ValueError):
        st.decode(8, np.zeros(spec.hidden))
