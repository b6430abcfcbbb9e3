"""Weights from a safetensors checkpoint under VoxCPM2's names (load_stack, decode.rs:738-776;
load_lm_side, lm_side.rs:496-533; load_sampler, local/dit.rs:329-365; load_encoder,
local/encoder.rs:129-162) give, bit for bit, what the same values loaded tensor by tensor under the
library's names give: q/k/v and gate/up joined along their rows in the checkpoint's order."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

FEAT, FRAMES, STEPS, LATENT, LEVELS = 64, 4, 10, 256, 9


def _stack_entries(w, prefix, spec):
    """A stack's tensors (the library's names, joined) under the checkpoint's names (split)."""
    q, kv, inner = spec.heads * spec.head_dim, spec.kv_heads * spec.head_dim, spec.inner
    out = {}
    for l in range(spec.layers):
        at = f"{prefix}layers.{l}."
        qkv = w[f"layers.{l}.qkv_proj"]
        out[at + "self_attn.q_proj.weight"] = qkv[:q]
        out[at + "self_attn.k_proj.weight"] = qkv[q:q + kv]
        out[at + "self_attn.v_proj.weight"] = qkv[q + kv:]
        out[at + "self_attn.o_proj.weight"] = w[f"layers.{l}.o_proj"]
        gu = w[f"layers.{l}.gate_up_proj"]
        out[at + "mlp.gate_proj.weight"] = gu[:inner]
        out[at + "mlp.up_proj.weight"] = gu[inner:]
        out[at + "mlp.down_proj.weight"] = w[f"layers.{l}.down_proj"]
        out[at + "input_layernorm.weight"] = w[f"layers.{l}.input_layernorm"]
        out[at + "post_attention_layernorm.weight"] = w[f"layers.{l}.post_attention_layernorm"]
    out[prefix + "norm.weight"] = w["norm"]
    return out


def _save(path, entries, f32=()):
    """bf16 tensors (the values are bf16-rounded already), those named in `f32` in f32."""
    import torch
    from safetensors.torch import save_file

    tensors = {}
    for name, v in entries.items():
        t = torch.from_numpy(np.ascontiguousarray(v, dtype=np.float32))
        tensors[name] = t if name in f32 else t.to(torch.bfloat16)
    save_file(tensors, str(path), metadata={"format": "pt"})


def _shape(spec, capacity, rope=True):
    import tgx

    return tgx.Shape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads,
                     head_dim=spec.head_dim, layers=spec.layers, capacity=capacity, eps=spec.eps,
                     rope_theta=spec.rope_theta, rope=rope)


def test_a_decoder_loads_from_a_checkpoint_as_by_name(ctx, tmp_path):
    import tgx
    from tgx.checkpoint import Checkpoint
    from tgx.synth import StackSpec, embeddings, stack_weights

    spec = StackSpec(layers=2, seed=31)
    w = stack_weights(spec)
    entries = _stack_entries(w, "base_lm.", spec)
    _save(tmp_path / "bf16.safetensors", entries)
    # q in f32 beside k and v in bf16: the join reads all three as f32, the same values.
    _save(tmp_path / "mixed.safetensors", entries, f32={"base_lm.layers.0.self_attn.q_proj.weight"})
    by_name = tgx.Decoder(ctx, _shape(spec, 256), tgx.Batch(rows=1, slots=1))
    for name, v in w.items():
        by_name.load(name, v)
    x = embeddings(33, "ckpt.decode", 4, spec.hidden)
    want = [by_name.step(p, x[p]) for p in range(4)]
    by_name.close()
    for file in ("bf16", "mixed"):
        with Checkpoint(tmp_path / f"{file}.safetensors") as ck:
            dec = tgx.Decoder(ctx, _shape(spec, 256), tgx.Batch(rows=1, slots=1))
            dec.load_checkpoint(ck, "base_lm.")
            got = [dec.step(p, x[p]) for p in range(4)]
            dec.close()
        print(f"[checkpoint] decoder from {file}: {len(got)} steps", flush=True)
        for p in range(4):
            assert np.array_equal(got[p], want[p]), (file, p)


def test_a_missing_tensor_is_named(ctx, tmp_path):
    import tgx
    from tgx.checkpoint import Checkpoint
    from tgx.synth import StackSpec, stack_weights

    spec = StackSpec(layers=1, seed=32)
    entries = _stack_entries(stack_weights(spec), "", spec)
    del entries["layers.0.mlp.up_proj.weight"]
    _save(tmp_path / "short.safetensors", entries)
    dec = tgx.Decoder(ctx, _shape(spec, 64), tgx.Batch(rows=1, slots=1))
    with Checkpoint(tmp_path / "short.safetensors") as ck, pytest.raises(tgx.TgxError) as e:
        dec.load_checkpoint(ck)
    dec.close()
    assert e.value.kind == "weights" and "layers.0.mlp.up_proj.weight: no such tensor" in str(e.value)


def test_the_patch_step_loads_from_one_checkpoint_as_by_name(ctx, tmp_path):
    """The LM side, the sampler and the encoder from one VoxCPM2-named file; the patch step they
    make runs bit for bit as theirs loaded by name do."""
    import tgx
    from tgx.checkpoint import Checkpoint
    from tgx.patch import Encoder, HeadsShape, LmSide, PatchShape, PatchStep, Sampler
    from tgx.synth import StackSpec, encoder_weights, lm_side_weights, sampler_weights

    rows = 2
    base, residual = StackSpec(layers=2, seed=41), StackSpec(layers=1, seed=42)
    dit, local = StackSpec(layers=1, seed=43), StackSpec(layers=1, seed=44)
    lm_w = lm_side_weights(base, residual, 1024, 1024, LATENT)
    dit_w = sampler_weights(dit, FEAT)
    enc_w = encoder_weights(local, FEAT)
    entries = {}
    entries.update(_stack_entries({k[8:]: v for k, v in lm_w.items() if k.startswith("base_lm.")}, "base_lm.", base))
    entries.update(_stack_entries({k[12:]: v for k, v in lm_w.items() if k.startswith("residual_lm.")}, "residual_lm.",
                                  residual))
    entries.update({k: v for k, v in lm_w.items() if not k.startswith(("base_lm.", "residual_lm."))})
    entries.update(_stack_entries(dit_w, "feat_decoder.estimator.decoder.", dit))
    entries.update({f"feat_decoder.estimator.{k}": v for k, v in dit_w.items() if not k.startswith(("layers.", "norm"))})
    entries.update(_stack_entries(enc_w, "feat_encoder.encoder.", local))
    entries.update({f"feat_encoder.{k}": v for k, v in enc_w.items() if not k.startswith(("layers.", "norm"))})
    _save(tmp_path / "voxcpm2.safetensors", entries)

    patch = PatchShape(FEAT, FRAMES, STEPS, rows)

    def build():
        side = LmSide(ctx, _shape(base, 256), _shape(residual, 256, rope=False), tgx.Batch(rows=rows, slots=rows),
                      HeadsShape(1024, 1024, LATENT, LEVELS))
        smp = Sampler(ctx, _shape(dit, 16), patch)
        enc = Encoder(ctx, _shape(local, 16), patch)
        return side, smp, enc

    rng = np.random.default_rng(45)
    cond = rng.standard_normal((rows, FEAT, FRAMES)).astype(np.float32)
    noise = rng.standard_normal((rows, FEAT, FRAMES)).astype(np.float32)
    sampling = np.array([[1.0, 2.0], [0.8, 1.5]], dtype=np.float32)
    results = []
    for how in ("by name", "checkpoint"):
        side, smp, enc = build()
        if how == "by name":
            side.load_all(lm_w)
            smp.load_all(dit_w)
            enc.load_all(enc_w)
        else:
            with Checkpoint(tmp_path / "voxcpm2.safetensors") as ck:
                side.load_checkpoint(ck)
                smp.load_checkpoint(ck)
                enc.load_checkpoint(ck)
        step = PatchStep(enc, side, smp)
        out = [step.run_rows([tgx.Row(p, r) for r in range(rows)], cond, noise, sampling) for p in range(2)]
        print(f"[checkpoint] patch step {how}: done", flush=True)
        step.close()
        for o in (enc, smp, side):
            o.close()
        results.append(out)
    for (pa, sa), (pb, sb) in zip(*results):
        assert np.array_equal(pa, pb) and np.array_equal(sa, sb)
        assert np.isfinite(pa).all()
