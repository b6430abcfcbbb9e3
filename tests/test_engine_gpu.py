"""The engine (crates/tgtts/src/rt.rs:92-111, crates/graph/src/generator.rs) on the GPU, built from a
config.json and a VoxCPM2-named checkpoint as Generator::new builds it: requests started in slots
from their prompts, stepped together, ended by the stop head's argmax or their most patches, and
finished; a request comes out bit for bit as it does alone, whatever runs beside it."""

import json

import numpy as np
import pytest

from test_checkpoint_gpu import _save, _stack_entries

pytestmark = pytest.mark.gpu

FEAT, FRAMES, LATENT, LEVELS, VOCAB = 64, 4, 256, 9, 48
LAYOUT = [True] * 4 + [False] * 6 + [True] * 5


# The LMs' width: the backbone's (1024 wide, heads of 64) unless a test asks for VoxCPM2's own
# (2048 wide, an FFN of 6144, heads of 128; crates/graph/src/lm_side.rs:665-679).
BACKBONE = dict(hidden=1024, inner=4096, head_dim=64)
VOXCPM2 = dict(hidden=2048, inner=6144, head_dim=128)


def _config(lm_shape=BACKBONE):
    from tgx.config import Config

    h, d = lm_shape["hidden"], lm_shape["head_dim"]
    lm = {"bos_token_id": 1, "eos_token_id": 2, "hidden_size": h, "intermediate_size": lm_shape["inner"],
          "max_position_embeddings": 256, "num_attention_heads": 16, "num_hidden_layers": 2, "num_key_value_heads": 2,
          "rms_norm_eps": 1e-5, "rope_theta": 10000, "kv_channels": d,
          "rope_scaling": {"type": "longrope", "long_factor": [1.0] * (d // 2), "short_factor": [1.0] * (d // 2),
                           "original_max_position_embeddings": 256},
          "vocab_size": VOCAB, "use_mup": False, "scale_emb": 12, "dim_model_base": 256, "scale_depth": 1.4}
    local = {"hidden_dim": 1024, "ffn_dim": 4096, "num_heads": 16, "num_layers": 1, "kv_channels": 64}
    return Config.from_json(json.dumps({
        "architecture": "voxcpm2", "lm_config": lm, "patch_size": FRAMES, "feat_dim": FEAT,
        "scalar_quantization_latent_dim": LATENT, "scalar_quantization_scale": LEVELS,
        "residual_lm_num_layers": 1, "residual_lm_no_rope": True, "encoder_config": local,
        "dit_config": dict(local, cfm_config={"solver": "euler"}),
    }))


def _checkpoint(tmp_path, stops=False, lm_shape=BACKBONE):
    """A VoxCPM2-named checkpoint; unless `stops`, the stop head's two rows are the same, so that
    its logits tie and it never says to stop (a tie goes on: patch.rs:232-235)."""
    from tgx.synth import StackSpec, bf16_round, encoder_weights, lm_side_weights, normal, sampler_weights

    base, residual = StackSpec(layers=2, seed=71, **lm_shape), StackSpec(layers=1, seed=72, **lm_shape)
    dit, local = StackSpec(layers=1, seed=73), StackSpec(layers=1, seed=74)
    lm_w = lm_side_weights(base, residual, 1024, 1024, LATENT)
    dit_w, enc_w = sampler_weights(dit, FEAT), encoder_weights(local, FEAT)
    e = {}
    e.update(_stack_entries({k[8:]: v for k, v in lm_w.items() if k.startswith("base_lm.")}, "base_lm.", base))
    e.update(_stack_entries({k[12:]: v for k, v in lm_w.items() if k.startswith("residual_lm.")}, "residual_lm.", residual))
    e.update({k: v for k, v in lm_w.items() if not k.startswith(("base_lm.", "residual_lm."))})
    e.update(_stack_entries(dit_w, "feat_decoder.estimator.decoder.", dit))
    e.update({f"feat_decoder.estimator.{k}": v for k, v in dit_w.items() if not k.startswith(("layers.", "norm"))})
    e.update(_stack_entries(enc_w, "feat_encoder.encoder.", local))
    e.update({f"feat_encoder.{k}": v for k, v in enc_w.items() if not k.startswith(("layers.", "norm"))})
    if not stops:
        e["stop_head.weight"] = np.stack([e["stop_head.weight"][0]] * 2)
    h = lm_shape["hidden"]
    e["base_lm.embed_tokens.weight"] = bf16_round(normal(75, "embed_tokens", VOCAB * h, np.float32)).reshape(VOCAB, h)
    path = tmp_path / "model.safetensors"
    _save(path, e)
    return path


def _prompt(seed):
    from tgx.prompt import Prompt

    rng = np.random.default_rng(seed)
    n = len(LAYOUT)
    return Prompt(rng.integers(0, VOCAB, n).astype(np.uint32), rng.standard_normal((n, FRAMES, FEAT)).astype(np.float32),
                  np.array(LAYOUT, dtype=np.uint8)), rng.standard_normal((4 * FRAMES, FEAT)).astype(np.float32)


def _engine(ctx, ck, slots=4, lm_shape=BACKBONE):
    from tgx.engine import Engine, Settings

    return Engine.from_config(ctx, _config(lm_shape), ck, Settings(slots=slots, capacity=256, max_rows=64, timesteps=10,
                                                           prompt_cache_bytes=1 << 28))


def _noise(seed, slots):
    return np.random.default_rng(seed).standard_normal((slots, FEAT, FRAMES)).astype(np.float32)


def _generate(engine, steps):
    """`steps` steps of the engine, noise drawn per step; the outcomes of each step by slot."""
    out = []
    for k in range(steps):
        outcomes = engine.step(_noise(100 + k, engine.settings.slots))
        out.append({o.slot: o for o in outcomes})
    return out


@pytest.mark.parametrize("lm_shape", [BACKBONE, VOXCPM2], ids=["backbone", "voxcpm2"])
def test_requests_step_together_as_each_does_alone(ctx, tmp_path, lm_shape):
    """Two requests started from their prompts and stepped together, then the first again alone
    in another slot with the same noise: bit for bit. At the backbone's LM width and at VoxCPM2's
    own (2048 wide, FFN 6144, heads of 128), built from config.json sizes and a checkpoint."""
    from tgx import TgxError
    from tgx.checkpoint import Checkpoint

    print(f"[engine] LMs {lm_shape}", flush=True)
    ck = Checkpoint(_checkpoint(tmp_path, lm_shape=lm_shape))
    (pa, va), (pb, vb) = _prompt(81), _prompt(82)
    engine = _engine(ctx, ck, lm_shape=lm_shape)
    assert engine.slots() == 4
    assert engine.start(0, pa, va, max_patches=3, temperature=1.0, cfg=2.0) == len(pa)
    assert engine.start(2, pb, vb, max_patches=5, temperature=0.8, cfg=1.5) == len(pb)
    together = _generate(engine, 5)
    for k, step in enumerate(together):
        print(f"[engine] step {k}: " + ", ".join(f"slot {s} last {o.last} stop {np.round(o.stop_logits, 4).tolist()}"
                                                for s, o in step.items()), flush=True)
    # Each request's outcomes follow its stop head and its most patches; it steps until its last.
    for slot, most in ((0, 3), (2, 5)):
        sampled = 0
        for k, step in enumerate(together):
            if slot not in step:
                assert sampled and together[k - 1][slot].last
                break
            o = step[slot]
            assert o.status == 0 and o.frames.shape == (FRAMES, FEAT) and np.isfinite(o.frames).all()
            sampled += 1
            assert o.last == (o.stop_logits[1] > o.stop_logits[0] or sampled == most), (slot, k)
            if o.last:
                break
    frames_a = engine.finish(0)
    assert frames_a.shape == (FRAMES * sum(0 in s for s in together), FEAT)
    with pytest.raises(TgxError):
        engine.finish(0)  # nothing under way there any more
    # The same request alone, in another slot, with the same noise at each step: bit for bit.
    engine.start(3, pa, va, max_patches=3, temperature=1.0, cfg=2.0)
    alone = []
    for k in range(len(together)):
        noise = _noise(100 + k, 4)
        noise[3] = noise[0]  # the noise slot 0 drew beside the other
        step = {o.slot: o for o in engine.step(noise)}
        if 3 not in step:
            break
        alone.append(step[3])
    got = [s[0] for s in together if 0 in s]
    assert len(alone) == len(got)
    for a, b in zip(alone, got):
        assert np.array_equal(a.frames, b.frames) and a.stop_logits == b.stop_logits
    assert np.array_equal(engine.finish(3), frames_a)
    engine.close()
    ck.close()


def test_teacher_forcing_a_patch_before_and_what_the_engine_refuses(ctx, tmp_path):
    from tgx import TgxError
    from tgx.checkpoint import Checkpoint

    ck = Checkpoint(_checkpoint(tmp_path))
    (pa, va), _ = _prompt(83), None
    engine = _engine(ctx, ck, slots=2)
    results = []
    for forced in (None, "same", "other"):
        engine.start(1, pa, va, max_patches=2)
        first = engine.step(_noise(200, 2))[0]
        assert not first.last
        if forced == "same":
            engine.sample_after(1, first.frames)
        elif forced == "other":
            engine.sample_after(1, np.zeros((FRAMES, FEAT), np.float32))
        results.append(engine.step(_noise(201, 2))[0])
        levels = engine.levels(1)  # the quantizer's levels the patch was sampled after: integers
        assert levels.shape == (LATENT,) and np.all(levels == np.round(levels)) and np.abs(levels).max() <= LEVELS
        engine.finish(1)
    assert np.array_equal(results[0].frames, results[1].frames)  # after its own patch: as without
    assert not np.array_equal(results[0].frames, results[2].frames)
    for bad in (lambda: engine.start(2, pa, va, max_patches=1),           # no such slot
                lambda: engine.start(0, pa, va, max_patches=256),         # past the cache
                lambda: engine.sample_after(0, np.zeros((FRAMES, FEAT), np.float32))):  # no request
        with pytest.raises(TgxError) as e:
            bad()
        assert e.value.kind == "shape"
    assert engine.step(_noise(202, 2)) == []  # nothing under way
    engine.close()
    ck.close()


def test_the_stop_heads_argmax_ends_a_request_before_its_most(ctx, tmp_path):
    from tgx.checkpoint import Checkpoint

    ck = Checkpoint(_checkpoint(tmp_path, stops=True))
    (pa, va) = _prompt(84)
    engine = _engine(ctx, ck, slots=2)
    engine.start(0, pa, va, max_patches=5)
    sampled = 0
    while True:
        step = engine.step(_noise(300 + sampled, 2))
        if not step:
            break
        (o,) = step
        sampled += 1
        assert o.last == (o.stop_logits[1] > o.stop_logits[0] or sampled == 5)
        if o.last:
            break
    print(f"[engine] stopped after {sampled} of at most 5 patches, logits {o.stop_logits}", flush=True)
    assert engine.step(_noise(399, 2)) == [] and len(engine.finish(0)) == FRAMES * sampled
    engine.close()
    ck.close()
