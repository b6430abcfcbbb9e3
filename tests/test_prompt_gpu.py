"""The prompt path (crates/graph/src/prompt.rs) on the GPU: a prompt's positions but its last run
through both LMs into a slot of the patch step's caches, checked stage by stage against the oracle
fed the GPU's input to each stage (as the LM side's test does); the first patch step after it
reading the caches the prompt wrote; and the PromptCache: a prompt that begins as a kept one in the
same voice runs only its new positions and leaves the caches as a full run does, bit for bit."""

import numpy as np
import pytest

from conftest import distance, within

pytestmark = pytest.mark.gpu

FEAT, FRAMES, STEPS, LATENT, LEVELS = 64, 4, 10, 256, 9
VOCAB = 48
# A prompt as the service lays one out: the voice's patches, the text, then patches, ending in audio.
LAYOUT = [True] * 4 + [False] * 7 + [True] * 9


def _strip(w, prefix):
    return {k[len(prefix):]: v for k, v in w.items() if k.startswith(prefix)}


class Parts:
    """An LM side, encoder and sampler at 2 rows and 2 slots, their patch step, and a checkpoint
    holding the base LM's embedding table."""

    def __init__(self, ctx, tmp_path, max_rows=64):
        import torch
        from safetensors.torch import save_file

        import tgx
        from tgx.checkpoint import Checkpoint
        from tgx.patch import Encoder, HeadsShape, LmSide, PatchShape, PatchStep, Sampler
        from tgx.prompt import Prompter
        from tgx.synth import StackSpec, bf16_round, encoder_weights, lm_side_weights, normal, sampler_weights

        self.base, self.residual = StackSpec(layers=2, seed=51), StackSpec(layers=1, seed=52)
        self.local, self.dit = StackSpec(layers=1, seed=53), StackSpec(layers=1, seed=54)
        self.w = lm_side_weights(self.base, self.residual, 1024, 1024, LATENT)
        self.enc_w = encoder_weights(self.local, FEAT)
        patch = PatchShape(FEAT, FRAMES, STEPS, 2)
        self.side = LmSide(ctx, tgx.Shape(layers=2, capacity=256), tgx.Shape(layers=1, capacity=256, rope=False),
                           tgx.Batch(rows=2, slots=2), HeadsShape(1024, 1024, LATENT, LEVELS))
        self.side.load_all(self.w)
        self.enc = Encoder(ctx, tgx.Shape(layers=1, capacity=16), patch)
        self.enc.load_all(self.enc_w)
        self.smp = Sampler(ctx, tgx.Shape(layers=1, capacity=16), patch)
        self.smp.load_all(sampler_weights(self.dit, FEAT))
        self.step = PatchStep(self.enc, self.side, self.smp)
        self.prompter = Prompter(self.step, max_rows)
        table = bf16_round(normal(55, "embed_tokens", VOCAB * 1024, np.float32).reshape(VOCAB, 1024))
        self.table = table
        path = tmp_path / "embed.safetensors"
        save_file({"base_lm.embed_tokens.weight": torch.from_numpy(table).to(torch.bfloat16)}, str(path))
        self.ck = Checkpoint(path)

    def close(self):
        self.ck.close()
        for o in (self.prompter, self.step, self.smp, self.enc, self.side):
            o.close()


def _prompt(seed, voice=None, text=None, layout=LAYOUT):
    from tgx.prompt import Prompt

    rng = np.random.default_rng(seed)
    n = len(layout)
    patches = rng.standard_normal((n, FRAMES, FEAT)).astype(np.float32)
    tokens = rng.integers(0, VOCAB, n).astype(np.uint32)
    if voice is not None:
        patches[: len(voice)] = voice
    if text is not None:
        tokens[4:11] = text
    return Prompt(tokens, patches, np.array(layout, dtype=np.uint8))


def test_a_patch_embeds_as_the_encoder_and_enc_to_lm_proj_do(ctx, tmp_path):
    """Prompter::embed (prompt.rs:559-566): the encoder's output for the patch (laid out as the
    step's cond) through enc_to_lm_proj, bit for bit as the LM side embeds the same encoding, and
    within the tolerance of the oracle's."""
    import patch_oracle as po
    import tgx

    p = Parts(ctx, tmp_path)
    rng = np.random.default_rng(56)
    patch = rng.standard_normal((FRAMES, FEAT)).astype(np.float32)  # [patch_size][feat_dim]
    got = p.prompter.embed(patch)
    cond = np.stack([patch.T, np.zeros((FEAT, FRAMES), np.float32)])
    enc = p.enc.encode(cond)
    p.side.step_rows([tgx.Row(0, 0), tgx.Row(0, 1)], enc)
    assert np.array_equal(got, p.side.read("embed")[0])
    s = po.StackShape(hidden=1024, inner=4096, heads=16, kv_heads=2, layers=1, eps=1e-5, rope_theta=10000.0)
    want = po.linear(p.w, "enc_to_lm_proj", po.encode(p.enc_w, s, FEAT, FRAMES, patch.T[None])[0])
    d = distance(got, want)
    print(f"[prompt] embed: {d}", flush=True)
    assert within(d), d
    p.close()


def test_a_prompt_runs_stage_by_stage_as_the_oracle_and_the_step_after_it_reads_its_caches(ctx, tmp_path):
    import oracle
    import patch_oracle as po
    import tgx

    p = Parts(ctx, tmp_path)
    pr = _prompt(57)
    n = len(pr) - 1
    slot = 1
    p.prompter.run(0, p.ck, _prompt(65))  # the step's other row reads a prompt of its own
    p.prompter.run(slot, p.ck, pr)
    x, audio_x = p.prompter.embeddings(p.ck, pr)
    audio = pr.audio[:n].astype(bool)
    # Text positions are the table's rows, exactly; audio ones the patches' embeddings, zero in x's
    # audio copy at text.
    assert np.array_equal(x[~audio], p.table[pr.tokens[:n][~audio]])
    assert np.all(audio_x[~audio] == 0) and np.array_equal(audio_x[audio], x[audio])
    t = {name: p.prompter.read(name, n) for name in p.prompter.TENSORS}
    base = oracle.Stack(p.base, _strip(p.w, "base_lm."), 256, "f64")
    res = oracle.Stack(p.residual, _strip(p.w, "residual_lm."), 256, "f64", rope=False)
    base_ref = np.stack([base.decode(q, x[q]) for q in range(n)])
    pre, lv = po.quantizer(p.w, t["base_out"], LEVELS)
    diff = (t["levels"] != lv.astype(np.float32))[audio]
    quantized = po.linear(p.w, "fsq_layer.out_proj", t["levels"])
    assert np.array_equal(t["lm_hidden"][~audio], t["base_out"][~audio])  # the base LM's at text
    residual_in = po.linear(p.w, "fusion_concat_proj", np.concatenate([t["lm_hidden"], audio_x], axis=1))
    res_ref = np.stack([res.decode(q, t["residual_in"][q]) for q in range(n)])
    checks = {"base_out": (t["base_out"], base_ref), "quantized": (t["quantized"][audio], quantized[audio]),
              "lm_hidden": (t["lm_hidden"][audio], quantized[audio]), "residual_in": (t["residual_in"], residual_in),
              "residual_out": (t["residual_out"], res_ref)}
    bad = []
    for name, (got, want) in checks.items():
        for r in range(len(got)):
            d = distance(got[r], want[r])
            if r == 0:
                print(f"[prompt] {name}: {d}", flush=True)
            if not within(d):
                bad.append((name, r, d))
    assert not bad, bad[:4]
    # Levels the quantizer rounds the other way only at a tie (as the LM side's test allows).
    if diff.any():
        frac = np.abs(np.tanh(np.abs(pre[audio][diff])) * LEVELS % 1.0 - 0.5)
        assert np.all(frac < 0.05), frac
    assert diff.mean() < 0.05
    # The first patch step runs the last position, the patch before being the prompt's last patch.
    last = pr.patches[n].T
    cond = np.stack([_prompt(65).patches[n].T, last])
    noise = np.random.default_rng(58).standard_normal((2, FEAT, FRAMES)).astype(np.float32)
    sampling = np.array([[1.0, 2.0], [1.0, 2.0]], dtype=np.float32)
    p.step.run_rows([tgx.Row(n, 0), tgx.Row(n, slot)], cond, noise, sampling)
    embed = p.side.read("embed")[1]
    assert np.array_equal(embed, p.prompter.embed(pr.patches[n]))
    d = distance(p.side.read("base_out")[1], base.decode(n, embed))
    print(f"[prompt] the step after it, base_out: {d}", flush=True)
    assert within(d), d
    p.close()


def test_a_prompt_in_a_kept_voice_runs_its_new_positions_alone_and_ends_as_a_full_run(ctx, tmp_path):
    """Prompter::run_cached (prompt.rs:585-641): the voice's positions up to its last text kept
    after the first prompt; a second prompt beginning with them copies their keys and values back
    and runs the rest; the step after it is bit for bit the step after the same prompt run whole."""
    import tgx
    from tgx.prompt import PromptCache

    p = Parts(ctx, tmp_path, max_rows=8)  # runs in pieces of 8
    rng = np.random.default_rng(59)
    voice = rng.standard_normal((4, FRAMES, FEAT)).astype(np.float32)
    text = rng.integers(0, VOCAB, 7).astype(np.uint32)
    first, second = _prompt(60, voice, text), _prompt(61, voice, text)
    n = len(first) - 1
    cache = PromptCache(ctx, 1 << 30)
    assert p.prompter.run_cached(0, p.ck, first, voice, cache) == len(first)
    assert cache.voices() == 1 and cache.bytes() > 0
    held = 11  # the voice's 4 patches and the 7 tokens
    assert p.prompter.run_cached(1, p.ck, second, voice, cache) == len(second) - held
    p.prompter.run(0, p.ck, second)  # the same prompt run whole into slot 0
    last = second.patches[n].T
    noise = np.random.default_rng(62).standard_normal((1, FEAT, FRAMES)).astype(np.float32)
    cond, noise2 = np.stack([last, last]), np.concatenate([noise, noise])
    sampling = np.array([[1.0, 2.0], [1.0, 2.0]], dtype=np.float32)
    patch, stop = p.step.run_rows([tgx.Row(n, 0), tgx.Row(n, 1)], cond, noise2, sampling)
    print(f"[prompt] whole vs kept: stop {stop.tolist()}", flush=True)
    assert np.array_equal(patch[0], patch[1]) and np.array_equal(stop[0], stop[1])
    # Another voice within a budget for one: the one used longest ago makes room.
    small = PromptCache(ctx, cache.bytes() + 1024)
    assert p.prompter.run_cached(0, p.ck, first, voice, small) == len(first)
    other = rng.standard_normal((4, FRAMES, FEAT)).astype(np.float32)
    p.prompter.run_cached(1, p.ck, _prompt(63, other, text), other, small)
    assert small.voices() == 1 and small.bytes() <= cache.bytes() + 1024
    for c in (cache, small):
        c.close()
    p.close()


def test_a_prompt_that_does_not_end_in_audio_is_refused(ctx, tmp_path):
    import tgx

    p = Parts(ctx, tmp_path)
    pr = _prompt(64, layout=[True] * 3 + [False] * 2)
    with pytest.raises(tgx.TgxError) as e:
        p.prompter.run(0, p.ck, pr)
    assert e.value.kind == "shape" and "must end in audio" in str(e.value)
    p.close()
