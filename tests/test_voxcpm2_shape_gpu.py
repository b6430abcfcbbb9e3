"""VoxCPM2's own LM shape on the GPU against the oracle: hidden 2048, an FFN of 6144, 16 query heads
over 2 KV heads of 128 dimensions (crates/graph/src/decode.rs:919-933,
crates/graph/src/lm_side.rs:665-679), a few layers of it with bf16 weights drawn N(0, 0.02).

- The decoder and the prefill: two runs prefilled at once in two slots (one of 700 positions, so
  that the decode attention's waves take more than two turns each), both against the oracle per
  position; each run bit for bit as alone; then decode steps of both rows against the oracle, each
  row bit for bit as alone; the cache the kernels wrote against the oracle's.
- The LM side at that width (2 base layers, 1 residual layer without RoPE, the heads between them
  from and to the 1024-wide encoder and DiT): every stage against the oracle fed the GPU's input.

Tolerance (bf16 on the GPU against the float64 oracle over the same bf16 weights): cosine >= 0.999
and max|got - ref| / max|ref| <= 1e-2, per position or step.
"""

import numpy as np
import pytest

from conftest import distance, within

pytestmark = pytest.mark.gpu

LM = dict(hidden=2048, inner=6144, heads=16, kv_heads=2, head_dim=128)


def lm_spec(layers, seed, rope=True):
    from tgx.synth import StackSpec

    return StackSpec(layers=layers, dtype="bf16", seed=seed, **LM)


def make_decoder(ctx, spec, capacity, rows=1, slots=None, rope=True, weights=None):
    import tgx
    from tgx.synth import stack_weights

    shape = tgx.Shape(layers=spec.layers, capacity=capacity, eps=spec.eps, rope_theta=spec.rope_theta, rope=rope, **LM)
    dec = tgx.Decoder(ctx, shape, tgx.Batch(rows=rows, slots=slots or rows))
    dec.load_all(weights if weights is not None else stack_weights(spec))
    return dec


def test_voxcpm2_lm_prefill_and_decode_match_the_oracle_and_rows_are_as_alone(ctx):
    import oracle
    import tgx
    from tgx.synth import bf16_round, embeddings, stack_weights

    spec = lm_spec(2, seed=31)
    w = stack_weights(spec)
    wr = {k: bf16_round(v) for k, v in w.items()}
    cap, lengths, steps = 1024, (700, 45), 6
    print(f"[voxcpm2] decoder {LM}, 2 layers, runs {lengths}, {steps} steps", flush=True)
    x = embeddings(spec.seed + 1, "x", sum(lengths) + 2 * steps, spec.hidden)
    runs_x = [x[:700], x[700:745]]
    dec = make_decoder(ctx, spec, cap, rows=2, slots=2, weights=w)
    together = dec.prefill_runs([(0, 0, 700), (1, 0, 45)], x[:745])
    refs = []
    row = 0
    for slot, n in enumerate(lengths):
        ref = oracle.Stack(spec, wr, cap, "f64")
        want = ref.prefill_rows(0, runs_x[slot])
        refs.append(ref)
        worst = None
        for t in range(n):
            d = distance(together[row + t], want[t])
            assert within(d), f"run {slot} position {t}: {d}"
            worst = d if worst is None or d["cosine"] < worst["cosine"] else worst
        print(f"[voxcpm2] prefill run {slot} ({n} positions) worst {worst}", flush=True)
        alone = make_decoder(ctx, spec, cap, weights=w)
        got = alone.prefill(0, runs_x[slot])
        assert np.array_equal(got.view(np.uint32), together[row : row + n].view(np.uint32)), f"run {slot} alone"
        alone.close()
        row += n
    alones = []
    for slot in range(2):
        a = make_decoder(ctx, spec, cap, weights=w)
        a.prefill(0, runs_x[slot])
        alones.append(a)
    xs = x[745:].reshape(steps, 2, spec.hidden)
    for s in range(steps):
        got = dec.step_rows([tgx.Row(lengths[0] + s, 0), tgx.Row(lengths[1] + s, 1)], xs[s])
        for b in range(2):
            d = distance(got[b], refs[b].decode(lengths[b] + s, xs[s, b]))
            assert within(d), f"row {b} step {s}: {d}"
            one = alones[b].step(lengths[b] + s, xs[s, b])
            assert np.array_equal(one.view(np.uint32), got[b].view(np.uint32)), f"row {b} step {s} alone"
        print(f"[voxcpm2] decode step {s}: both rows within tolerance and as alone, last {d}", flush=True)
    # The caches the prefill and the steps wrote, against the oracle's (rounded to bf16 there).
    for slot, n in enumerate(lengths):
        k, v = dec.read_cache(slot, n + steps)
        for name, got, want in (("k", k, refs[slot].k[:, :, : n + steps]), ("v", v, refs[slot].v[:, :, : n + steps])):
            d = distance(got, want)
            assert within(d), f"slot {slot} {name} cache: {d}"
    for a in alones:
        a.close()
    dec.close()


def test_voxcpm2_lm_side_matches_the_oracle_stage_by_stage_and_a_row_is_as_alone(ctx):
    """LmSide (crates/graph/src/lm_side.rs:246-491) at VoxCPM2's LM width: enc_to_lm_proj from the
    1024-wide encoder, the base LM, the quantizer (fsq_layer, 512 latents, 9 levels), the residual
    LM, fusion_concat_proj over two 2048-wide rows, the stop head and mu for the 1024-wide DiT."""
    import oracle
    import patch_oracle as po
    import tgx
    from tgx.patch import HeadsShape, LmSide
    from tgx.synth import lm_side_weights

    latent, levels, rows, steps, cap = 512, 9, 3, 3, 256
    base_spec, res_spec = lm_spec(2, seed=41), lm_spec(1, seed=42)
    w = lm_side_weights(base_spec, res_spec, 1024, 1024, latent)

    def side_of(n):
        base = tgx.Shape(layers=2, capacity=cap, **LM)
        residual = tgx.Shape(layers=1, capacity=cap, rope=False, **LM)
        s = LmSide(ctx, base, residual, tgx.Batch(rows=n, slots=n), HeadsShape(1024, 1024, latent, levels))
        s.load_all(w)
        return s

    strip = lambda prefix: {k[len(prefix):]: v for k, v in w.items() if k.startswith(prefix)}
    side = side_of(rows)
    base = [oracle.Stack(base_spec, strip("base_lm."), cap, "f64") for _ in range(rows)]
    res = [oracle.Stack(res_spec, strip("residual_lm."), cap, "f64", rope=False) for _ in range(rows)]
    rng = np.random.default_rng(17)
    record = []
    for step in range(steps):
        enc = rng.standard_normal((rows, 1024)).astype(np.float32)
        mu, stop = side.step_rows([tgx.Row(step, r) for r in range(rows)], enc)
        record.append((enc, mu, stop))
        t = {n: side.read(n) for n in side.TENSORS}
        checks = {"embed": (t["embed"], po.linear(w, "enc_to_lm_proj", enc)),
                  "base_out": (t["base_out"], np.stack([base[r].decode(step, t["embed"][r]) for r in range(rows)]))}
        pre, lv = po.quantizer(w, t["base_out"], levels)
        diff = t["levels"] != lv.astype(np.float32)
        if diff.any():
            frac = np.abs(np.tanh(np.abs(pre[diff])) * levels % 1.0 - 0.5)
            assert np.all(frac < 0.05) and diff.mean() < 0.05, frac
        lm_hidden, residual_in, to_dit, stop_hidden, logits = po.heads_after_levels(w, t["levels"], t["embed"])
        checks["lm_hidden"] = (t["lm_hidden"], lm_hidden)
        checks["residual_in"] = (t["residual_in"], residual_in)
        checks["mu[:dit]"] = (mu[:, :1024], to_dit)
        checks["stop_hidden"] = (t["stop_hidden"], stop_hidden)
        bound = 2.0**-8 * (np.abs(w["stop_head.weight"]).astype(np.float64) @ np.abs(t["stop_hidden"]).T).T
        assert np.all(np.abs(stop - logits) <= bound + 1e-7), (step, stop, logits)
        checks["residual_out"] = (t["residual_out"], np.stack([res[r].decode(step, t["residual_in"][r]) for r in range(rows)]))
        checks["mu[dit:]"] = (mu[:, 1024:], po.linear(w, "res_to_dit_proj", t["residual_out"]))
        for name, (got, want) in checks.items():
            for r in range(rows):
                d = distance(got[r], want[r])
                assert within(d), f"step {step} row {r} {name}: {d}"
        print(f"[voxcpm2] LM side step {step}: every stage within tolerance, {int(diff.sum())} levels at a tie", flush=True)
    side.close()
    one = side_of(1)
    for step, (enc, mu, stop) in enumerate(record):
        m1, s1 = one.step_rows([tgx.Row(step, 0)], enc[1:2])
        assert np.array_equal(m1[0], mu[1]) and np.array_equal(s1[0], stop[1]), f"step {step} row 1 alone"
    one.close()
