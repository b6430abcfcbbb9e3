"""The patch sampler and the LM side on the GPU against the oracle (oracle/patch_oracle.py):
the local DiT's Euler steps with CFG-Zero* (crates/graph/src/local/dit.rs) and the layers between
the LMs with both LMs (crates/graph/src/lm_side.rs), at the workload's shape (hidden 1024, 16/2
heads, FFN 4096, a 4-layer DiT over patches of 4 frames x 64 channels, 10 steps, guidance 2.0).

Tolerance, as for the decoder: cosine >= 0.999 and max|got - ref| / max|ref| <= 1e-2 (bf16
weights and activations against float64). The patch is compared twice: whole, and as what the
Euler steps moved it (patch - temperature noise), which the noise it starts from would otherwise
hide. Rows are independent: a row sampled beside others comes out bit for bit as alone."""

import numpy as np
import pytest

from conftest import COSINE_MIN, REL_MAX, distance, within

pytestmark = pytest.mark.gpu

FEAT, FRAMES, STEPS = 64, 4, 10


def _dit_spec(layers=4):
    from tgx.synth import StackSpec

    return StackSpec(layers=layers, hidden=1024, inner=4096, dtype="bf16", seed=11)


def _sampler(ctx, rows, spec, weights, timesteps=STEPS):
    import tgx
    from tgx.patch import PatchShape, Sampler

    shape = tgx.Shape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads,
                      head_dim=spec.head_dim, layers=spec.layers, capacity=16, eps=spec.eps,
                      rope_theta=spec.rope_theta)
    s = Sampler(ctx, shape, PatchShape(FEAT, FRAMES, timesteps, rows))
    s.load_all(weights)
    return s


def _inputs(rows, seed=5):
    rng = np.random.default_rng(seed)
    mu = rng.standard_normal((rows, 2, 1024)).astype(np.float32)
    cond = rng.standard_normal((rows, FEAT, FRAMES)).astype(np.float32)
    noise = rng.standard_normal((rows, FEAT, FRAMES)).astype(np.float32)
    sampling = np.array([[1.0, 2.0]] * rows, dtype=np.float32)
    if rows > 1:
        sampling[1] = [0.7, 1.5]
    return mu, cond, noise, sampling


def _oracle(spec, weights, mu, cond, noise, sampling, timesteps=STEPS, rope_on=True):
    import patch_oracle as po

    s = po.StackShape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads,
                      layers=spec.layers, eps=spec.eps, rope_theta=spec.rope_theta)
    return po.sample(weights, s, FEAT, FRAMES, timesteps, mu, cond, noise, sampling, rope_on)


def test_the_sampler_matches_the_oracle(ctx):
    from tgx.synth import sampler_weights

    spec = _dit_spec()
    w = sampler_weights(spec, FEAT)
    rows = 3
    mu, cond, noise, sampling = _inputs(rows)
    s = _sampler(ctx, rows, spec, w)
    print(f"[sampler] rows {rows}, {s.dispatches()} dispatches", flush=True)
    got = s.sample(mu, cond, noise, sampling)
    x0, want = _oracle(spec, w, mu, cond, noise, sampling)
    for r in range(rows):
        moved = distance(got[r] - x0[r], want[r] - x0[r])
        whole = distance(got[r], want[r])
        print(f"[sampler] row {r}: moved {moved}, whole {whole}", flush=True)
        assert within(moved), moved
        assert within(whole), whole
    s.close()


def test_a_planted_defect_in_the_oracle_is_caught(ctx):
    """The same comparison against the oracle without RoPE in the DiT must fail it."""
    from tgx.synth import sampler_weights

    spec = _dit_spec(2)
    w = sampler_weights(spec, FEAT)
    mu, cond, noise, sampling = _inputs(1)
    s = _sampler(ctx, 1, spec, w)
    got = s.sample(mu, cond, noise, sampling)
    x0, want = _oracle(spec, w, mu, cond, noise, sampling)
    _, wrong = _oracle(spec, w, mu, cond, noise, sampling, rope_on=False)
    assert within(distance(got[0] - x0[0], want[0] - x0[0]))
    assert not within(distance(got[0] - x0[0], wrong[0] - x0[0]))
    s.close()


def test_a_row_samples_the_same_patch_beside_others_as_alone(ctx):
    from tgx.synth import sampler_weights

    spec = _dit_spec()
    w = sampler_weights(spec, FEAT)
    mu, cond, noise, sampling = _inputs(16, seed=9)
    one = _sampler(ctx, 1, spec, w)
    # 1 row (22 tokens) takes the direct GEMMs; 5 rows (110 tokens, 128 padded) and 16 (352, 384)
    # the ring GEMMs with 8 token tiles to a gate/up workgroup, 6 rows (132, 192) with 4.
    for rows, picks in ((5, (0, 3)), (6, (5,)), (16, (0, 9, 15))):
        many = _sampler(ctx, rows, spec, w)
        got = many.sample(mu[:rows], cond[:rows], noise[:rows], sampling[:rows])
        again = many.sample(mu[:rows], cond[:rows], noise[:rows], sampling[:rows])
        assert np.array_equal(got, again)
        many.close()
        for r in picks:
            alone = one.sample(mu[r : r + 1], cond[r : r + 1], noise[r : r + 1], sampling[r : r + 1])
            assert np.array_equal(alone[0], got[r]), (rows, r)
    one.close()


def test_repeated_samples_are_the_same_bits(ctx):
    """The same inputs sampled again and again give the same bits: at 5 rows (128 tokens, the ring
    GEMM with 4 and 8 token tiles) and 16 rows (384), every workgroup's loads, waits and barriers
    read what they wait for (a race would show as a sample that differs from the first)."""
    from tgx.synth import sampler_weights

    spec = _dit_spec()
    w = sampler_weights(spec, FEAT)
    for rows in (5, 16):
        s = _sampler(ctx, rows, spec, w)
        mu, cond, noise, sampling = _inputs(rows, seed=13)
        first = s.sample(mu, cond, noise, sampling)
        for i in range(12):
            again = s.sample(mu, cond, noise, sampling)
            assert np.array_equal(first, again), (rows, i)
        s.close()


def test_with_out_proj_reading_nothing_the_patch_is_the_euler_closed_form(ctx):
    import patch_oracle as po
    from tgx.synth import sampler_weights

    spec = _dit_spec(1)
    w = dict(sampler_weights(spec, FEAT))
    w["out_proj.weight"] = np.zeros_like(w["out_proj.weight"])
    mu, cond, noise, sampling = _inputs(2, seed=4)
    s = _sampler(ctx, 2, spec, w)
    got = s.sample(mu, cond, noise, sampling)
    b = np.asarray(w["out_proj.bias"], np.float64)[:, None] * np.ones((1, FRAMES))
    total = sum(dt for _, dt in po.euler_steps(STEPS))
    for r in range(2):
        want = sampling[r, 0].astype(np.float64) * noise[r] - total * po.cfg_zero_star(b, b, float(sampling[r, 1]))
        assert np.max(np.abs(got[r] - want)) < 1e-5
    s.close()


def test_the_sampler_refuses_what_it_cannot_run(ctx):
    import tgx
    from tgx.patch import PatchShape, Sampler

    shape = tgx.Shape(layers=1, capacity=16)
    for p in (PatchShape(64, 8, 10, 1), PatchShape(60, 4, 10, 1), PatchShape(64, 4, 0, 1), PatchShape(64, 4, 10, 0)):
        with pytest.raises(tgx.TgxError) as e:
            Sampler(ctx, shape, p)
        assert e.value.kind == "shape"
    s = Sampler(ctx, shape, PatchShape(64, 4, 10, 1))
    with pytest.raises(tgx.TgxError) as e:
        s.load("in_proj.weight", np.zeros(10, np.float32))
    assert e.value.kind == "weights"
    with pytest.raises(tgx.TgxError) as e:  # the time MLPs are not loaded
        s.sample(*_inputs(1))
    assert e.value.kind == "weights"
    s.close()


# ---- the LM side ----

BASE_LAYERS, RESIDUAL_LAYERS, LATENT, LEVELS = 3, 2, 256, 9


def _lm_side(ctx, rows, w):
    import tgx
    from tgx.patch import HeadsShape, LmSide

    base = tgx.Shape(layers=BASE_LAYERS, capacity=256)
    residual = tgx.Shape(layers=RESIDUAL_LAYERS, capacity=256, rope=False)
    side = LmSide(ctx, base, residual, tgx.Batch(rows=rows, slots=rows), HeadsShape(1024, 1024, LATENT, LEVELS))
    side.load_all(w)
    return side


def _lm_weights():
    from tgx.synth import StackSpec, lm_side_weights

    base = StackSpec(layers=BASE_LAYERS, seed=21)
    residual = StackSpec(layers=RESIDUAL_LAYERS, seed=22)
    return base, residual, lm_side_weights(base, residual, 1024, 1024, LATENT)


def _strip(w, prefix):
    return {k[len(prefix):]: v for k, v in w.items() if k.startswith(prefix)}


def test_the_lm_side_matches_the_oracle_stage_by_stage(ctx):
    """Each stage against the oracle fed the GPU's input to it, so that a level the quantizer
    rounds the other way near a tie does not carry on: the levels may differ from the oracle's only
    by one step, only where the oracle's value sits within 5 % of a step of the boundary (the
    quantizer's input is summed from bf16 weights and activations), and at few places."""
    import oracle
    import patch_oracle as po
    import tgx

    base_spec, res_spec, w = _lm_weights()
    rows, steps = 3, 4
    side = _lm_side(ctx, rows, w)
    print(f"[lm_side] rows {rows}, {side.dispatches()} dispatches", flush=True)
    base = [oracle.Stack(base_spec, _strip(w, "base_lm."), 256, "f64") for _ in range(rows)]
    res = [oracle.Stack(res_spec, _strip(w, "residual_lm."), 256, "f64", rope=False) for _ in range(rows)]
    rng = np.random.default_rng(7)
    for step in range(steps):
        enc = rng.standard_normal((rows, 1024)).astype(np.float32)
        rows_at = [tgx.Row(step, r) for r in range(rows)]
        mu, stop = side.step_rows(rows_at, enc)
        t = {n: side.read(n) for n in side.TENSORS}
        assert np.array_equal(t["mu"], mu) and np.array_equal(t["stop_logits"], stop)
        checks = {"embed": (t["embed"], po.linear(w, "enc_to_lm_proj", enc))}
        base_ref = np.stack([base[r].decode(step, t["embed"][r]) for r in range(rows)])
        checks["base_out"] = (t["base_out"], base_ref)
        pre, lv = po.quantizer(w, t["base_out"], LEVELS)
        lv = lv.astype(np.float32)  # k / L as the GPU stores it
        diff = t["levels"] != lv
        lm_hidden, residual_in, to_dit, stop_hidden, logits = po.heads_after_levels(w, t["levels"], t["embed"])
        checks["lm_hidden"] = (t["lm_hidden"], lm_hidden)
        checks["residual_in"] = (t["residual_in"], residual_in)
        checks["mu[:dit]"] = (mu[:, :1024], to_dit)
        checks["stop_hidden"] = (t["stop_hidden"], stop_hidden)
        # Two logits from a sum that cancels: bounded as a bf16 dot product is (the reference's
        # bound for its GEMVs, crates/vulkan/tests/glsl.rs:170-186, at bf16's unit roundoff):
        # |got - ref| <= 2^-8 sum_k |W[n][k] x[k]|.
        bound = 2.0**-8 * (np.abs(w["stop_head.weight"]).astype(np.float64) @ np.abs(t["stop_hidden"]).T).T
        assert np.all(np.abs(stop - logits) <= bound + 1e-7), (step, stop, logits, bound)
        res_ref = np.stack([res[r].decode(step, t["residual_in"][r]) for r in range(rows)])
        checks["residual_out"] = (t["residual_out"], res_ref)
        checks["mu[dit:]"] = (mu[:, 1024:], po.linear(w, "res_to_dit_proj", t["residual_out"]))
        bad = []
        for name, (got, want) in checks.items():
            for r in range(rows):
                d = distance(got[r], want[r])
                if r == 0:
                    print(f"[lm_side] step {step} {name}: {d}", flush=True)
                if not within(d):
                    bad.append((name, r, d))
        if diff.any():
            i = np.argwhere(diff)[:6]
            print(f"[lm_side] step {step}: {int(diff.sum())} of {diff.size} levels differ; e.g. rows/cols {i.tolist()} "
                  f"gpu {t['levels'][diff][:6]} oracle {lv[diff][:6]} pre {pre[diff][:6]}", flush=True)
        assert not bad, bad
        if diff.any():
            frac = np.abs(np.tanh(np.abs(pre[diff])) * LEVELS % 1.0 - 0.5)
            assert np.all(frac < 0.05), frac
            assert np.allclose(np.abs(t["levels"][diff] - lv[diff]), 1.0 / LEVELS)
        assert diff.mean() < 0.05
        print(f"[lm_side] step {step}: every stage within tolerance; {int(diff.sum())} levels at a tie", flush=True)
    side.close()


def test_a_row_of_the_lm_side_is_the_same_beside_others_as_alone(ctx):
    import tgx

    _, _, w = _lm_weights()
    rng = np.random.default_rng(8)
    encs = [rng.standard_normal((4, 1024)).astype(np.float32) for _ in range(3)]
    many = _lm_side(ctx, 4, w)
    outs = [many.step_rows([tgx.Row(s, r) for r in range(4)], encs[s]) for s in range(3)]
    many.close()
    one = _lm_side(ctx, 1, w)
    for s in range(3):
        mu, stop = one.step_rows([tgx.Row(s, 0)], encs[s][2:3])
        assert np.array_equal(mu[0], outs[s][0][2]) and np.array_equal(stop[0], outs[s][1][2]), s
    one.close()


# ---- the local encoder and the whole patch step ----

def _encoder(ctx, rows, spec, weights):
    import tgx
    from tgx.patch import Encoder, PatchShape

    shape = tgx.Shape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads,
                      head_dim=spec.head_dim, layers=spec.layers, capacity=16, eps=spec.eps,
                      rope_theta=spec.rope_theta)
    e = Encoder(ctx, shape, PatchShape(FEAT, FRAMES, STEPS, rows))
    e.load_all(weights)
    return e


def _encoder_spec(layers=4):
    from tgx.synth import StackSpec

    return StackSpec(layers=layers, hidden=1024, inner=4096, dtype="bf16", seed=13)


def test_the_encoder_matches_the_oracle_and_a_row_encodes_as_alone(ctx):
    """Encoder::encode (crates/graph/src/local/encoder.rs:194-198) against the oracle within the
    tolerance; the frames reversed (which only RoPE tells apart) must fail it; a row beside others
    is bit for bit as alone."""
    import patch_oracle as po
    from tgx.synth import encoder_weights

    spec = _encoder_spec()
    w = encoder_weights(spec, FEAT)
    rng = np.random.default_rng(14)
    patches = rng.standard_normal((3, FEAT, FRAMES)).astype(np.float32)
    e = _encoder(ctx, 3, spec, w)
    print(f"[encoder] rows 3, {e.dispatches()} dispatches", flush=True)
    got = e.encode(patches)
    assert np.array_equal(got, e.encode(patches))
    s = po.StackShape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads,
                      layers=spec.layers, eps=spec.eps, rope_theta=spec.rope_theta)
    want = po.encode(w, s, FEAT, FRAMES, patches)
    for r in range(3):
        d = distance(got[r], want[r])
        print(f"[encoder] row {r}: {d}", flush=True)
        assert within(d), (r, d)
    wrong = po.encode(w, s, FEAT, FRAMES, patches[:, :, ::-1])
    assert not all(within(distance(got[r], wrong[r])) for r in range(3))
    e.close()
    one = _encoder(ctx, 1, spec, w)
    assert np.array_equal(one.encode(patches[2:3])[0], got[2])
    one.close()


def test_the_patch_step_is_the_encoder_the_lm_side_and_the_sampler_in_turn(ctx):
    """PatchStep::run_rows (crates/graph/src/patch.rs:356-415) on the device throughout gives, bit
    for bit, what the three give when each is run alone and the host hands their outputs on:
    the encoder's embedding of the patch before to the LM side, its mu to the sampler."""
    import tgx
    from tgx.patch import PatchStep
    from tgx.synth import encoder_weights, sampler_weights

    rows = 3
    espec, dspec = _encoder_spec(2), _dit_spec(2)
    enc = _encoder(ctx, rows, espec, encoder_weights(espec, FEAT))
    smp = _sampler(ctx, rows, dspec, sampler_weights(dspec, FEAT))
    _, _, w = _lm_weights()
    side = _lm_side(ctx, rows, w)
    _, cond, noise, sampling = _inputs(rows, seed=15)
    at = [tgx.Row(0, r) for r in range(rows)]
    embedding = enc.encode(cond)
    mu, stop = side.step_rows(at, embedding)
    patch = smp.sample(mu, cond, noise, sampling)
    step = PatchStep(enc, side, smp)
    got_patch, got_stop = step.run_rows(at, cond, noise, sampling)
    assert np.array_equal(got_stop, stop)
    assert np.array_equal(got_patch, patch)
    # On to the next position, launched over what the device holds, then read back.
    at1 = [tgx.Row(1, r) for r in range(rows)]
    mu1, stop1 = side.step_rows(at1, embedding)
    patch1 = smp.sample(mu1, cond, noise, sampling)
    got_patch1, got_stop1 = step.run_rows(at1, cond, noise, sampling)
    assert np.array_equal(got_patch1, patch1) and np.array_equal(got_stop1, stop1)
    step.close()
    for o in (enc, smp, side):
        o.close()


def test_launched_patch_steps_move_the_rows_on_as_single_runs_do(ctx):
    """PatchStep launched over what the device holds (the benchmark's path: each placed row moved
    on a position by the step): a run at position p, k launched steps (p again, then on) and a run
    at p + k give what runs at p, p + 1, ..., p + k give, bit for bit."""
    import tgx
    from tgx.patch import PatchStep
    from tgx.synth import encoder_weights, sampler_weights

    rows, k = 2, 3
    espec, dspec = _encoder_spec(1), _dit_spec(1)
    _, _, w = _lm_weights()
    _, cond, noise, sampling = _inputs(rows, seed=17)
    steps = []
    for _ in range(2):
        enc = _encoder(ctx, rows, espec, encoder_weights(espec, FEAT))
        smp = _sampler(ctx, rows, dspec, sampler_weights(dspec, FEAT))
        side = _lm_side(ctx, rows, w)
        steps.append((PatchStep(enc, side, smp), enc, smp, side))
    a, b = steps[0][0], steps[1][0]
    at = lambda t: [tgx.Row(t, r) for r in range(rows)]
    a.run_rows(at(0), cond, noise, sampling)
    a.launch(k, advance=True)
    a.wait()
    got = a.run_rows(at(k), cond, noise, sampling)
    for t in range(k + 1):
        want = b.run_rows(at(t), cond, noise, sampling)
    assert np.array_equal(got[0], want[0]) and np.array_equal(got[1], want[1])
    for step, *parts in steps:
        step.close()
        for o in parts:
            o.close()


def test_a_step_of_fewer_rows_runs_on_the_fewest_program_each_row_as_on_the_largest(ctx):
    """Generator::step (crates/graph/src/generator.rs:115-123, 286-318): a patch step has a
    program for each power of two below its rows and for its rows; a step of n rows runs on the
    fewest that holds them, the rest spare, and each row comes out bit for bit as on the largest
    beside the others, in whichever row it runs."""
    import tgx
    from tgx.patch import PatchStep
    from tgx.synth import encoder_weights, sampler_weights

    rows = 5  # programs of 1, 2, 4 and 5 rows
    espec, dspec = _encoder_spec(1), _dit_spec(1)
    enc = _encoder(ctx, rows, espec, encoder_weights(espec, FEAT))
    smp = _sampler(ctx, rows, dspec, sampler_weights(dspec, FEAT))
    _, _, w = _lm_weights()
    side = _lm_side(ctx, rows, w)
    step = PatchStep(enc, side, smp)
    _, cond, noise, sampling = _inputs(rows, seed=16)
    # Every run at position 0, which each run rewrites with the same keys and values.
    full_patch, full_stop = step.run_rows([tgx.Row(0, r) for r in range(rows)], cond, noise, sampling)
    for pick in ([3], [1, 4], [0, 2, 4], [4, 3, 2, 1, 0]):
        patch, stop = step.run_rows([tgx.Row(0, r) for r in pick], cond[pick], noise[pick], sampling[pick])
        for k, r in enumerate(pick):
            dp = float(np.abs(patch[k].astype(np.float64) - full_patch[r]).max())
            ds = float(np.abs(stop[k].astype(np.float64) - full_stop[r]).max())
            assert np.array_equal(patch[k], full_patch[r]) and np.array_equal(stop[k], full_stop[r]), (
                f"rows {pick}, row {r}: patch max|d| {dp:.3g}, stop max|d| {ds:.3g}")
    # The components' own entry points take the whole batch again.
    embedding = enc.encode(cond)
    mu, stop = side.step_rows([tgx.Row(0, r) for r in range(rows)], embedding)
    assert np.array_equal(stop, full_stop)
    assert np.array_equal(smp.sample(mu, cond, noise, sampling), full_patch)
    step.close()
    for o in (enc, smp, side):
        o.close()


def test_fresh_patch_steps_beside_used_ones_give_a_warm_steps_bits_on_their_first_run(ctx):
    """The case that once exposed reads of LDS slots before their loads landed (the local ring's
    waits counting loads in an order the compiler had changed): a patch step made fresh, its
    encoder, LM side and sampler new beside ones just used and closed, so that its first run meets
    cold caches. Five fresh sets in turn, 5 rows each: every first run's patches and stop logits,
    of all 5 rows and of 3 rows alone, bit for bit as a warm step's (the batch-invariance contract,
    crates/graph/src/decode.rs:8-11, on cold caches); the test stops at the first that differs."""
    import tgx
    from tgx.patch import PatchStep
    from tgx.synth import encoder_weights, sampler_weights

    rows = 5
    espec, dspec = _encoder_spec(1), _dit_spec(1)
    ew, dw = encoder_weights(espec, FEAT), sampler_weights(dspec, FEAT)
    _, _, w = _lm_weights()
    _, cond, noise, sampling = _inputs(rows, seed=16)
    at = [tgx.Row(0, r) for r in range(rows)]

    def make():
        enc, smp, side = _encoder(ctx, rows, espec, ew), _sampler(ctx, rows, dspec, dw), _lm_side(ctx, rows, w)
        return (enc, smp, side), PatchStep(enc, side, smp)

    def close(parts, step):
        step.close()
        for o in parts:
            o.close()

    parts, step = make()
    step.run_rows(at, cond, noise, sampling)
    warm = step.run_rows(at, cond, noise, sampling)
    close(parts, step)
    for trial in range(5):
        parts, step = make()
        first = step.run_rows(at, cond, noise, sampling)
        for got, want, what in ((first[0], warm[0], "patches"), (first[1], warm[1], "stop logits")):
            assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"fresh set {trial}: {what} of its first run"
        pick = [1, 3, 4]
        alone = step.run_rows([tgx.Row(0, r) for r in pick], cond[pick], noise[pick], sampling[pick])
        assert np.array_equal(alone[0].view(np.uint32), warm[0][pick].view(np.uint32)), f"fresh set {trial}: rows {pick}"
        close(parts, step)
        print(f"[patch] fresh set {trial}: first run bit for bit as the warm step's", flush=True)
