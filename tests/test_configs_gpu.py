"""The benchmark's five configurations on the GPU at their own shapes, through the C ABI, held to
the oracle (oracle/) as crates/graph/tests/{decode,prefill}.rs hold the reference's model:

  C1  the tiny stack (4 layers, fp32 weights): a 32-position prefill and 16 teacher-forced steps
      against the oracle's float64 and float32 paths over the unrounded fp32 weights (the GPU
      rounds them to bf16 on load)
  C2  the 24-layer bf16 backbone at batch 1: a 256-position prefill, then 500 decode steps, every
      step against the float64 oracle (decode.rs:331-336 reports the same distances)
  C3  32 requests at contexts U[64,1024] in 64-position blocks, 200 steps: every request's every
      output bit for bit as the same request alone (decode.rs:243-250)
  C4  8 runs of 2048 positions prefilled at once, then 32 decode steps at batch 8: run 0's
      outputs and cache against the oracle (prefill.rs:365-377), the other seven bit for bit as
      alone
  C5  the 16-request patch step (24-layer backbone, 8-layer residual LM, 4-layer LocDiT and
      encoder) for 300 steps, rows rotating: two requests' LMs at every step and every stage at
      four steps against the oracle, all 16 requests bit for bit as run alone over the 300 steps

Tolerance (bf16 on the GPU against the fp32 oracle): cosine >= 0.999 and
max|got - ref| / max|ref| <= 1e-2, per position or step.
"""

import os
import time

import numpy as np
import pytest

from conftest import distance, within

pytestmark = pytest.mark.gpu


def log(msg: str) -> None:
    print(f"[configs] {msg}", flush=True)


def _threads() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


@pytest.fixture(scope="module", autouse=True)
def oracle_threads():
    import oracle

    oracle.set_threads(_threads())


@pytest.fixture(scope="module")
def backbone():
    """The 24-layer backbone's bf16 weights, N(0, 0.02) from seed 0, drawn once."""
    from tgx.synth import StackSpec, stack_weights

    spec = StackSpec(layers=24, dtype="bf16", seed=0)
    t0 = time.time()
    w = stack_weights(spec)
    log(f"24-layer bf16 weights drawn in {time.time() - t0:.1f} s")
    return spec, w


def _shape(spec, capacity, rope=True):
    import tgx

    return tgx.Shape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads,
                     head_dim=spec.head_dim, layers=spec.layers, capacity=capacity, eps=spec.eps,
                     rope_theta=spec.rope_theta, rope=rope)


def _decoder(ctx, spec, w, capacity, rows=1, slots=None):
    import tgx
    from tgx.synth import bf16_bits

    dec = tgx.Decoder(ctx, _shape(spec, capacity), tgx.Batch(rows=rows, slots=slots or rows))
    for name, v in w.items():
        dec.load(name, bf16_bits(v) if spec.dtype == "bf16" else v)
    return dec


class Worst:
    """The worst distance seen (lowest cosine, highest max relative error) and where."""

    def __init__(self):
        self.cos, self.rel = None, None

    def add(self, d: dict, where) -> None:
        if self.cos is None or d["cosine"] < self.cos[0]["cosine"]:
            self.cos = (d, where)
        if self.rel is None or d["rel_max"] > self.rel[0]["rel_max"]:
            self.rel = (d, where)

    def __str__(self):
        return f"lowest cosine {self.cos}; largest rel_max {self.rel}"


def _same_bits(a, b) -> bool:
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32), np.ascontiguousarray(b, np.float32).view(np.uint32))


def test_c1_tiny_stack_with_fp32_weights_against_the_float64_and_float32_models(ctx):
    """C1: 4 layers, fp32 weights N(0, 0.02), a 32-position prefill of N(0, 1) embeddings, then 16
    teacher-forced steps. The GPU holds the weights in bf16: its distance to the models over the
    unrounded weights includes that rounding (alone rel_max ~5e-3 at this shape)."""
    import oracle
    from tgx.synth import StackSpec, embeddings, stack_weights

    spec = StackSpec(layers=4, dtype="f32", seed=0)
    w = stack_weights(spec)
    cap = 64
    dec = _decoder(ctx, spec, w, cap)
    refs = {p: oracle.Stack(spec, w, cap, p) for p in ("f64", "f32")}
    x = embeddings(spec.seed + 1, "x", 48, spec.hidden)
    got = np.concatenate([dec.prefill(0, x[:32]), np.stack([dec.step(t, x[t]) for t in range(32, 48)])])
    dec.close()
    for p, ref in refs.items():
        want = np.concatenate([ref.prefill(0, x[:32]), np.stack([ref.decode(t, x[t]) for t in range(32, 48)])])
        worst = Worst()
        for t in range(48):
            d = distance(got[t], want[t])
            worst.add(d, t)
            assert within(d), f"{p} position {t}: {d}"
        log(f"C1 against the {p} model over fp32 weights: {worst}")


def test_c2_backbone_256_prefill_then_500_steps_against_the_float64_oracle(ctx, backbone):
    """C2: the 24-layer backbone at batch 1, a 256-position prefill then 500 decode steps, each
    step's hidden state against the float64 oracle (over the same bf16 weights)."""
    import oracle
    from tgx.synth import embeddings

    spec, w = backbone
    prompt, steps = 256, 500
    cap = 768
    dec = _decoder(ctx, spec, w, cap)
    ref = oracle.Stack(spec, w, cap, "f64")
    x = embeddings(2, "c2.x", prompt + steps, spec.hidden)
    t0 = time.time()
    got = dec.prefill(0, x[:prompt])
    want = ref.prefill_rows(0, x[:prompt])
    worst = Worst()
    for t in range(prompt):
        d = distance(got[t], want[t])
        worst.add(d, t)
        assert within(d), f"prefill position {t}: {d}"
    log(f"C2 prefill of {prompt}: {worst} ({time.time() - t0:.1f} s)")
    worst = Worst()
    for t in range(prompt, prompt + steps):
        d = distance(dec.step(t, x[t]), ref.decode(t, x[t]))
        worst.add(d, t)
        assert within(d), f"step at {t}: {d}"
        if (t - prompt) % 100 == 99:
            log(f"C2 {t - prompt + 1} steps, {time.time() - t0:.1f} s: {worst}")
    log(f"C2 {steps} steps from {prompt}: {worst}")
    dec.close()


def test_c3_32_ragged_requests_each_bit_for_bit_as_alone(ctx, backbone):
    """C3: 32 requests at contexts drawn U[64, 1024] (seeded), prefilled at once into their slots'
    64-position blocks, then 200 steps with the requests in rows that change from step to step
    (decode.rs:142-210): every request's prefill outputs and every step's output bit for bit as the
    same request alone in a batch of one; request 0's first steps against the oracle too."""
    import oracle
    import tgx
    from tgx.synth import embeddings

    spec, w = backbone
    n, steps = 32, 200
    contexts = [int(c) for c in np.random.default_rng(3).integers(64, 1025, n)]
    cap = 1280
    prompts = [embeddings(300 + r, "c3.prompt", c, spec.hidden) for r, c in enumerate(contexts)]
    xs = [embeddings(300 + r, "c3.x", steps, spec.hidden) for r in range(n)]
    t0 = time.time()
    batch = _decoder(ctx, spec, w, cap, rows=n)
    pre = batch.prefill_runs([(r, 0, c) for r, c in enumerate(contexts)], np.concatenate(prompts))
    outs = np.empty((steps, n, spec.hidden), dtype=np.float32)
    for t in range(steps):
        order = np.roll(np.arange(n), 5 * t)  # row i runs request order[i]
        placed = [tgx.Row(contexts[r] + t, r) for r in order]
        out = batch.step_rows(placed, np.stack([xs[r][t] for r in order]))
        outs[t, order] = out
    batch.close()
    log(f"C3 batch of {n}: contexts {min(contexts)}..{max(contexts)}, {steps} steps in {time.time() - t0:.1f} s")
    ref = oracle.Stack(spec, w, cap, "f64")
    ref.prefill_rows(0, prompts[0])
    for t in range(4):
        d = distance(outs[t, 0], ref.decode(contexts[0] + t, xs[0][t]))
        assert within(d), f"request 0 step {t}: {d}"
    alone = _decoder(ctx, spec, w, cap)
    row = 0
    for r, c in enumerate(contexts):
        alone.release_slot(0)
        a = alone.prefill(0, prompts[r])
        assert _same_bits(a, pre[row : row + c]), f"request {r} ({c} positions): prefill"
        row += c
        for t in range(steps):
            assert _same_bits(alone.step(c + t, xs[r][t]), outs[t, r]), f"request {r} ({c} positions), step {t}"
    alone.close()
    log(f"C3 every request bit for bit as alone, {time.time() - t0:.1f} s in all")


def test_c4_8x2048_prefill_then_32_steps(ctx, backbone):
    """C4: 8 runs of 2048 positions prefilled at once, then 32 decode steps at batch 8. Run 0's
    2048 outputs and its keys and values at every layer against the float64 oracle, its 32 steps
    too; runs 1..7 bit for bit as each alone (prefill and steps)."""
    import oracle
    import tgx
    from tgx.synth import embeddings

    spec, w = backbone
    L, runs, steps = 2048, 8, 32
    cap = 2304
    x = embeddings(40, "c4.x", runs * L, spec.hidden)
    xs = embeddings(41, "c4.steps", steps * runs, spec.hidden).reshape(steps, runs, spec.hidden)
    t0 = time.time()
    dec = _decoder(ctx, spec, w, cap, rows=runs)
    out = dec.prefill_runs([(r, 0, L) for r in range(runs)], x)
    k, v = dec.read_cache(0, L)
    after = [dec.step_rows([tgx.Row(L + t, r) for r in range(runs)], xs[t]) for t in range(steps)]
    dec.close()
    log(f"C4 on the GPU in {time.time() - t0:.1f} s")
    ref = oracle.Stack(spec, w, cap, "f64")
    want = ref.prefill_rows(0, x[:L])
    log(f"C4 oracle prefill of {L} positions, {time.time() - t0:.1f} s")
    worst = Worst()
    for t in range(L):
        d = distance(out[t], want[t])
        worst.add(d, t)
        assert within(d), f"run 0 position {t}: {d}"
    log(f"C4 run 0 prefill outputs: {worst}")
    for name, got_c, want_c in (("keys", k, ref.k), ("values", v, ref.v)):
        for l in range(spec.layers):
            d = distance(got_c[l], want_c[l, :, :L])
            assert within(d), f"{name} of layer {l}: {d}"
    worst = Worst()
    for t in range(steps):
        d = distance(after[t][0], ref.decode(L + t, xs[t][0]))
        worst.add(d, t)
        assert within(d), f"run 0 step {t}: {d}"
    log(f"C4 run 0 steps from {L}: {worst}")
    alone = _decoder(ctx, spec, w, cap)
    for r in range(1, runs):
        alone.release_slot(0)
        assert _same_bits(alone.prefill(0, x[r * L : (r + 1) * L]), out[r * L : (r + 1) * L]), f"run {r} prefill"
        for t in range(steps):
            assert _same_bits(alone.step(L + t, xs[t][r]), after[t][r]), f"run {r} step {t}"
    alone.close()
    log(f"C4 runs 1..7 bit for bit as alone, {time.time() - t0:.1f} s in all")


def test_c5_16_request_patch_step_300_steps_stage_by_stage_and_each_request_as_alone(ctx, backbone):
    """C5: the full per-patch step at 16 requests for 300 steps, each LM's cache first filled to 64
    prompt positions: the 4-layer encoder over the patch before, the 24-layer backbone and the
    8-layer residual LM with the heads between them, the 4-layer LocDiT's 10 Euler steps with
    CFG-Zero* (guidance 2.0 over both sequences). Requests move to another row every step (request
    i in row (i + t) mod 16), as crates/graph/tests/patch.rs:175-211 rotates them.

    Checked: for two requests, the backbone's and the residual LM's outputs at all 300 steps
    against the oracle (its layer-major restatement over the GPU's inputs to each LM, the
    positions after the prompt at once) and, at steps 0, 1, 2 and 299, every stage (encoder, heads,
    quantizer levels but those at a tie, sampler, stop logits within the dot product's bound), each
    stage fed the GPU's input to it; then every one of the 16 requests run alone on the patch
    step's one-row program over its whole 300 steps (patch.rs:257-278), each patch and stop logit
    bit for bit as among the 16 (patch.rs:286-317)."""
    import oracle
    import patch_oracle as po
    import tgx
    from tgx.patch import Encoder, HeadsShape, LmSide, PatchShape, PatchStep, Sampler
    from tgx.synth import StackSpec, embeddings, encoder_weights, lm_side_weights, sampler_weights

    rows, context, feat, frames, levels, steps = 16, 64, 64, 4, 9, 300
    staged = (0, 1, 2, steps - 1)
    base_spec, res_spec = StackSpec(layers=24, seed=0), StackSpec(layers=8, seed=1)
    dit_spec, enc_spec = StackSpec(layers=4, seed=2), StackSpec(layers=4, seed=3)
    w = lm_side_weights(base_spec, res_spec, 1024, 1024, 256)
    dw, ew = sampler_weights(dit_spec, feat), encoder_weights(enc_spec, feat)
    cap = 384
    t0 = time.time()
    side = LmSide(ctx, tgx.Shape(layers=24, capacity=cap), tgx.Shape(layers=8, capacity=cap, rope=False),
                  tgx.Batch(rows=rows, slots=rows), HeadsShape(1024, 1024, 256, levels))
    side.load_all(w)
    sampler = Sampler(ctx, tgx.Shape(layers=4, capacity=16), PatchShape(feat, frames, 10, rows))
    sampler.load_all(dw)
    encoder = Encoder(ctx, tgx.Shape(layers=4, capacity=16), PatchShape(feat, frames, 10, rows))
    encoder.load_all(ew)
    prompts = [embeddings(50 + which, "c5.prompt", rows * context, 1024) for which in (0, 1)]
    for which in (0, 1):
        side.decoder(which).prefill_runs([(r, 0, context) for r in range(rows)], prompts[which])
    step = PatchStep(encoder, side, sampler)
    rng = np.random.default_rng(55)
    sampling = np.array([[1.0, 2.0]] * rows, dtype=np.float32)
    sampling[3] = [0.8, 1.5]
    sampling[12] = [1.3, 3.0]
    picks = (0, 9)
    stack = lambda s: po.StackShape(hidden=s.hidden, inner=s.inner, heads=s.heads, kv_heads=s.kv_heads, layers=s.layers,
                                    eps=s.eps, rope_theta=s.rope_theta)
    cond = rng.standard_normal((rows, feat, frames)).astype(np.float32)
    conds, noises, patches, stops = [], [], [], []
    lm_in = {r: {"embed": [], "base_out": [], "residual_in": [], "residual_out": []} for r in picks}
    for k in range(steps):
        noise = rng.standard_normal((rows, feat, frames)).astype(np.float32)
        order = [(j - k) % rows for j in range(rows)]  # the request in row j
        at = [tgx.Row(context + k, i) for i in order]
        patch_rows, stop_rows = step.run_rows(at, cond[order], noise[order], sampling[order])
        patch, stop = np.empty_like(patch_rows), np.empty_like(stop_rows)
        patch[order], stop[order] = patch_rows, stop_rows
        conds.append(cond.copy())
        noises.append(noise)
        patches.append(patch)
        stops.append(stop)
        t = {n: side.read(n) for n in side.TENSORS}
        row_of = {i: j for j, i in enumerate(order)}
        for r in picks:
            for name in lm_in[r]:
                lm_in[r][name].append(t[name][row_of[r]].copy())
        if k in staged:
            embedding = encoder.encode(cond[order])
            for r in picks:
                j = row_of[r]
                checks = {"encoder": (embedding[j], po.encode(ew, stack(enc_spec), feat, frames, cond[r : r + 1])[0]),
                          "embed": (t["embed"][j], po.linear(w, "enc_to_lm_proj", embedding[j : j + 1])[0])}
                pre, lv = po.quantizer(w, t["base_out"][j : j + 1], levels)
                tie = t["levels"][j] != lv[0].astype(np.float32)
                if tie.any():
                    frac = np.abs(np.tanh(np.abs(pre[0][tie])) * levels % 1.0 - 0.5)
                    assert np.all(frac < 0.05) and tie.mean() < 0.05, (k, r, frac)
                lm_hidden, residual_in, to_dit, stop_hidden, logits = po.heads_after_levels(w, t["levels"][j : j + 1],
                                                                                             t["embed"][j : j + 1])
                checks["lm_hidden"] = (t["lm_hidden"][j], lm_hidden[0])
                checks["residual_in"] = (t["residual_in"][j], residual_in[0])
                checks["mu"] = (t["mu"][j], np.concatenate([to_dit[0], po.linear(w, "res_to_dit_proj", t["residual_out"][j : j + 1])[0]]))
                bound = 2.0**-8 * (np.abs(w["stop_head.weight"]).astype(np.float64) @ np.abs(t["stop_hidden"][j]))
                assert np.all(np.abs(stop[r] - logits[0]) <= bound + 1e-7), (k, r, stop[r], logits[0])
                x0, want = po.sample(dw, stack(dit_spec), feat, frames, 10, t["mu"][j].reshape(1, 2, 1024), cond[r : r + 1],
                                     noise[r : r + 1], sampling[r : r + 1])
                checks["patch moved"] = (patch[r] - x0[0], want[0] - x0[0])
                checks["patch"] = (patch[r], want[0])
                for name, (g, e) in checks.items():
                    d = distance(g, e)
                    assert within(d), f"step {k} request {r} {name}: {d}"
                log(f"C5 step {k} request {r} (row {j}): every stage within tolerance, {int(tie.sum())} levels at a tie")
        cond = patch.astype(np.float32)  # the next step samples after this one's patch
        if k % 50 == 49:
            log(f"C5 {k + 1} 16-request steps, {time.time() - t0:.1f} s")
    # The two LMs over all 300 steps for the picked requests: the oracle's caches hold the prompt,
    # then every step's input the GPU gave each LM, the positions after the prompt at once.
    for r in picks:
        base_ref = oracle.Stack(base_spec, {k[8:]: v for k, v in w.items() if k.startswith("base_lm.")}, cap, "f64")
        res_ref = oracle.Stack(res_spec, {k[12:]: v for k, v in w.items() if k.startswith("residual_lm.")}, cap, "f64",
                               rope=False)
        base_ref.prefill_rows(0, prompts[0][r * context : (r + 1) * context])
        res_ref.prefill_rows(0, prompts[1][r * context : (r + 1) * context])
        for name, ref, inp in (("base_out", base_ref, "embed"), ("residual_out", res_ref, "residual_in")):
            want = ref.prefill_rows(context, np.stack(lm_in[r][inp]))
            worst = None
            for k in range(steps):
                d = distance(lm_in[r][name][k], want[k])
                assert within(d), f"request {r} {name} step {k}: {d}"
                worst = d if worst is None or d["cosine"] < worst["cosine"] else worst
            log(f"C5 request {r} {name} at all {steps} steps within tolerance, worst {worst}")
    # Every request alone on the one-row program, its whole run from the prompt on (its slot's
    # cache past the prompt rewritten step by step as it goes).
    for r in range(rows):
        for k in range(steps):
            p1, s1 = step.run_rows([tgx.Row(context + k, r)], conds[k][r : r + 1], noises[k][r : r + 1], sampling[r : r + 1])
            assert _same_bits(p1[0], patches[k][r]) and _same_bits(s1[0], stops[k][r]), f"request {r} step {k} alone"
        if r % 4 == 3:
            log(f"C5 requests 0..{r} alone bit for bit as among 16 over {steps} steps, {time.time() - t0:.1f} s")
    step.close()
    for o in (side, sampler, encoder):
        o.close()
    log(f"C5 all 16 requests alone bit for bit as among 16, {time.time() - t0:.1f} s in all")
