"""The decode step on the GPU through the C ABI against the oracle, as the reference's
crates/graph/tests/decode.rs holds its decode step to goldens: per-step accuracy, each row of a
batch bit for bit as it is alone, a defect that must fail, the KV cache itself, spare rows and
the paged cache's refusals.

Tolerance (bf16 weights and activations on the GPU, the fp64 oracle over the same bf16 weights):
cosine >= 0.999 and max|got - ref| / max|ref| <= 1e-2 at every step.
"""

import numpy as np
import pytest

from conftest import COSINE_MIN, REL_MAX, distance, within

pytestmark = pytest.mark.gpu


def tiny_spec(layers=4, dtype="f32", seed=0):
    from tgx.synth import StackSpec

    return StackSpec(layers=layers, dtype=dtype, seed=seed)


def make_decoder(ctx, spec, capacity, rows=1, slots=None, rope=True, blocks=0):
    import tgx
    from tgx.synth import stack_weights

    shape = tgx.Shape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads,
                      head_dim=spec.head_dim, layers=spec.layers, capacity=capacity, eps=spec.eps,
                      rope_theta=spec.rope_theta, rope=rope)
    dec = tgx.Decoder(ctx, shape, tgx.Batch(rows=rows, slots=slots or rows, blocks=blocks))
    dec.load_all(stack_weights(spec))
    return dec


def oracle_stack(spec, capacity, rope=True, shift=0):
    import oracle
    from tgx.synth import bf16_round, stack_weights

    # The GPU holds bf16 weights: the oracle runs over the same values.
    w = {k: bf16_round(v) for k, v in stack_weights(spec).items()}
    return oracle.Stack(spec, w, capacity, "f64", rope=rope, shift=shift)


def inputs(spec, n, name="x"):
    from tgx.synth import embeddings

    return embeddings(spec.seed + 1, name, n, spec.hidden)


def test_tiny_decoder_32_prefill_positions_and_16_steps_match_the_oracle(ctx):
    """The tiny MiniCPM-4-shaped decoder (4 layers, fp32 weights drawn from a seed) through decode
    steps: 32 positions then 16 teacher-forced steps, the CPU-runnable case."""
    spec = tiny_spec()
    cap = 64
    dec = make_decoder(ctx, spec, cap)
    ref = oracle_stack(spec, cap)
    x = inputs(spec, 48)
    worst = None
    for t in range(48):
        got = dec.step(t, x[t])
        want = ref.decode(t, x[t])
        d = distance(got, want)
        assert within(d), f"step {t}: {d}"
        if worst is None or d["cosine"] < worst["cosine"]:
            worst = d
    print(f"tiny decoder, worst step: {worst}")
    # The cache holds the oracle's keys and values (rounded to bf16).
    k, v = dec.read_cache(0, 48)
    for name, got, want in (("k", k, ref.k[:, :, :48]), ("v", v, ref.v[:, :, :48])):
        d = distance(got, want)
        assert d["cosine"] >= COSINE_MIN and d["rel_max"] <= REL_MAX, f"{name} cache: {d}"


def test_positions_one_slot_on_fail_the_tolerance(ctx):
    """Defect (crates/graph/tests/decode.rs:252-255): every position one slot on in the cache, so
    that each query also attends to the empty position 0."""
    spec = tiny_spec(layers=1)
    cap = 64
    dec = make_decoder(ctx, spec, cap)
    ref = oracle_stack(spec, cap)
    x = inputs(spec, 40)
    failed = 0
    for t in range(40):
        d = distance(dec.step(t + 1, x[t]), ref.decode(t, x[t]))
        failed += not within(d)
    assert failed > 0, "positions one slot on pass"


def test_a_stack_without_rope_matches_and_rotating_it_fails(ctx):
    """The residual LM attends without RoPE (decode.rs:47-50); rotating it is a defect
    (crates/graph/tests/decode.rs:372-378)."""
    spec = tiny_spec(layers=2)
    cap = 64
    dec = make_decoder(ctx, spec, cap, rope=False)
    ref = oracle_stack(spec, cap, rope=False)
    rotated = oracle_stack(spec, cap, rope=True)
    x = inputs(spec, 40)
    failed = 0
    for t in range(40):
        got = dec.step(t, x[t])
        d = distance(got, ref.decode(t, x[t]))
        assert within(d), f"step {t}: {d}"
        failed += not within(distance(got, rotated.decode(t, x[t])))
    assert failed > 0


def run_rows(ctx, spec, x, rows, cap, shift=0):
    """crates/graph/tests/decode.rs:142-210: `rows` requests at once, request r from step 2r on
    in slot rows - 1 - r, in a row that changes from step to step, the rows without one spare."""
    import tgx

    dec = make_decoder(ctx, spec, cap, rows=rows)
    n = x.shape[0]
    got = [[] for _ in range(rows)]
    for t in range(n + 2 * (rows - 1)):
        placed = [None] * rows
        inp = np.zeros((rows, spec.hidden), dtype=np.float32)
        for r in range(rows):
            i = t - 2 * r
            if not (0 <= i < n):
                continue
            row = (r + t) % rows
            placed[row] = tgx.Row(i + shift, rows - 1 - r)
            inp[row] = x[i]
        out = dec.step_rows(placed, inp)
        for r in range(rows):
            if 2 * r <= t < 2 * r + n:
                got[r].append(out[(r + t) % rows].copy())
    dec.close()
    return [np.stack(g) for g in got]


@pytest.mark.parametrize("rows", [3, 16, 20, 40])  # one tile, a full one, two tiles, three (ragged)
def test_each_row_of_a_batch_is_bit_for_bit_as_it_is_alone(ctx, rows):
    spec = tiny_spec(layers=2)
    cap = 320
    x = inputs(spec, 300)
    alone = run_rows(ctx, spec, x, 1, cap)[0]
    batched = run_rows(ctx, spec, x, rows, cap)
    for r, got in enumerate(batched):
        differ = int(np.sum(got.view(np.uint32) != alone.view(np.uint32)))
        assert differ == 0, f"row {r} of {rows}: {differ} values differ from alone"


def test_batch_of_64_rows_is_as_alone(ctx):
    """The largest batch the kernels take: four column tiles of 16."""
    import tgx

    spec = tiny_spec(layers=1)
    cap = 128
    x = inputs(spec, 100)
    alone = run_rows(ctx, spec, x[:70], 1, cap)[0]
    dec = make_decoder(ctx, spec, cap, rows=64)
    outs = []
    for t in range(70):
        rows = [tgx.Row(t, s) for s in range(64)]
        inp = np.repeat(x[t : t + 1], 64, axis=0)
        out = dec.step_rows(rows, inp)
        outs.append(out)
    outs = np.stack(outs)  # [t][row][hidden]
    for r in (0, 17, 63):
        assert np.array_equal(outs[:, r].view(np.uint32), alone.view(np.uint32)), f"row {r}"


def test_long_contexts_match_the_oracle_and_each_row_is_as_alone(ctx):
    """Past 256 positions each of the attention's waves takes more than one 32-position turn (two
    at a time): a row at 1100 positions (35 turns, five for some waves) matches the oracle step by
    step, and each row of a batch of long and short contexts is bit for bit as it is alone."""
    import tgx

    spec = tiny_spec(layers=1)
    cap = 1280
    n = 1100
    x = inputs(spec, n + 6)
    ref = oracle_stack(spec, cap)
    ref.prefill(0, x[:n])
    dec = make_decoder(ctx, spec, cap)
    dec.prefill_runs([(0, 0, n)], x[:n])
    for t in range(n, n + 6):
        d = distance(dec.step(t, x[t]), ref.decode(t, x[t]))
        assert within(d), f"step {t}: {d}"
    dec.close()
    lens = [1100, 70, 600, 513]  # 18 blocks, 2, 10, 9
    xs = [inputs(spec, L + 4, name=f"row{r}") for r, L in enumerate(lens)]
    batch = make_decoder(ctx, spec, cap, rows=len(lens))
    batch.prefill_runs([(r, 0, L) for r, L in enumerate(lens)], np.concatenate([xr[:L] for xr, L in zip(xs, lens)]))
    together = [batch.step_rows([tgx.Row(L + k, r) for r, L in enumerate(lens)], np.stack([xr[L + k] for xr, L in zip(xs, lens)]))
                for k in range(4)]
    batch.close()
    for r, L in enumerate(lens):
        alone = make_decoder(ctx, spec, cap)
        alone.prefill_runs([(0, 0, L)], xs[r][:L])
        for k in range(4):
            got = alone.step(L + k, xs[r][L + k])
            assert np.array_equal(got.view(np.uint32), together[k][r].view(np.uint32)), f"row {r} ({L} positions), step {k}"
        alone.close()


def test_a_row_past_16384_positions_steps_as_the_prefill_computes_and_as_alone(ctx):
    """Past 16384 positions a wave of the attention has more than 64 turns, their cache blocks in a
    second register: a row at 20000 positions steps as a prefill of one more position computes its
    last output (the prefill's own kernels, checked against the oracle elsewhere; the oracle would
    take minutes over 20000 positions), and beside a short row bit for bit as alone."""
    import tgx

    spec = tiny_spec(layers=1, dtype="bf16")
    cap, n = 20480, 20000
    x = inputs(spec, n + 2)
    print(f"[decode] a row at {n} positions of {cap}", flush=True)
    whole = make_decoder(ctx, spec, cap)
    want = whole.prefill_runs([(0, 0, n + 1)], x[: n + 1])[n]
    whole.close()
    dec = make_decoder(ctx, spec, cap)
    dec.prefill_runs([(0, 0, n)], x[:n])
    got = dec.step(n, x[n])
    d = distance(got, want)
    assert within(d), f"step at {n}: {d}"
    two = make_decoder(ctx, spec, cap, rows=2)
    two.prefill_runs([(0, 0, n), (1, 0, 40)], np.concatenate([x[:n], x[:40]]))
    both = two.step_rows([tgx.Row(n, 0), tgx.Row(40, 1)], np.stack([x[n], x[40]]))
    assert np.array_equal(both[0].view(np.uint32), got.view(np.uint32))
    two.close()
    dec.close()


def test_launched_steps_move_the_rows_on_as_single_steps_do(ctx):
    """The recorded step replayed (Decoder::launch with advance, each placed row moved on a
    position by the step itself; the benchmark's path): k launched steps and one more leave the
    output and the caches that k + 1 single steps leave, bit for bit."""
    import tgx

    spec = tiny_spec(layers=2)
    cap = 128
    x = inputs(spec, 2)
    prompt = inputs(spec, 14, name="prompt")
    decs = []
    for _ in range(2):
        d = make_decoder(ctx, spec, cap, rows=2)
        d.prefill_runs([(0, 0, 5), (1, 0, 9)], prompt)
        for slot in range(2):
            d.reserve(slot, 40)
        decs.append(d)
    a, b = decs
    k = 6
    a.set_rows([tgx.Row(5, 0), tgx.Row(9, 1)], x)
    a.launch(k, advance=True)
    a.wait()
    a.start()
    a.wait()
    got = a.output()
    for t in range(k + 1):
        want = b.step_rows([tgx.Row(5 + t, 0), tgx.Row(9 + t, 1)], x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for slot, n in ((0, 5 + k + 1), (1, 9 + k + 1)):
        ka, va = a.read_cache(slot, n)
        kb, vb = b.read_cache(slot, n)
        assert np.array_equal(ka, kb) and np.array_equal(va, vb), f"slot {slot}"
    for d in decs:
        d.close()


def test_spare_rows_write_no_cache_and_leave_others_alone(ctx):
    import tgx

    spec = tiny_spec(layers=1)
    cap = 128
    x = inputs(spec, 10)
    dec = make_decoder(ctx, spec, cap, rows=2, slots=2)
    alone = make_decoder(ctx, spec, cap, rows=1)
    for t in range(10):
        out = dec.step_rows([None, tgx.Row(t, 1)], np.stack([x[(t + 3) % 10], x[t]]))
        a = alone.step(t, x[t])
        assert np.array_equal(out[1].view(np.uint32), a.view(np.uint32))
    # Slot 0 was never placed: it holds no blocks at all.
    assert dec.free_blocks() == 2 * 2 - 1


def test_placements_the_batch_cannot_hold_are_refused(ctx):
    import tgx

    spec = tiny_spec(layers=1)
    dec = make_decoder(ctx, spec, 64, rows=3, slots=4)
    x = np.zeros((3, spec.hidden), dtype=np.float32)
    for rows in ([tgx.Row(5, 2), tgx.Row(9, 2), None], [tgx.Row(64, 0), None, None], [tgx.Row(1, 4), None, None]):
        with pytest.raises(tgx.TgxError) as e:
            dec.step_rows(rows, x)
        assert e.value.kind == "shape"
    with pytest.raises(tgx.TgxError):
        dec.step_rows([None, None], x[:2])


def test_a_pool_too_small_for_the_slots_is_refused_when_it_runs_out(ctx):
    import tgx

    spec = tiny_spec(layers=1)
    dec = make_decoder(ctx, spec, 256, rows=2, slots=2, blocks=3)
    x = np.zeros((2, spec.hidden), dtype=np.float32)
    dec.step_rows([tgx.Row(127, 0), None], x)  # two blocks
    dec.step_rows([None, tgx.Row(10, 1)], x)  # a third
    with pytest.raises(tgx.TgxError) as e:
        dec.step_rows([tgx.Row(128, 0), None], x)  # a fourth: none left
    assert e.value.kind == "shape"
    dec.release_slot(1)
    dec.step_rows([tgx.Row(128, 0), None], x)


def test_nan_left_in_a_reused_block_past_the_position_never_reaches_the_output(ctx):
    """crates/vulkan/tests/glsl.rs:690-699: what lies past the position must not reach the output,
    NaN included. A request fed NaN leaves NaN keys and values at positions 0..99 of its slot's
    blocks; the slot is released and the next request, handed the same blocks, runs positions
    0..69 (every step's block holds NaN past its position): each step finite and bit for bit as
    on a fresh decoder."""
    spec = tiny_spec(layers=2)
    cap = 128
    x = inputs(spec, 70)
    dec = make_decoder(ctx, spec, cap)
    fresh = make_decoder(ctx, spec, cap)
    poison = np.full(spec.hidden, np.nan, dtype=np.float32)
    for t in range(100):
        dec.step(t, poison)
    k, v = dec.read_cache(0, 100)
    assert np.isnan(k).all() and np.isnan(v).all()
    dec.release_slot(0)
    for t in range(70):
        got, want = dec.step(t, x[t]), fresh.step(t, x[t])
        assert np.all(np.isfinite(got)), f"step {t}"
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"step {t}"
    k, v = dec.read_cache(0, 128)
    assert np.isfinite(k[:, :, :70]).all() and np.isnan(k[:, :, 70:100]).all()
    dec.close()
    fresh.close()


def test_a_step_writes_its_own_position_and_no_other(ctx):
    """glsl.rs:590-597: a cache row past the position is never written. Positions 0..63 hold
    known values (a prefill of 64); a step at 20 then rewrites row 20 alone, in every layer."""
    spec = tiny_spec(layers=2)
    cap = 128
    x = inputs(spec, 65)
    dec = make_decoder(ctx, spec, cap)
    dec.prefill_runs([(0, 0, 64)], x[:64])
    k0, v0 = dec.read_cache(0, 64)
    dec.step(20, x[64])
    k1, v1 = dec.read_cache(0, 64)
    for before, after in ((k0, k1), (v0, v1)):
        changed = np.any(before != after, axis=(0, 1, 3))
        assert changed[20] and changed.sum() == 1, np.flatnonzero(changed)
    dec.close()


def test_launched_steps_past_the_reserved_blocks_hold_them_and_match_single_steps(ctx):
    """Decoder::launch with advance past what reserve held: the launch holds the blocks each row's
    positions reach (positions 60..139 of a slot reserved to 64), so that the launched steps leave
    the output and the caches single steps leave, bit for bit; a launch that would take a row past
    the capacity is refused on the host, before anything runs."""
    import tgx

    spec = tiny_spec(layers=2)
    cap = 192
    x = inputs(spec, 1)
    prompt = inputs(spec, 60, name="prompt")
    a = make_decoder(ctx, spec, cap)
    b = make_decoder(ctx, spec, cap)
    for d in (a, b):
        d.prefill_runs([(0, 0, 60)], prompt)
    k = 80
    a.set_rows([tgx.Row(60, 0)], x)
    a.launch(k, advance=True)
    a.wait()
    a.start()  # at 60 + k: the host follows the rows the device moved on
    a.wait()
    got = a.output()[0]
    for t in range(k + 1):
        want = b.step(60 + t, x[0])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    ka, va = a.read_cache(0, 60 + k + 1)
    kb, vb = b.read_cache(0, 60 + k + 1)
    assert np.array_equal(ka, kb) and np.array_equal(va, vb)
    a.set_rows([tgx.Row(150, 0)], x)
    with pytest.raises(tgx.TgxError) as e:
        a.launch(cap - 150 + 1, advance=True)
    assert e.value.kind == "shape"
    a.launch(cap - 150, advance=True)  # up to the last position: allowed
    a.wait()
    a.close()
    b.close()


def test_rows_set_again_before_a_step_run_as_last_set(ctx):
    """The host's staging for a step's inputs (placement, block tables, x) is refilled only once
    the copies queued from it have run: rows and inputs set, a slot's blocks reserved, and rows set
    again with other inputs and positions before the step run the last ones, bit for bit as a
    decoder that only ever saw them; steps through host arrays one after another, each with new
    inputs, as single steps on a fresh decoder."""
    import tgx

    spec = tiny_spec(layers=2)
    cap = 256
    prompt = inputs(spec, 70, name="prompt")
    x = inputs(spec, 12)
    a = make_decoder(ctx, spec, cap, rows=2, slots=2)
    b = make_decoder(ctx, spec, cap, rows=2, slots=2)
    for d in (a, b):
        d.prefill_runs([(0, 0, 40), (1, 0, 30)], prompt)
    rows = [tgx.Row(40, 0), tgx.Row(30, 1)]
    a.set_rows([tgx.Row(30, 1), tgx.Row(40, 0)], x[2:4])  # replaced before any step
    a.reserve(0, 200)
    a.set_rows(rows, x[0:2])
    a.start()
    a.wait()
    got = a.output()
    want = b.step_rows(rows, x[0:2])
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for t in range(1, 5):
        rows_t = [tgx.Row(40 + t, 0), tgx.Row(30 + t, 1)]
        got = a.step_rows(rows_t, x[2 * t : 2 * t + 2])
        want = b.step_rows(rows_t, x[2 * t : 2 * t + 2])
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"step {t}"
    a.close()
    b.close()
