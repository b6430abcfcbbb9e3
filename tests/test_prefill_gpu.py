"""The prefill on the GPU through the C ABI against the oracle, as crates/graph/tests/prefill.rs
holds the reference's: its outputs and the cache it writes, decode steps going on from that cache
(prefill.rs:255-258), runs not a multiple of any tile, a run continuing another, several runs at
once each bit for bit as alone.

Tolerance as the decode step's: cosine >= 0.999 and max|got - ref| / max|ref| <= 1e-2 against the
fp64 oracle over the same bf16 weights, per position.
"""

import numpy as np
import pytest

from conftest import distance, within
from test_decode_gpu import inputs, make_decoder, oracle_stack, tiny_spec

pytestmark = pytest.mark.gpu


def check_rows(got, want, what):
    worst = None
    for t in range(want.shape[0]):
        d = distance(got[t], want[t])
        assert within(d), f"{what} row {t}: {d}"
        if worst is None or d["cosine"] < worst["cosine"]:
            worst = d
    return worst


def test_tiny_decoder_32_position_prefill_then_16_steps_match_the_oracle(ctx):
    """The tiny MiniCPM-4-shaped decoder (4 layers): a 32-position prefill, then 16 teacher-forced
    decode steps, the CPU-runnable case."""
    spec = tiny_spec()
    cap = 64
    dec = make_decoder(ctx, spec, cap)
    ref = oracle_stack(spec, cap)
    x = inputs(spec, 48)
    got = dec.prefill(0, x[:32])
    want = ref.prefill(0, x[:32])
    worst = check_rows(got, want, "prefill")
    for t in range(32, 48):
        d = distance(dec.step(t, x[t]), ref.decode(t, x[t]))
        assert within(d), f"step {t}: {d}"
    print(f"tiny decoder, prefill worst row: {worst}")
    k, v = dec.read_cache(0, 48)
    assert within(distance(k, ref.k[:, :, :48])) and within(distance(v, ref.v[:, :, :48]))


@pytest.mark.parametrize("lengths", [(77,), (40, 37), (1, 130)])
def test_runs_of_any_length_continue_each_other(ctx, lengths):
    spec = tiny_spec(layers=2)
    cap = 256
    dec = make_decoder(ctx, spec, cap)
    ref = oracle_stack(spec, cap)
    total = sum(lengths)
    x = inputs(spec, total + 4)
    start = 0
    for n in lengths:
        got = dec.prefill(start, x[start : start + n])
        want = ref.prefill(start, x[start : start + n])
        check_rows(got, want, f"run from {start}")
        start += n
    for t in range(total, total + 4):
        assert within(distance(dec.step(t, x[t]), ref.decode(t, x[t])))


@pytest.mark.parametrize("lengths", [(192,), (191, 1), (17, 175)])
def test_runs_that_end_at_the_capacity_match_the_oracle(ctx, lengths):
    """Runs ending at the cache's last position (capacity 192: three 64-position blocks, the last
    run's tiles ending on it), against the oracle, outputs and the whole cache."""
    spec = tiny_spec(layers=2)
    cap = 192
    dec = make_decoder(ctx, spec, cap)
    ref = oracle_stack(spec, cap)
    x = inputs(spec, cap)
    print(f"[prefill] runs {lengths} to the capacity {cap}", flush=True)
    start = 0
    for n in lengths:
        check_rows(dec.prefill(start, x[start : start + n]), ref.prefill(start, x[start : start + n]), f"run from {start}")
        start += n
    k, v = dec.read_cache(0, cap)
    assert within(distance(k, ref.k[:, :, :cap])) and within(distance(v, ref.v[:, :, :cap]))
    dec.close()


def test_several_runs_at_once_are_bit_for_bit_as_alone(ctx):
    spec = tiny_spec(layers=2)
    cap = 512
    lengths = [300, 45, 129]
    x = inputs(spec, sum(lengths))
    dec = make_decoder(ctx, spec, cap, rows=3, slots=3)
    together = dec.prefill_runs([(2, 0, 300), (0, 0, 45), (1, 0, 129)], x)
    row = 0
    for n in lengths:
        alone_dec = make_decoder(ctx, spec, cap)
        alone = alone_dec.prefill(0, x[row : row + n])
        assert np.array_equal(together[row : row + n].view(np.uint32), alone.view(np.uint32)), f"run of {n}"
        alone_dec.close()
        row += n


def test_a_run_in_a_decoder_of_16_row_strips_is_bit_for_bit_as_in_one_of_4_row_strips(ctx):
    """A decoder of more than 16 rows keeps o_proj and down_proj in 16-row strips, one of 16 or
    fewer in 4-row strips: the same runs prefilled in each (together in the 20-row one, alone in
    1-row ones) give the same bits, outputs and the steps after them."""
    import tgx

    spec = tiny_spec(layers=2)
    cap = 512
    lengths = [300, 45, 129]
    x = inputs(spec, sum(lengths) + 1)
    wide = make_decoder(ctx, spec, cap, rows=20, slots=20)
    print(f"[prefill] runs {lengths} in a 20-row decoder against 1-row ones", flush=True)
    together = wide.prefill_runs([(5, 0, 300), (0, 0, 45), (19, 0, 129)], x[: sum(lengths)])
    row = 0
    for slot, n in zip((5, 0, 19), lengths):
        alone_dec = make_decoder(ctx, spec, cap)
        alone = alone_dec.prefill(0, x[row : row + n])
        assert np.array_equal(together[row : row + n].view(np.uint32), alone.view(np.uint32)), f"run of {n}"
        # The step after the run reads the cache the prefill wrote.
        a = alone_dec.step(n, x[-1])
        b = wide.step_rows([tgx.Row(position=n, slot=slot)] + [None] * 19, np.repeat(x[-1:], 20, axis=0))[0]
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step after the run of {n}"
        alone_dec.close()
        row += n
    wide.close()


def test_a_long_run_in_slots_past_the_first(ctx):
    """Two runs of 600 positions in slots 1 and 2 of a 2-layer stack, against the oracle."""
    spec = tiny_spec(layers=2)
    cap = 640
    dec = make_decoder(ctx, spec, cap, rows=2, slots=3)
    x = inputs(spec, 1200)
    got = dec.prefill_runs([(1, 0, 600), (2, 0, 600)], x)
    for r in range(2):
        ref = oracle_stack(spec, cap)
        want = ref.prefill(0, x[600 * r : 600 * (r + 1)])
        check_rows(got[600 * r : 600 * (r + 1)], want, f"run {r}")


def test_runs_the_cache_cannot_hold_are_refused(ctx):
    import tgx

    spec = tiny_spec(layers=1)
    dec = make_decoder(ctx, spec, 64, rows=1, slots=2)
    x = np.zeros((65, spec.hidden), dtype=np.float32)
    for runs in ([(0, 0, 65)], [(2, 0, 4)], [(0, 60, 5)], [(0, 0, 4), (0, 4, 4)], [(0, 0, 0)]):
        n = sum(r[2] for r in runs)
        with pytest.raises(tgx.TgxError) as e:
            dec.prefill_runs(runs, x[: max(n, 1)])
        assert e.value.kind == "shape"


def test_nan_left_in_a_reused_block_past_the_run_never_reaches_its_outputs(ctx):
    """attention_rows.comp:1-13: keys and values past the workgroup's last position read as zero.
    A request fed NaN leaves NaN at positions 0..149 of its slot's blocks; released, the next
    request in the same blocks prefills 0..99 (a run ending inside a NaN block) and steps on:
    finite, and bit for bit as on a fresh decoder."""
    spec = tiny_spec(layers=2)
    cap = 256
    x = inputs(spec, 104)
    dec = make_decoder(ctx, spec, cap)
    fresh = make_decoder(ctx, spec, cap)
    dec.prefill(0, np.full((150, spec.hidden), np.nan, dtype=np.float32))
    dec.release_slot(0)
    got, want = dec.prefill(0, x[:100]), fresh.prefill(0, x[:100])
    assert np.all(np.isfinite(got))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for t in range(100, 104):
        a, b = dec.step(t, x[t]), fresh.step(t, x[t])
        assert np.all(np.isfinite(a)) and np.array_equal(a.view(np.uint32), b.view(np.uint32)), t
    dec.close()
    fresh.close()
