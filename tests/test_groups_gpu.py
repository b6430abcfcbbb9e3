"""Groups of query heads to a KV head the shape check takes, on the GPU against the oracle: 16
query heads over 16, 8 and 4 KV heads (groups 1, 2 and 4), and 32 over 2 (a group of 16; its
q/k/v rows a multiple of the prefill GEMM's 256) and at head_dim 128 16 over 1 (the backbone's 16
over 2, a group of 8, is every other test's shape); groups that do not divide 16, whose prefill
column groups leave columns spare: 3 (48 over 16), 5 (80 over 16), 6 (48 over 8) and 12 (48 over
4) at head_dim 64, 3 and 5 at 128 (24 and 40 over 8). The reference's attention takes any group
(kernels/glsl/attention_split.comp:24-27); here a prefill attention instance takes the groups
whose column groups hold the same number of positions, and the decode attention's columns past
the group read its last head again.

For each group, a 2-layer stack: two prefill runs at once in two slots (ragged lengths, a tile
of positions left part-filled), then decode steps of both rows, per position against the fp64
oracle over the same bf16 weights (cosine >= 0.999 and max|got - ref| / max|ref| <= 1e-2); each
run's prefill bit for bit as alone, and each decode row bit for bit as alone.
"""

import numpy as np
import pytest

from conftest import distance, within
from test_decode_gpu import inputs, make_decoder, oracle_stack

pytestmark = pytest.mark.gpu


def group_spec(kv_heads, head_dim=64, heads=16):
    from tgx.synth import StackSpec

    return StackSpec(layers=2, heads=heads, kv_heads=kv_heads, head_dim=head_dim, dtype="bf16", seed=heads + kv_heads + head_dim)


@pytest.mark.parametrize(
    "heads,kv_heads,head_dim",
    [(16, 16, 64), (16, 8, 64), (16, 4, 64), (32, 2, 64), (16, 1, 128), (48, 16, 64), (80, 16, 64), (48, 8, 64), (48, 4, 64),
     (24, 8, 128), (40, 8, 128)],
)
def test_prefill_and_decode_at_each_group_match_the_oracle_and_rows_are_as_alone(ctx, heads, kv_heads, head_dim):
    spec = group_spec(kv_heads, head_dim, heads)
    print(f"group {spec.heads // kv_heads}: {spec.heads} heads over {kv_heads} KV heads, 2 layers", flush=True)
    cap = 256
    lengths = (130, 45)
    steps = 6
    x = inputs(spec, sum(lengths) + 2 * steps)
    runs_x = [x[:130], x[130:175]]
    dec = make_decoder(ctx, spec, cap, rows=2, slots=2)
    together = dec.prefill_runs([(0, 0, 130), (1, 0, 45)], x[:175])
    row = 0
    for slot, n in enumerate(lengths):
        ref = oracle_stack(spec, cap)
        want = ref.prefill(0, runs_x[slot])
        for t in range(n):
            d = distance(together[row + t], want[t])
            assert within(d), f"group {spec.heads // kv_heads}, run {slot}, position {t}: {d}"
        alone = make_decoder(ctx, spec, cap)
        got = alone.prefill(0, runs_x[slot])
        assert np.array_equal(got.view(np.uint32), together[row : row + n].view(np.uint32)), f"run {slot} alone"
        alone.close()
        row += n
    # Decode steps of both rows together, each against the oracle (continuing its prefill) and
    # bit for bit as the same row stepped alone.
    import tgx

    refs = []
    for slot, n in enumerate(lengths):
        r = oracle_stack(spec, cap)
        r.prefill(0, runs_x[slot])
        refs.append(r)
    alones = []
    for slot, n in enumerate(lengths):
        a = make_decoder(ctx, spec, cap)
        a.prefill(0, runs_x[slot])
        alones.append(a)
    xs = x[175:].reshape(steps, 2, spec.hidden)
    for s in range(steps):
        rows = [tgx.Row(lengths[0] + s, 0), tgx.Row(lengths[1] + s, 1)]
        got = dec.step_rows(rows, xs[s])
        for b in range(2):
            want = refs[b].decode(lengths[b] + s, xs[s, b])
            d = distance(got[b], want)
            assert within(d), f"group {spec.heads // kv_heads}, row {b}, step {s}: {d}"
            one = alones[b].step(lengths[b] + s, xs[s, b])
            assert np.array_equal(one.view(np.uint32), got[b].view(np.uint32)), f"row {b} step {s} alone"
    for a in alones:
        a.close()
    dec.close()
