"""tgx_prefill_runs_noalloc (no counterpart in the reference; for callers that cannot allocate
device memory) against tgx_prefill_runs, through the C ABI: two calls in a row, the second
smaller than the first (the scratch keeps the first call's larger tensors), each bit for bit as
the allocating entry point's outputs, cache writes and the steps that read them; no device memory
allocated; runs past the scratch refused before anything runs."""

import numpy as np
import pytest

from test_decode_gpu import inputs, make_decoder, tiny_spec

pytestmark = pytest.mark.gpu


def _same(a, b) -> bool:
    return np.array_equal(np.ascontiguousarray(a, np.float32).view(np.uint32), np.ascontiguousarray(b, np.float32).view(np.uint32))


def test_the_prefill_without_allocating_is_the_prefill_bit_for_bit(ctx):
    import tgx

    spec = tiny_spec(layers=2)
    cap = 1280
    x = inputs(spec, 1200)
    alloc = make_decoder(ctx, spec, cap, rows=2, slots=2)
    fixed = make_decoder(ctx, spec, cap, rows=2, slots=2)
    before = fixed.device_bytes()
    print(f"[no_alloc] decoders of {before} device bytes each", flush=True)
    calls = [
        ([(0, 0, 300), (1, 0, 260)], x[:560]),  # 560 rows, padded to 768
        ([(0, 300, 40)], x[560:600]),  # 40 rows, padded to 256: a smaller call after a larger one
    ]
    for k, (runs, xs) in enumerate(calls):
        print(f"[no_alloc] call {k}: runs {runs}", flush=True)
        got = fixed.prefill_runs_noalloc(runs, xs)
        want = alloc.prefill_runs(runs, xs)
        assert np.all(np.isfinite(got)), k
        assert _same(got, want), f"call {k}: outputs differ"
    assert fixed.device_bytes() == before, "the no-alloc prefill allocated device memory"
    assert alloc.device_bytes() > before  # the allocating prefill grew its tensors
    for slot, n in ((0, 340), (1, 260)):
        ka, va = alloc.read_cache(slot, n)
        kb, vb = fixed.read_cache(slot, n)
        assert _same(ka, kb) and _same(va, vb), f"slot {slot} cache"
    at = [tgx.Row(340, 0), tgx.Row(260, 1)]
    assert _same(fixed.step_rows(at, x[600:602]), alloc.step_rows(at, x[600:602]))
    # 1100 positions need 1280 rows of tensors, past the 32 MiB scratch at this shape: refused,
    # the cache and the decoder's memory as they were.
    k0, v0 = fixed.read_cache(0, 341)
    with pytest.raises(tgx.TgxError) as e:
        fixed.prefill_runs_noalloc([(0, 0, 1100)], x[:1100])
    assert e.value.kind == "shape" and "scratch" in str(e.value), str(e.value)
    k1, v1 = fixed.read_cache(0, 341)
    assert _same(k0, k1) and _same(v0, v1)
    assert fixed.device_bytes() == before
    alloc.close()
    fixed.close()
