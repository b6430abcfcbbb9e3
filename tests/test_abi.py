"""The C ABI on the CPU: the library loads and exports every entry point include/tgx.h declares,
and the host-side decisions the reference unit-tests without a GPU — shape refusals
(crates/graph/src/decode.rs:1011-1028), Batch::placement's words and refusals
(decode.rs:1073-1092), Shape::weight_bytes (decode.rs:947) — hold here."""

import ctypes
import re
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent


def header_functions():
    text = (ROOT / "include" / "tgx.h").read_text()
    return sorted(set(re.findall(r"^(?:tgx_status|void|const char\*|int|uint64_t)\s+(tgx_\w+)\(", text, re.M)))


def test_the_library_exports_every_function_the_header_declares():
    import tgx

    lib = tgx.library()
    names = header_functions()
    assert len(names) >= 25
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    assert set(tgx.EXPORTS) <= set(names)


def test_without_a_device_a_context_is_refused_not_faked():
    import tgx

    try:
        import torch

        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if has_gpu:
        pytest.skip("a GPU is present")
    with pytest.raises(tgx.TgxError) as e:
        tgx.Context(0)
    assert e.value.kind in ("no_device", "hip")


def test_weight_bytes_as_the_reference_counts_them():
    import tgx

    ref = tgx.Shape(hidden=2048, inner=6144, heads=16, kv_heads=2, head_dim=128, layers=28)
    assert ref.weight_bytes() == 2_642_644_992  # decode.rs:947
    assert tgx.Shape().weight_bytes() == 717_326_336  # the 24-layer backbone at hidden 1024
    assert tgx.Shape().kv_bytes_per_position() == 12_288


def test_spare_rows_are_placed_past_every_position_and_a_slot_is_taken_once():
    """decode.rs:1073-1092, word for word."""
    import tgx

    at = tgx.Row
    assert tgx.placement(4, 64, [at(5, 2), None, at(0, 0)]) == [5, tgx.SPARE, 0, 2, tgx.SPARE, 0]
    for rows in ([at(5, 2), at(9, 2), None], [at(64, 0), None, None], [at(1, 4), None, None]):
        with pytest.raises(tgx.TgxError) as e:
            tgx.placement(4, 64, rows)
        assert e.value.kind == "shape"


@pytest.mark.parametrize(
    "change, batch",
    [
        (dict(head_dim=96), dict()),
        (dict(head_dim=256), dict()),
        # hidden past 2048 (VoxCPM2's LMs are 2048 wide), an FFN or heads x head_dim past 6144
        (dict(hidden=4096), dict()),
        (dict(hidden=2048, inner=7168, head_dim=128), dict()),
        (dict(heads=64, kv_heads=8, head_dim=128), dict()),
        (dict(head_dim=128, capacity=16385), dict()),
        (dict(heads=16, kv_heads=3), dict()),
        # 32 query heads to a KV head: past the decode attention's 16 columns
        (dict(heads=32, kv_heads=1), dict()),
        # a group of 16 whose q/k/v rows (18 heads of 64) are not a multiple of the prefill's 256
        (dict(heads=16, kv_heads=1), dict()),
        (dict(capacity=0), dict()),
        (dict(hidden=1000), dict()),
        (dict(inner=5000), dict()),
        (dict(inner=8192), dict()),
        (dict(), dict(rows=3, slots=2)),
        (dict(), dict(rows=65, slots=65)),
        (dict(), dict(block_tokens=32)),
        (dict(), dict(rows=0, slots=1)),
    ],
)
def test_shapes_the_kernels_cannot_cover_are_refused(change, batch):
    import tgx

    shape = tgx.Shape(**change)
    b = tgx.Batch(**{**dict(rows=1, slots=1), **batch})
    with pytest.raises(tgx.TgxError) as e:
        tgx.check_shape(shape, b)
    assert e.value.kind == "shape"


def test_voxcpm2s_own_lm_shapes_are_taken():
    """VoxCPM2's base and residual LMs (crates/graph/src/decode.rs:919-933,
    crates/graph/src/lm_side.rs:665-679): hidden 2048, FFN 6144, 16 heads over 2 KV heads of 128
    dimensions, at the reference's capacity of 1024 and at 4096."""
    import tgx

    for capacity in (1024, 4096):
        for rope in (True, False):
            shape = tgx.Shape(hidden=2048, inner=6144, heads=16, kv_heads=2, head_dim=128, layers=28, capacity=capacity,
                              rope=rope)
            for rows in (1, 16, 64):
                tgx.check_shape(shape, tgx.Batch(rows=rows, slots=rows))


def test_the_backbone_shapes_are_taken():
    import tgx

    for rows in (1, 16, 17, 32, 64):
        tgx.check_shape(tgx.Shape(capacity=2048), tgx.Batch(rows=rows, slots=rows))
    tgx.check_shape(tgx.Shape(rope=False, layers=8), tgx.Batch(rows=4, slots=8))


@pytest.mark.parametrize("heads,kv_heads", [(16, 16), (16, 8), (16, 4), (16, 2), (32, 2), (48, 16), (80, 16), (48, 8), (80, 8), (48, 4)])
def test_groups_of_one_to_sixteen_query_heads_a_kv_head_are_taken(heads, kv_heads):
    """Groups of 1 to 16 query heads to a KV head (here 1, 2, 4, 8, 16 and 3, 5, 6, 10, 12), each
    with a prefill attention instance and decode attention columns."""
    import tgx

    tgx.check_shape(tgx.Shape(heads=heads, kv_heads=kv_heads), tgx.Batch(rows=4, slots=4))


def test_groups_of_one_to_sixteen_are_taken_and_thirty_two_refused_with_its_reason():
    import tgx

    for heads, kv, head_dim in ((16, 16, 64), (16, 8, 64), (16, 4, 64), (16, 2, 64), (32, 2, 64), (16, 1, 128), (16, 2, 128),
                                (32, 2, 128), (48, 3, 128), (24, 8, 128), (40, 8, 128), (48, 16, 64)):
        tgx.check_shape(tgx.Shape(heads=heads, kv_heads=kv, head_dim=head_dim), tgx.Batch(rows=1, slots=1))
    for heads, kv in ((32, 1), (34, 2), (16, 3)):
        with pytest.raises(tgx.TgxError) as e:
            tgx.check_shape(tgx.Shape(heads=heads, kv_heads=kv), tgx.Batch(rows=1, slots=1))
        assert e.value.kind == "shape" and "a whole group of 1 to 16" in str(e.value)


def test_null_arguments_are_refused_with_a_message():
    import tgx

    lib = tgx.library()
    assert lib.tgx_decoder_step(None, 0, None, None) == 8
    assert b"null" in lib.tgx_last_error()


def test_handles_made_from_a_context_close_newest_first():
    """A patch step (or an engine, or a prompter) uses the encoder, LM side and sampler made
    before it, which must outlive it (include/tgx.h): the context's close and the exit handler
    close the handles made from it newest first."""
    import tgx

    closed = []

    class Handle:
        def __init__(self, n):
            self.n = n

        def close(self):
            closed.append(self.n)

    handles = [Handle(n) for n in range(5)]
    for h in handles:
        tgx._opened(h)
    try:
        for h in tgx._newest_first(list(tgx._open_decoders)):
            if h in handles:
                h.close()
        assert closed == [4, 3, 2, 1, 0]
    finally:
        for h in handles:
            tgx._open_decoders.discard(h)
