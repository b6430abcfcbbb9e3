"""The runtime beneath the models on the CPU (no device): the kernel table by name with its
bindings in order (crates/graph/src/kernels.rs:104-161 keeps the same per kernel), the RoPE tables
as Shape::rope_tables computes them (crates/graph/src/decode.rs:143-168, unit-tested at
decode.rs:1232-1242), and the weight tiles' refusals."""

import numpy as np
import pytest


def test_the_kernels_keep_the_reference_names_and_binding_order():
    import tgx.runtime as rt

    table = {k.name: k for k in rt.kernels()}
    # attention_decode does attention_split's and attention_combine's work in one kernel.
    decode = {"gemv_qkv_rope", "attention_decode", "gemv_residual", "gemv_gate_up", "rmsnorm", "stream_read"}
    assert decode <= set(table)
    table = {k: table[k] for k in decode}
    names = lambda k: [b.name for b in table[k].bindings]
    # The reference's bindings keep their relative order (kernels.rs:104-161): x, gain, W, cos,
    # sin, position -> q, cache; x, W, residual -> out; x, gain -> out; data -> out.
    qkv = names("gemv_qkv_rope")
    for a, b in zip(["x", "gain", "w", "cos", "sin", "positions", "q", "kv"], ["gain", "w", "cos", "sin", "positions", "q", "kv", None]):
        if b is not None:
            assert qkv.index(a) < qkv.index(b), (a, b)
    assert names("gemv_residual")[:3] == ["x", "w", "residual"] and names("gemv_residual")[4] == "out"
    assert names("rmsnorm")[:3] == ["x", "gain", "out"]
    assert names("stream_read") == ["data", "out"]
    # What each kernel writes, and only that.
    writes = {k: [b.name for b in table[k].bindings if b.access == rt.WRITE] for k in table}
    assert writes == {
        "gemv_qkv_rope": ["q", "kv"],
        "attention_decode": ["attended"],
        "gemv_residual": ["out", "out_n", "out_sq"],
        "gemv_gate_up": ["mlp"],
        "rmsnorm": ["out", "positions"],
        "stream_read": ["out"],
    }
    common = ("hidden", "inner", "heads", "kv_heads", "rows", "capacity", "slots", "max_blocks", "blocks", "eps", "rope",
              "head_dim")
    assert table["attention_decode"].constants == common
    for k in ("gemv_qkv_rope", "gemv_gate_up"):
        assert table[k].constants == common + ("sq_cols",)
    assert table["gemv_residual"].constants == common + ("K", "N", "strip_rows")
    assert table["rmsnorm"].constants == common + ("advance",)
    assert table["stream_read"].constants == ()


PREFILL = ("rows", "hidden", "inner", "heads", "kv_heads", "head_dim", "capacity", "slots", "max_blocks", "blocks", "eps", "rope")
LOCAL = ("tokens", "seq_tokens", "hidden", "inner", "heads", "kv_heads", "eps", "rope")

# Each kernel past the decode step's: its bindings in order, what it writes, and its constants.
# The reference declares prefill.rs:32-81 (norm_rows, add_norm_rows, rope_rows, attention_rows,
# silu_mul_rows beside its GEMMs), local/mod.rs:28-113 (local_norm .. dit_euler), lm_side.rs:28-38
# (gemv_linear) and prompt.rs:55-67 (select_rows), reads first and writes after, which these keep.
# Where a GEMM carries the reference's row kernel as its epilogue the name says both, and the
# run binding (rows in the reference's run buffer) is a constant here.
WIDER = {
    "norm_rows": (["x", "gain", "out"], ["out"], PREFILL),
    "final_norm_rows": (["x", "gain", "out"], ["out"], PREFILL),
    "gemm_rope_rows": (["x", "w", "row_sq", "cos", "sin", "positions", "slots", "table", "q", "kv"], ["q", "kv"], PREFILL),
    "attention_rows": (["q", "kv", "table", "tiles", "attended"], ["attended"], PREFILL + ("tiles",)),
    "gemm_add_norm_rows": (["x", "w", "residual", "next_gain", "out", "out_n", "out_sq"], ["out", "out_n", "out_sq"],
                           PREFILL + ("K", "N", "strip_rows", "residual_in")),
    "gemm_silu_mul_rows": (["x", "w", "row_sq", "mlp"], ["mlp"], PREFILL + ("K", "N")),
    "local_norm": (["x", "gain", "normed", "row_sq"], ["normed", "row_sq"], LOCAL),
    "local_qkv_rope": (["x", "w", "row_sq", "cos", "sin", "q", "k", "v"], ["q", "k", "v"], LOCAL),
    "local_attention": (["q", "k", "v", "attended"], ["attended"], LOCAL),
    "local_partial": (["x", "w", "partial"], ["partial"], LOCAL + ("K", "N", "parts")),
    "local_add_norm": (["partial", "residual", "gain", "sum", "normed", "row_sq"], ["sum", "normed", "row_sq"], LOCAL + ("parts",)),
    "local_final_norm": (["partial", "residual", "gain", "sum", "out"], ["sum", "out"], LOCAL + ("parts",)),
    "local_gemm_add_norm": (["x", "w", "residual", "next_gain", "sum", "normed", "row_sq"], ["sum", "normed", "row_sq"],
                            LOCAL + ("K", "N", "parts")),
    "local_gate_up": (["x", "w", "row_sq", "mlp"], ["mlp"], LOCAL),
    "local_embed": (["frames", "w", "bias", "tokens", "gain", "x0", "normed", "row_sq"], ["x0", "normed", "row_sq"],
                    LOCAL + ("patch_rows", "channels", "frames", "first", "copy_at", "copies", "guided", "shared", "seqs")),
    "cfm_noise": (["noise", "sampling", "state"], ["state"], ("rows", "len")),
    "dit_euler": (["x", "row_sq", "gain", "w", "bias", "sampling", "state"], ["state"],
                  LOCAL + ("patch_rows", "channels", "frames", "first", "dt")),
    "gemv_linear": (["x0", "x1", "w", "bias", "out"], ["out"], ("rows", "K0", "K1", "N", "offset", "stride", "act", "levels")),
    "select_rows": (["flags", "a", "b", "out"], ["out"], ("rows", "K")),
}


def test_the_prefill_local_stack_dit_and_heads_kernels_are_in_the_table_by_name():
    import tgx.runtime as rt

    table = {k.name: k for k in rt.kernels()}
    assert set(table) == set(WIDER) | {"gemv_qkv_rope", "attention_decode", "gemv_residual", "gemv_gate_up", "rmsnorm",
                                       "stream_read"}
    for name, (bindings, writes, constants) in WIDER.items():
        k = table[name]
        assert [b.name for b in k.bindings] == bindings, name
        assert [b.name for b in k.bindings if b.access == rt.WRITE] == writes, name
        # reads first, then writes, as the reference declares them
        access = [b.access for b in k.bindings]
        assert access == sorted(access), name
        assert k.constants == constants, name
        assert rt.kernel(name).name == name


def test_an_unknown_kernel_is_refused():
    import tgx
    import tgx.runtime as rt

    with pytest.raises(tgx.TgxError) as e:
        rt.kernel("attention_split")
    assert e.value.kind == "kernels"


def test_rope_tables_as_the_reference_unit_tests_them():
    """decode.rs:1232-1242: identity at t = 0, cos 1 and sin 1 at t = 1 for j = 0; every entry the
    f32 recipe 1 / theta^(2j / d), t r inv, as the oracle restates it."""
    import oracle
    import tgx
    import tgx.runtime as rt

    shape = tgx.Shape(capacity=96)
    cos, sin = rt.rope_tables(shape)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)
    # f32's cos(1) and sin(1): the double values rounded once to f32.
    assert cos[1, 0] == np.float32(np.cos(1.0)) and sin[1, 0] == np.float32(np.sin(1.0))
    ref_cos, ref_sin = oracle.rope_tables(96, 64)
    assert np.array_equal(cos, ref_cos) and np.array_equal(sin, ref_sin)


def test_weight_tiles_take_whole_strips_and_k_blocks():
    import tgx.runtime as rt

    assert rt.tiles_bytes(rt.TILES_QKV, 1280, 1024) == 1280 * 1024 * 2
    assert rt.tiles_bytes(rt.TILES_4, 1024, 4096) == 1024 * 4096 * 2
    assert rt.tiles_bytes(rt.TILES_16, 8192, 1024) == 8192 * 1024 * 2
    assert rt.tiles_bytes(rt.TILES_16, 1000, 1024) == 0  # rows in strips of 16
    assert rt.tiles_bytes(rt.TILES_4, 1024, 1000) == 0  # columns in k-blocks of 32
    assert rt.tiles_bytes(rt.TILES_QKV, 1040, 1024) == 0  # q/k/v rows a multiple of the head
    assert rt.tiles_bytes(7, 16, 32) == 0


def test_attention_tiles_take_the_positions_of_the_groups_instance():
    """tgx_attention_tile: the positions a prefill attention tile may hold, by the group's instance
    (16 / group positions to a column group), and 0 for a shape the kernels do not take."""
    import tgx.runtime as rt

    for (heads, kv, d), want in {(16, 16, 64): 32, (16, 8, 64): 32, (48, 16, 64): 40, (16, 4, 64): 32, (80, 16, 64): 24,
                                 (48, 8, 64): 16, (16, 2, 64): 16, (16, 2, 128): 16, (48, 4, 64): 16, (48, 4, 128): 8,
                                 (32, 2, 64): 16, (32, 2, 128): 8, (24, 8, 128): 40}.items():
        assert rt.attention_tile(heads, kv, d) == want, (heads, kv, d)
    for heads, kv, d in ((32, 1, 64), (16, 3, 64), (16, 2, 96), (16, 0, 64)):
        assert rt.attention_tile(heads, kv, d) == 0, (heads, kv, d)
