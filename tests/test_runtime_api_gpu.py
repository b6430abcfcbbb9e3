"""The runtime beneath the models on the GPU: a decode step composed from the library's kernels by
name, over memory the caller holds, recorded as a program (as the graph crate records
decode_batch_graph over crates/vulkan, crates/graph/src/decode.rs:456-736) gives the decoder's
own step bit for bit; timed programs, programs without barriers, stream_read against the host's
XOR of the same words, copy regions, and the refusals a recording makes on the host
(crates/vulkan/src/recording.rs:89-119, crates/graph/src/kernels.rs Kernels::check).

Workload: a 2-layer MiniCPM-4 stack at hidden 1024 (16/2 heads, FFN 4096), 3 rows in 3 slots,
4 steps from position 0; a stream read of 64 KiB."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


class StepProgram:
    """A decode step of `spec`'s stack at `rows` rows recorded from the kernels by name: five
    dispatches a layer and the final norm, each after the one before (barrier)."""

    def __init__(self, ctx, spec, capacity, rows, slots, strip_rows=4, timed=False):
        import tgx
        import tgx.runtime as rt
        from tgx.synth import stack_weights

        self.rows, self.spec = rows, spec
        h, inner, H, KV = spec.hidden, spec.inner, spec.heads, spec.kv_heads
        max_blocks = (capacity + 63) // 64
        blocks = slots * max_blocks
        M = lambda n: rt.Memory(ctx, n)
        w = stack_weights(spec)
        self.mem = []

        def keep(m):
            self.mem.append(m)
            return m

        L = spec.layers
        self.qkv = [keep(M(rt.tiles_bytes(rt.TILES_QKV, spec.qkv_rows, h))) for _ in range(L)]
        self.o = [keep(M(h * H * 64 * 2)) for _ in range(L)]
        self.gu = [keep(M(2 * inner * h * 2)) for _ in range(L)]
        self.down = [keep(M(h * inner * 2)) for _ in range(L)]
        self.in_norm = [keep(M(h * 4)) for _ in range(L)]
        self.post_norm = [keep(M(h * 4)) for _ in range(L)]
        tiles = rt.TILES_4 if strip_rows == 4 else rt.TILES_16
        for l in range(L):
            self.qkv[l].write_tiles(w[f"layers.{l}.qkv_proj"], rt.TILES_QKV)
            self.o[l].write_tiles(w[f"layers.{l}.o_proj"], tiles)
            self.gu[l].write_tiles(w[f"layers.{l}.gate_up_proj"], rt.TILES_16)
            self.down[l].write_tiles(w[f"layers.{l}.down_proj"], tiles)
            self.in_norm[l].write(w[f"layers.{l}.input_layernorm"].astype(np.float32))
            self.post_norm[l].write(w[f"layers.{l}.post_attention_layernorm"].astype(np.float32))
        self.final_norm = keep(M(h * 4))
        self.final_norm.write(w["norm"].astype(np.float32))
        shape = tgx.Shape(hidden=h, inner=inner, heads=H, kv_heads=KV, head_dim=64, layers=L, capacity=capacity,
                          eps=spec.eps, rope_theta=spec.rope_theta)
        cos, sin = rt.rope_tables(shape)
        self.cos, self.sin = keep(M(cos.nbytes)), keep(M(sin.nbytes))
        self.cos.write(cos)
        self.sin.write(sin)
        # Each slot's blocks in order, the pool one slot after another.
        table = np.arange(blocks, dtype=np.uint32).reshape(slots, max_blocks)
        self.table_host = table
        self.table = keep(M(table.nbytes))
        self.table.write(table)
        self.positions, self.slots_mem = keep(M(rows * 4)), keep(M(rows * 4))
        self.row_table = keep(M(rows * max_blocks * 4))
        self.kv = [keep(M(blocks * KV * 2 * 64 * 64 * 2)) for _ in range(L)]
        self.x = keep(M(rows * h * 4))
        self.h_a, self.h_b, self.out = keep(M(rows * h * 4)), keep(M(rows * h * 4)), keep(M(rows * h * 4))
        self.xn_a, self.xn_b = keep(M(rows * h * 2)), keep(M(rows * h * 2))
        self.sq_a, self.sq_b = keep(M(rows * h)), keep(M(rows * h))  # [rows][h / 4] f32
        self.q, self.att = keep(M(rows * H * 64 * 2)), keep(M(rows * H * 64 * 2))
        self.mlp = keep(M(rows * inner * 2))
        c = [h, inner, H, KV, rows, capacity, slots, max_blocks, blocks, rt.f32_bits(spec.eps), 1, 64]
        self.program = p = rt.Program(ctx, timed=timed)
        for l in range(L):
            first = l == 0
            x_in = self.x if first else self.h_a
            p.dispatch("gemv_qkv_rope", [self.x if first else None, None if first else self.xn_a, None if first else self.sq_a,
                                         self.in_norm[l], self.qkv[l], self.cos, self.sin, self.positions, self.slots_mem,
                                         self.table, self.q, self.kv[l]], c + [strip_rows])
            p.dispatch("attention_decode", [self.q, self.kv[l], self.positions, self.row_table, self.att], c)
            p.dispatch("gemv_residual", [self.att, self.o[l], x_in, self.post_norm[l], self.h_b, self.xn_b, self.sq_b],
                       c + [H * 64, h, strip_rows])
            # The squares gemv_residual leaves span its strips' rows.
            p.dispatch("gemv_gate_up", [self.xn_b, self.sq_b, self.gu[l], self.mlp], c + [strip_rows])
            last = l == L - 1
            p.dispatch("gemv_residual", [self.mlp, self.down[l], self.h_b, None if last else self.in_norm[l + 1], self.h_a,
                                         None if last else self.xn_a, None if last else self.sq_a], c + [inner, h, strip_rows])
        p.dispatch("rmsnorm", [self.h_a, self.final_norm, self.out, None], c + [0])
        p.end()

    def step(self, rows, x):
        """rows: (position, slot) each; x [rows][hidden] f32."""
        pos = np.array([r[0] for r in rows], np.uint32)
        slot = np.array([r[1] for r in rows], np.uint32)
        self.positions.write(pos)
        self.slots_mem.write(slot)
        self.row_table.write(self.table_host[slot])
        self.x.write(np.ascontiguousarray(x, np.float32))
        self.program.run()
        return self.out.read(np.float32, self.rows * self.spec.hidden).reshape(self.rows, -1)

    def close(self):
        self.program.close()
        for m in self.mem:
            m.close()


def reference_decoder(ctx, spec, capacity, rows):
    import tgx
    from tgx.synth import stack_weights

    shape = tgx.Shape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads, head_dim=64,
                      layers=spec.layers, capacity=capacity, eps=spec.eps, rope_theta=spec.rope_theta)
    dec = tgx.Decoder(ctx, shape, tgx.Batch(rows=rows, slots=rows))
    dec.load_all(stack_weights(spec))
    return dec


@pytest.mark.parametrize("strip_rows", [4, 16])
def test_a_step_composed_by_kernel_name_is_the_decoders_step_bit_for_bit(ctx, strip_rows):
    """2 layers, 3 rows in slots 2, 0, 1, 4 steps from position 0: every output bit the decoder's
    (whose o_proj and down_proj take 4-row strips at 3 rows; 16-row strips give the same bits)."""
    import tgx
    from tgx.synth import StackSpec, embeddings

    spec = StackSpec(layers=2, seed=3)
    cap, rows = 128, 3
    print(f"[runtime api] 2 layers, {rows} rows, strips of {strip_rows}", flush=True)
    prog = StepProgram(ctx, spec, cap, rows, rows, strip_rows=strip_rows)
    dec = reference_decoder(ctx, spec, cap, rows)
    x = embeddings(7, "runtime-api", 4 * rows, spec.hidden).reshape(4, rows, spec.hidden)
    slots = [2, 0, 1]
    for t in range(4):
        got = prog.step([(t, s) for s in slots], x[t])
        want = dec.step_rows([tgx.Row(t, s) for s in slots], x[t])
        assert np.all(np.isfinite(got))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"step {t}"
    prog.close()
    dec.close()


def test_a_timed_program_gives_the_same_bits_and_each_dispatchs_time(ctx):
    import tgx
    from tgx.synth import StackSpec, embeddings

    spec = StackSpec(layers=2, seed=4)
    cap, rows = 64, 2
    timed = StepProgram(ctx, spec, cap, rows, rows, timed=True)
    plain = StepProgram(ctx, spec, cap, rows, rows)
    x = embeddings(8, "runtime-api-timed", 2 * rows, spec.hidden).reshape(2, rows, spec.hidden)
    for t in range(2):
        a = timed.step([(t, 0), (t, 1)], x[t])
        b = plain.step([(t, 0), (t, 1)], x[t])
        assert np.array_equal(a.view(np.uint32), b.view(np.uint32)), f"step {t}"
    times = timed.program.timings()
    assert [n for n, _ in times] == ["gemv_qkv_rope", "attention_decode", "gemv_residual", "gemv_gate_up", "gemv_residual"] * 2 + ["rmsnorm"]
    assert all(ms > 0 for _, ms in times)
    assert plain.program.timings() == []
    assert plain.program.elapsed_ms() > 0
    timed.close()
    plain.close()


def stream_words(data: np.ndarray) -> np.ndarray:
    """stream_read's output on the host: wave w of workgroup g XORs the 16-byte words
    256 g + 64 w + lane + i (grid 256) for its 64 lanes and i < 8 (grid = words / 2048)."""
    u4 = data.view(np.uint32).reshape(-1, 4)
    grid = u4.shape[0] // 2048
    stride = grid * 256
    out = np.zeros(grid * 4, np.uint32)
    for g in range(grid):
        for w in range(4):
            at = g * 256 + w * 64 + np.arange(64)
            idx = (at[:, None] + stride * np.arange(8)[None, :]).ravel()
            out[g * 4 + w] = np.bitwise_xor.reduce(u4[idx].ravel())
    return out


def test_stream_read_words_are_the_hosts_xor_and_dispatches_without_barrier_run_side_by_side(ctx):
    import tgx.runtime as rt

    rng = np.random.default_rng(5)
    a = rng.integers(0, 2**32, 16384, dtype=np.uint32)  # 64 KiB: 2 workgroups
    b = rng.integers(0, 2**32, 32768, dtype=np.uint32)  # 128 KiB: 4 workgroups
    ma, mb = rt.Memory(ctx, a.nbytes), rt.Memory(ctx, b.nbytes)
    ma.write(a)
    mb.write(b)
    oa, ob = rt.Memory(ctx, 8 * 4, rt.READBACK), rt.Memory(ctx, 16 * 4)
    p = rt.Program(ctx)
    p.dispatch("stream_read", [ma, oa], [], barrier=False)
    p.dispatch("stream_read", [mb, ob], [], barrier=False, groups=(4, 1, 1))
    p.end()
    p.run()
    assert np.array_equal(oa.read(np.uint32, 8), stream_words(a))
    assert np.array_equal(ob.read(np.uint32, 16), stream_words(b))
    p.close()
    for m in (ma, mb, oa, ob):
        m.close()


def test_copy_regions_move_the_bytes_named(ctx):
    import tgx.runtime as rt

    src = rt.Memory(ctx, 4096)
    data = np.arange(1024, dtype=np.uint32)
    src.write(data)
    dst = rt.Memory(ctx, 4096, rt.READBACK)
    rt.copy_regions(ctx, dst, src, [(0, 2048, 1024), (3072, 0, 512)])
    got = dst.read(np.uint32, 1024)
    assert np.array_equal(got[512:768], data[:256])
    assert np.array_equal(got[:128], data[768:896])
    assert np.all(got[128:512] == 0) and np.all(got[768:] == 0)
    with pytest.raises(Exception) as e:
        rt.copy_regions(ctx, dst, src, [(4000, 0, 200)])
    assert "shape" in str(e.value)
    src.close()
    dst.close()


def test_a_recording_refuses_on_the_host_what_the_kernels_could_not_run(ctx):
    """Bindings short of what the kernel reaches, a binding left out that is not optional, the
    wrong count of bindings or constants, a grid the kernel does not take, ranges past the memory
    (recording.rs binding_range), and memory freed while a program binds it."""
    import tgx
    import tgx.runtime as rt

    h, inner, H, KV, rows, cap = 1024, 4096, 16, 2, 2, 64
    c = [h, inner, H, KV, rows, cap, 2, 1, 2, rt.f32_bits(1e-5), 1, 64]
    q = rt.Memory(ctx, rows * H * 64 * 2)
    kv = rt.Memory(ctx, 2 * KV * 2 * 64 * 64 * 2)
    pos, row_table = rt.Memory(ctx, rows * 4), rt.Memory(ctx, rows * 4)
    att = rt.Memory(ctx, rows * H * 64 * 2)
    p = rt.Program(ctx)

    def refused(kind, *args, **kw):
        with pytest.raises(tgx.TgxError) as e:
            p.dispatch(*args, **kw)
        assert e.value.kind == kind, str(e.value)

    refused("shape", "attention_decode", [q, kv, pos, row_table, (att, 0, rows * H * 64 * 2 - 16)], c)
    refused("shape", "attention_decode", [q, kv, pos, row_table], c)
    refused("shape", "attention_decode", [q, kv, pos, None, att], c)
    refused("shape", "attention_decode", [q, kv, pos, row_table, att], c[:-1])
    refused("shape", "attention_decode", [q, kv, pos, row_table, att], c, groups=(2, 1, 1))
    refused("shape", "attention_decode", [q, (kv, 8, 0), pos, row_table, att], c)  # offset not 16-aligned
    refused("shape", "attention_decode", [q, kv, pos, row_table, att], c[:5] + [4096 * 64] + c[6:])  # capacity
    refused("shape", "attention_decode", [q, kv, pos, row_table, att], c[:7] + [0] + c[8:])  # a table too short
    refused("shape", "attention_decode", [q, kv, pos, row_table, att], c[:11] + [96])  # a head width not taken
    refused("shape", "attention_decode", [q, kv, pos, row_table, att], c[:11] + [128])  # q, kv short for 128
    refused("shape", "stream_read", [(q, 0, 1000), att], [])
    p.dispatch("attention_decode", [q, kv, pos, row_table, att], c, groups=(KV, rows, 1))
    with pytest.raises(tgx.TgxError) as e:
        q.close()
    assert e.value.kind == "busy"
    with pytest.raises(tgx.TgxError) as e:
        q.write(np.zeros(1, np.uint64), offset=q.nbytes - 4)
    assert e.value.kind == "shape"
    p.end()
    with pytest.raises(tgx.TgxError) as e:
        p.dispatch("attention_decode", [q, kv, pos, row_table, att], c)
    assert e.value.kind == "busy"
    # Every row spare: the program runs and writes nothing.
    pos.write(np.full(rows, 0xFFFFFFFF, np.uint32))
    p.run()
    p.close()
    for m in (q, kv, pos, row_table, att):
        m.close()


def test_a_calibration_places_a_programs_ends_on_the_hosts_clock(ctx):
    """Context::calibrate and Recording::ends (the reference's crates/vulkan/tests/recording.rs:
    346-372): two calibrations 50 ms apart measure the same time on both clocks; a run's ends are
    in order, apart by its elapsed time, and placed on the host's clock they fall between the
    host's readings before its start and after its wait."""
    import time

    import tgx.runtime as rt

    a = ctx.calibrate()
    time.sleep(0.05)
    b = ctx.calibrate()
    period = a["period_ns"]
    assert period > 0 and b["period_ns"] == period
    host = b["monotonic_ns"] - a["monotonic_ns"]
    gpu = (b["ticks"] - a["ticks"]) * period
    assert abs(gpu - host) <= a["deviation_ns"] + b["deviation_ns"] + 0.001 * host + 20_000, (gpu, host, a, b)
    data = np.random.default_rng(6).integers(0, 2**32, 16 << 20, dtype=np.uint32)  # 64 MiB
    m, o = rt.Memory(ctx, data.nbytes), rt.Memory(ctx, 8192 * 4)  # a word a wave: 2048 workgroups of 4
    m.write(data)
    p = rt.Program(ctx)
    p.dispatch("stream_read", [m, o], [])
    p.end()
    with pytest.raises(Exception):
        p.ends()  # no run yet
    p.run()
    cal = ctx.calibrate()
    before = time.monotonic_ns()
    p.start()
    p.wait()
    after = time.monotonic_ns()
    e0, e1 = p.ends()
    assert e1 > e0
    ms = p.elapsed_ms()
    assert abs((e1 - e0) * period * 1e-6 - ms) <= 0.01 + 0.01 * ms, (e0, e1, ms)
    on_host = lambda t: cal["monotonic_ns"] + (t - cal["ticks"]) * period
    slack = cal["deviation_ns"] + 50_000
    assert before - slack <= on_host(e0) <= on_host(e1) <= after + slack, (before, on_host(e0), on_host(e1), after)
    p.close()
    m.close()
    o.close()


def test_a_reset_program_takes_new_dispatches_and_lets_its_old_memory_go(ctx):
    """Recording::replace_program (recording.rs:219-244; the reference's recording.rs:260-280 test):
    a program re-recorded in place runs its new dispatches, timed when asked, and the memory only
    its old dispatches bound may be freed."""
    import tgx
    import tgx.runtime as rt

    rng = np.random.default_rng(7)
    a = rng.integers(0, 2**32, 16384, dtype=np.uint32)
    b = rng.integers(0, 2**32, 32768, dtype=np.uint32)
    ma, mb = rt.Memory(ctx, a.nbytes), rt.Memory(ctx, b.nbytes)
    ma.write(a)
    mb.write(b)
    oa, ob = rt.Memory(ctx, 8 * 4), rt.Memory(ctx, 16 * 4)
    p = rt.Program(ctx)
    p.dispatch("stream_read", [ma, oa], [])
    p.end()
    p.run()
    assert np.array_equal(oa.read(np.uint32, 8), stream_words(a))
    with pytest.raises(tgx.TgxError) as e:
        ma.close()
    assert e.value.kind == "busy"
    p.reset(timed=True)
    ma.close()
    p.dispatch("stream_read", [mb, ob], [])
    p.end()
    p.run()
    assert np.array_equal(ob.read(np.uint32, 16), stream_words(b))
    assert [n for n, _ in p.timings()] == ["stream_read"]
    p.close()
    for m in (mb, oa, ob):
        m.close()


def test_a_fence_spin_changes_how_waits_poll_and_not_what_they_give(ctx):
    """Context::set_fence_spin (context.rs:467-474): waits that poll for 2 ms before sleeping give
    the same words as waits that sleep at once, for programs and for a decoder's steps."""
    import tgx
    import tgx.runtime as rt
    from tgx.synth import StackSpec, embeddings

    data = np.random.default_rng(8).integers(0, 2**32, 16384, dtype=np.uint32)
    m, o = rt.Memory(ctx, data.nbytes), rt.Memory(ctx, 8 * 4)
    m.write(data)
    p = rt.Program(ctx)
    p.dispatch("stream_read", [m, o], [])
    p.end()
    spec = StackSpec(layers=2, seed=5)
    x = embeddings(9, "fence-spin", 2, spec.hidden)
    outs = []
    for spin in (2_000_000, 0):
        ctx.set_fence_spin(spin)
        p.run()
        dec = reference_decoder(ctx, spec, 64, 1)
        outs.append((o.read(np.uint32, 8), dec.step(0, x[0]), dec.step(1, x[1])))
        dec.close()
    for got, want in zip(outs[0], outs[1]):
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert np.array_equal(outs[1][0], stream_words(data))
    p.close()
    m.close()
    o.close()


def test_a_single_dispatch_runs_alone_and_is_timed(ctx):
    """Context::dispatch (context.rs:517-540, as the reference's kernel tests run one kernel): the
    stream-read words as a program gives them, a GPU time, and a refusal with its message."""
    import tgx
    import tgx.runtime as rt

    data = np.random.default_rng(9).integers(0, 2**32, 32768, dtype=np.uint32)
    m, o = rt.Memory(ctx, data.nbytes), rt.Memory(ctx, 16 * 4)
    m.write(data)
    ms = rt.dispatch(ctx, "stream_read", [m, o], [])
    assert ms > 0
    assert np.array_equal(o.read(np.uint32, 16), stream_words(data))
    with pytest.raises(tgx.TgxError) as e:
        rt.dispatch(ctx, "stream_read", [(m, 0, 1000), o], [])
    assert e.value.kind == "shape" and "stream_read" in str(e.value)
    m.close()  # the dispatch's program is gone: nothing binds the memory
    o.close()
