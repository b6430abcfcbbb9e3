"""Programs composed by kernel name past the decode step, over memory the caller holds (the
reference's registries: crates/graph/src/prefill.rs:32-81, local/mod.rs:28-113), each bit for bit
as the library's own run of the same work:

- a 2-layer prefill of two runs, then a run continuing one of them, against tgx_prefill_runs: the
  output rows and the cache both layers wrote;
- one DiT evaluation (a sample of 2 timesteps: one Euler step past CFG-Zero*'s zero init) against
  tgx_sampler_sample, at 1 row (22 tokens: the GEMMs' direct path, local_partial and
  local_add_norm) and 3 rows (66 tokens: the ring, local_gemm_add_norm).

Workload: MiniCPM-4-shaped stacks at hidden 1024 (16/2 heads of 64, FFN 4096); the prefill's
cache of 256 positions in 2 slots; the sampler's patches of 4 frames x 64 channels."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

SPARE = 0xFFFFFFFF


def key_index(p, d, D):
    return (((p // 16) * (D // 32) + d // 32) * 64 + ((d % 32) // 8) * 16 + p % 16) * 8 + d % 8


def value_index(p, d):
    return (((d // 16) * 2 + p // 32) * 64 + (((p % 32) % 16) // 4) * 16 + d % 16) * 8 + (p % 4) + 4 * ((p % 32) // 16)


def bf16_to_f32(u16):
    return (u16.astype(np.uint32) << 16).view(np.float32)


class PrefillStack:
    """A stack's weights, rotation tables and paged cache in memory the caller holds, and prefills
    of runs recorded from the prefill's kernels by name: norm_rows, then for each layer
    gemm_rope_rows, attention_rows, gemm_add_norm_rows (o_proj, the accumulators started at the
    residual), gemm_silu_mul_rows and gemm_add_norm_rows (down_proj), then final_norm_rows."""

    def __init__(self, ctx, spec, capacity, slots, strip_rows):
        import tgx
        import tgx.runtime as rt
        from tgx.synth import stack_weights

        self.ctx, self.spec, self.capacity, self.slots, self.strip_rows = ctx, spec, capacity, slots, strip_rows
        h, inner, H, KV, D = spec.hidden, spec.inner, spec.heads, spec.kv_heads, spec.head_dim
        self.max_blocks = (capacity + 63) // 64
        self.blocks = slots * self.max_blocks
        self.mem = []
        M = self.alloc
        w = stack_weights(spec)
        tiles = rt.TILES_4 if strip_rows == 4 else rt.TILES_16
        qkv_tiles = rt.TILES_QKV if D == 64 else rt.TILES_QKV128
        self.layers = []
        for l in range(spec.layers):
            L = {}
            for name, rows, cols, t in (("qkv_proj", spec.qkv_rows, h, qkv_tiles), ("o_proj", h, H * D, tiles),
                                        ("gate_up_proj", 2 * inner, h, rt.TILES_16), ("down_proj", h, inner, tiles)):
                L[name] = M(rt.tiles_bytes(t, rows, cols))
                L[name].write_tiles(w[f"layers.{l}.{name}"], t)
            for name in ("input_layernorm", "post_attention_layernorm"):
                L[name] = M(h * 4)
                L[name].write(w[f"layers.{l}.{name}"].astype(np.float32))
            L["kv"] = M(self.blocks * KV * 2 * 64 * D * 2)
            self.layers.append(L)
        self.final_norm = M(h * 4)
        self.final_norm.write(w["norm"].astype(np.float32))
        shape = tgx.Shape(hidden=h, inner=inner, heads=H, kv_heads=KV, head_dim=D, layers=spec.layers, capacity=capacity,
                          eps=spec.eps, rope_theta=spec.rope_theta)
        cos, sin = rt.rope_tables(shape)
        self.cos, self.sin = M(cos.nbytes), M(sin.nbytes)
        self.cos.write(cos)
        self.sin.write(sin)
        # Each slot's blocks in order, the pool one slot after another.
        self.table_host = np.arange(self.blocks, dtype=np.uint32).reshape(slots, self.max_blocks)
        self.table = M(self.table_host.nbytes)
        self.table.write(self.table_host)
        self.tile = rt.attention_tile(H, KV, D)  # positions an attention tile takes

    def alloc(self, nbytes):
        import tgx.runtime as rt

        m = rt.Memory(self.ctx, nbytes)
        self.mem.append(m)
        return m

    def run(self, runs, x):
        """runs: (slot, start, len) each, their rows one after another; x [rows][hidden] f32."""
        import tgx.runtime as rt

        spec = self.spec
        h, inner, H, KV, D = spec.hidden, spec.inner, spec.heads, spec.kv_heads, spec.head_dim
        rows = sum(n for _, _, n in runs)
        pad = (rows + 255) // 256 * 256
        pos = np.full(pad, SPARE, np.uint32)
        slot = np.full(pad, SPARE, np.uint32)
        tiles = []
        at = 0
        for s, start, n in runs:
            pos[at : at + n] = start + np.arange(n)
            slot[at : at + n] = s
            for t0 in range(0, n, self.tile):
                tiles.append((at + t0, start + t0, min(self.tile, n - t0), s))
            at += n
        tiles = np.array(tiles, np.uint32)
        local = []

        def M(nbytes):
            m = rt.Memory(self.ctx, nbytes)
            local.append(m)
            return m

        xin = M(pad * h * 4)
        xin.write(np.ascontiguousarray(x, np.float32))
        normed, row_sq = M(pad * h * 2), M(pad * (h // 128) * 4)
        q, attended = M(pad * H * D * 2), M(pad * H * D * 2)
        mid, hb, mlp, out = M(pad * h * 4), M(pad * h * 4), M(pad * inner * 2), M(rows * h * 4)
        positions, slots, tile_mem = M(pad * 4), M(pad * 4), M(tiles.nbytes)
        positions.write(pos)
        slots.write(slot)
        tile_mem.write(tiles)
        c = [rows, h, inner, H, KV, D, self.capacity, self.slots, self.max_blocks, self.blocks, rt.f32_bits(spec.eps), 1]
        p = rt.Program(self.ctx)
        Ls = self.layers
        p.dispatch("norm_rows", [xin, Ls[0]["input_layernorm"], normed], c)
        for l, L in enumerate(Ls):
            last = l + 1 == len(Ls)
            p.dispatch("gemm_rope_rows", [normed, L["qkv_proj"], None if l == 0 else row_sq, self.cos, self.sin, positions, slots,
                                          self.table, q, L["kv"]], c)
            p.dispatch("attention_rows", [q, L["kv"], self.table, tile_mem, attended], c + [len(tiles)])
            p.dispatch("gemm_add_norm_rows", [attended, L["o_proj"], xin if l == 0 else hb, L["post_attention_layernorm"], mid, normed,
                                              row_sq], c + [H * D, h, self.strip_rows, 1])
            p.dispatch("gemm_silu_mul_rows", [normed, L["gate_up_proj"], row_sq, mlp], c + [h, 2 * inner])
            p.dispatch("gemm_add_norm_rows", [mlp, L["down_proj"], mid, None if last else Ls[l + 1]["input_layernorm"], hb,
                                              None if last else normed, None if last else row_sq],
                       c + [inner, h, self.strip_rows, 0])
        p.dispatch("final_norm_rows", [hb, self.final_norm, out], c)
        p.end()
        p.run()
        got = out.read(np.float32, rows * h).reshape(rows, h)
        p.close()
        for m in local:
            m.close()
        return got

    def read_cache(self, slot, positions):
        """The cache as Decoder.read_cache gives it: k, v [layers][kv_heads][positions][head_dim]."""
        spec = self.spec
        KV, D = spec.kv_heads, spec.head_dim
        tile = 64 * D
        p = np.arange(positions)
        d = np.arange(D)
        kidx = key_index(p[:, None] % 64, d[None, :], D)
        vidx = value_index(p[:, None] % 64, d[None, :])
        blk = self.table_host[slot][p // 64]
        k = np.empty((spec.layers, KV, positions, D), np.float32)
        v = np.empty_like(k)
        for l, L in enumerate(self.layers):
            pool = L["kv"].read(np.uint16, self.blocks * KV * 2 * tile).reshape(self.blocks, KV, 2, tile)
            for kv in range(KV):
                k[l, kv] = bf16_to_f32(pool[blk[:, None], kv, 0, kidx])
                v[l, kv] = bf16_to_f32(pool[blk[:, None], kv, 1, vidx])
        return k, v

    def close(self):
        for m in self.mem:
            m.close()


@pytest.mark.parametrize("strip_rows,batch_rows", [(4, 2), (16, 20)])
def test_a_prefill_composed_by_kernel_name_is_tgx_prefill_runs_bit_for_bit(ctx, strip_rows, batch_rows):
    """2 layers; runs of 100 positions in slot 1 and 37 in slot 0 (137 rows, 256 padded), then 30
    more of slot 1 from position 100: every output bit and every cache bit the decoder's own
    prefill gives (its o_proj and down_proj in strips of `strip_rows`, as a decoder of
    `batch_rows` rows lays them)."""
    import tgx
    from tgx.synth import StackSpec, embeddings, stack_weights

    spec = StackSpec(layers=2, seed=17)
    cap, slots = 256, 2
    print(f"[prefill by name] strips of {strip_rows}", flush=True)
    stack = PrefillStack(ctx, spec, cap, slots, strip_rows)
    shape = tgx.Shape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads, head_dim=spec.head_dim,
                      layers=spec.layers, capacity=cap, eps=spec.eps, rope_theta=spec.rope_theta)
    dec = tgx.Decoder(ctx, shape, tgx.Batch(rows=batch_rows, slots=max(batch_rows, slots)))
    dec.load_all(stack_weights(spec))
    x = embeddings(9, "prefill-by-name", 167, spec.hidden)
    for runs, rows in (([(1, 0, 100), (0, 0, 37)], slice(0, 137)), ([(1, 100, 30)], slice(137, 167))):
        got = stack.run(runs, x[rows])
        want = dec.prefill_runs(runs, x[rows])
        assert np.all(np.isfinite(got))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), runs
    for s, n in ((0, 37), (1, 130)):
        gk, gv = stack.read_cache(s, n)
        wk, wv = dec.read_cache(s, n)
        assert np.array_equal(gk.view(np.uint32), wk.view(np.uint32)), f"keys of slot {s}"
        assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32)), f"values of slot {s}"
    dec.close()
    stack.close()


def test_a_long_prefill_composed_by_kernel_name_is_tgx_prefill_runs_bit_for_bit(ctx):
    """2 runs of 6700 positions (13,400 rows, 13,568 padded; the GEMMs past one round of
    workgroups, the attention's tiles reaching 105 cache blocks): every output bit and every
    cache bit as tgx_prefill_runs gives them."""
    import tgx
    from tgx.synth import StackSpec, embeddings, stack_weights

    spec = StackSpec(layers=2, seed=19)
    cap, slots, n = 6784, 2, 6700
    print("[prefill by name] 2 x 6700 positions", flush=True)
    stack = PrefillStack(ctx, spec, cap, slots, 4)
    shape = tgx.Shape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads, head_dim=spec.head_dim,
                      layers=spec.layers, capacity=cap, eps=spec.eps, rope_theta=spec.rope_theta)
    dec = tgx.Decoder(ctx, shape, tgx.Batch(rows=2, slots=slots))
    dec.load_all(stack_weights(spec))
    x = embeddings(11, "long-prefill-by-name", 2 * n, spec.hidden)
    runs = [(0, 0, n), (1, 0, n)]
    got = stack.run(runs, x)
    want = dec.prefill_runs(runs, x)
    assert np.all(np.isfinite(got))
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    for s in range(slots):
        gk, gv = stack.read_cache(s, n)
        wk, wv = dec.read_cache(s, n)
        assert np.array_equal(gk.view(np.uint32), wk.view(np.uint32)), f"keys of slot {s}"
        assert np.array_equal(gv.view(np.uint32), wv.view(np.uint32)), f"values of slot {s}"
    dec.close()
    stack.close()


FEAT, FRAMES = 64, 4
MU_TOKENS, TIME_AT, COND_AT = 2, 2, 3  # a sequence: mu, mu, time, cond frames, x frames


def euler_dt_of_two_timesteps():
    """The one Euler step a sample of 2 timesteps takes (dit.rs euler_schedule, the sampler's
    euler_steps): span = [1, t1, 0] with t1 = 0.5 + (cos(pi/2 0.5) - 1 + 0.5) in f32; the first
    step is CFG-Zero*'s zero init, the second goes from t1 by dt = t1. cos as the library's host
    code takes it: the C library's cosf."""
    libm = ctypes.CDLL("libm.so.6")
    libm.cosf.restype = ctypes.c_float
    libm.cosf.argtypes = [ctypes.c_float]
    f = np.float32
    t = f(0.5)
    c = f(libm.cosf(float(f(1.57079632679489661923) * t)))
    return float(t + ((c - f(1.0)) + t))


class DitEvaluation:
    """One sample of 2 timesteps recorded from the sampler's kernels by name: cfm_noise, the
    conditioning's local_embed (mu and the cond frames into both sequences, the unconditional's
    mu zero), the step's local_embed (the state's frames and the time token), the stack (up to 64
    tokens local_qkv_rope, local_attention, local_partial + local_add_norm, local_gate_up,
    local_partial + local_add_norm a layer; past 64 the pairs are local_gemm_add_norm), and
    dit_euler."""

    def __init__(self, ctx, spec, weights, rows, time_token):
        import tgx
        import tgx.runtime as rt

        self.ctx, self.rows = ctx, rows
        h, inner, H, KV = spec.hidden, spec.inner, spec.heads, spec.kv_heads
        C, F = FEAT, FRAMES
        T = COND_AT + 2 * F
        self.tokens = tokens = rows * 2 * T
        pad = (tokens + 15) // 16 * 16 if tokens <= 64 else (tokens + 63) // 64 * 64
        ring = pad > 64
        self.mem = []

        def M(nbytes):
            m = rt.Memory(ctx, nbytes)
            self.mem.append(m)
            return m

        def f32(name):
            a = np.ascontiguousarray(weights[name], np.float32)
            m = M(a.nbytes)
            m.write(a)
            return m

        def tiled(name, t):
            a = weights[name]
            m = M(rt.tiles_bytes(t, a.shape[0], a.shape[1]))
            m.write_tiles(a, t)
            return m

        layers = []
        for l in range(spec.layers):
            layers.append({
                "qkv": tiled(f"layers.{l}.qkv_proj", rt.TILES_QKV),
                "o": tiled(f"layers.{l}.o_proj", rt.TILES_16),
                "gu": tiled(f"layers.{l}.gate_up_proj", rt.TILES_16),
                "down": tiled(f"layers.{l}.down_proj", rt.TILES_16),
                "in": f32(f"layers.{l}.input_layernorm"),
                "post": f32(f"layers.{l}.post_attention_layernorm"),
            })
        final_norm = f32("norm")
        in_w, in_b, cond_w, cond_b = f32("in_proj.weight"), f32("in_proj.bias"), f32("cond_proj.weight"), f32("cond_proj.bias")
        out_w, out_b = tiled("out_proj.weight", rt.TILES_16), f32("out_proj.bias")
        time = M(h * 4)
        time.write(np.ascontiguousarray(time_token, np.float32))
        shape = tgx.Shape(hidden=h, inner=inner, heads=H, kv_heads=KV, head_dim=64, layers=spec.layers, capacity=T, eps=spec.eps,
                          rope_theta=spec.rope_theta)
        cos, sin = rt.rope_tables(shape)
        self.cos, self.sin = M(cos.nbytes), M(sin.nbytes)
        self.cos.write(cos)
        self.sin.write(sin)
        self.mu, self.cond, self.noise = M(rows * MU_TOKENS * h * 4), M(rows * C * F * 4), M(rows * C * F * 4)
        self.state, self.sampling = M(rows * C * F * 4), M(rows * 2 * 4)
        x0, xb, hb = M(pad * h * 4), M(pad * h * 4), M(pad * h * 4)
        normed0, row_sq0, normed, row_sq = M(pad * h * 2), M(pad * 16 * 4), M(pad * h * 2), M(pad * 16 * 4)
        q, k, v = M(pad * H * 64 * 2), M(pad * KV * 64 * 2), M(pad * KV * 64 * 2)
        attended, mlp, partial = M(pad * H * 64 * 2), M(pad * inner * 2), M(4 * pad * h * 4)
        c = [tokens, T, h, inner, H, KV, rt.f32_bits(spec.eps), 1]
        x_at = COND_AT + F
        self.program = p = rt.Program(ctx)
        p.dispatch("cfm_noise", [self.noise, self.sampling, self.state], [rows, C * F])
        p.dispatch("local_embed", [self.cond, cond_w, cond_b, self.mu, layers[0]["in"], x0, normed0, row_sq0],
                   c + [rows, C, F, COND_AT, 0, MU_TOKENS, 1, 0, 2])
        p.dispatch("local_embed", [self.state, in_w, in_b, time, layers[0]["in"], x0, normed0, row_sq0],
                   c + [rows, C, F, x_at, TIME_AT, 1, 0, 1, 2])
        for l, L in enumerate(layers):
            first = l == 0
            p.dispatch("local_qkv_rope", [normed0 if first else normed, L["qkv"], row_sq0 if first else row_sq, self.cos, self.sin,
                                          q, k, v], c)
            p.dispatch("local_attention", [q, k, v, attended], c)
            residual = x0 if first else xb
            if ring:
                p.dispatch("local_gemm_add_norm", [attended, L["o"], residual, L["post"], hb, normed, row_sq], c + [H * 64, h, 2])
            else:
                p.dispatch("local_partial", [attended, L["o"], partial], c + [H * 64, h, 2])
                p.dispatch("local_add_norm", [partial, residual, L["post"], hb, normed, row_sq], c + [2])
            p.dispatch("local_gate_up", [normed, L["gu"], row_sq, mlp], c)
            # After the last layer the final norm's sums of squares, for dit_euler to norm with.
            gain = layers[l + 1]["in"] if l + 1 < len(layers) else final_norm
            if ring:
                p.dispatch("local_gemm_add_norm", [mlp, L["down"], hb, gain, xb, normed, row_sq], c + [inner, h, 4])
            else:
                p.dispatch("local_partial", [mlp, L["down"], partial], c + [inner, h, 4])
                p.dispatch("local_add_norm", [partial, hb, gain, xb, normed, row_sq], c + [4])
        p.dispatch("dit_euler", [xb, row_sq, final_norm, out_w, out_b, self.sampling, self.state],
                   c + [rows, C, F, x_at, rt.f32_bits(euler_dt_of_two_timesteps())])
        p.end()

    def sample(self, mu, cond, noise, sampling):
        self.mu.write(np.ascontiguousarray(mu, np.float32))
        self.cond.write(np.ascontiguousarray(cond, np.float32))
        self.noise.write(np.ascontiguousarray(noise, np.float32))
        self.sampling.write(np.ascontiguousarray(sampling, np.float32))
        self.program.run()
        return self.state.read(np.float32, self.rows * FEAT * FRAMES).reshape(self.rows, FEAT, FRAMES)

    def close(self):
        self.program.close()
        for m in self.mem:
            m.close()


@pytest.mark.parametrize("rows", [1, 3])
def test_a_dit_evaluation_composed_by_kernel_name_is_tgx_sampler_sample_bit_for_bit(ctx, rows):
    """A 2-layer DiT; time MLPs whose second layers are zero, so the step's time token is the time
    MLP's last bias (the host's MLP then adds nothing to it): the sampled patch, bit for bit."""
    import tgx
    from tgx.patch import PatchShape, Sampler
    from tgx.synth import StackSpec, sampler_weights

    spec = StackSpec(layers=2, hidden=1024, inner=4096, dtype="bf16", seed=23)
    w = dict(sampler_weights(spec, FEAT))
    for m in ("time_mlp", "delta_time_mlp"):
        w[f"{m}.linear_2.weight"] = np.zeros_like(w[f"{m}.linear_2.weight"])
    w["delta_time_mlp.linear_2.bias"] = np.zeros_like(w["delta_time_mlp.linear_2.bias"])
    shape = tgx.Shape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads, head_dim=64,
                      layers=spec.layers, capacity=16, eps=spec.eps, rope_theta=spec.rope_theta)
    print(f"[dit by name] {rows} rows", flush=True)
    sampler = Sampler(ctx, shape, PatchShape(FEAT, FRAMES, 2, rows))
    sampler.load_all(w)
    composed = DitEvaluation(ctx, spec, w, rows, w["time_mlp.linear_2.bias"])
    rng = np.random.default_rng(31 + rows)
    mu = rng.standard_normal((rows, MU_TOKENS, spec.hidden)).astype(np.float32)
    cond = rng.standard_normal((rows, FEAT, FRAMES)).astype(np.float32)
    noise = rng.standard_normal((rows, FEAT, FRAMES)).astype(np.float32)
    sampling = np.array([[1.0, 2.0], [0.7, 1.5], [1.2, 3.0]][:rows], np.float32)
    want = sampler.sample(mu, cond, noise, sampling)
    got = composed.sample(mu, cond, noise, sampling)
    assert np.all(np.isfinite(got))
    # The step moved the patch: the comparison is of the Euler step, not of the noise alone.
    assert not np.array_equal(got, sampling[:, :1, None] * noise)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    composed.close()
    sampler.close()


def test_the_wider_kernels_refuse_on_the_host_what_they_could_not_run(ctx):
    """Each kernel past the decode step checks its constants and every binding's bytes before
    anything is recorded (Kernels::check, crates/graph/src/kernels.rs), as the decode kernels do."""
    import tgx
    import tgx.runtime as rt

    big = rt.Memory(ctx, 64 << 20)
    small = rt.Memory(ctx, 1024)  # short of a 1024-wide gain, or a 2 x 8 block table's 64 bytes and more
    tiny = rt.Memory(ctx, 16)
    p = rt.Program(ctx)

    def refused(name, bindings, constants):
        with pytest.raises(tgx.TgxError) as e:
            p.dispatch(name, bindings, constants)
        assert e.value.kind == "shape", (name, str(e.value))

    eps = rt.f32_bits(1e-5)
    pre = [256, 1024, 4096, 16, 2, 64, 512, 2, 8, 16, eps, 1]  # rows .. rope
    refused("norm_rows", [big, small, big], pre)  # gain short of 1024 floats
    refused("norm_rows", [big, big, big], [0] + pre[1:])  # no rows
    refused("attention_rows", [big, big, big, big, big], pre + [0])  # no tiles
    refused("attention_rows", [big, big, big, big, big], pre[:5] + [96] + pre[6:] + [4])  # a head width not taken
    refused("gemm_add_norm_rows", [big, big, big, None, big, None, None], pre + [1000, 1024, 4, 1])  # K
    refused("gemm_add_norm_rows", [big, big, big, big, big, None, None], pre + [1024, 1024, 4, 1])  # next norm in part
    refused("gemm_silu_mul_rows", [big, big, None, big], pre + [1024, 300])  # N
    refused("gemm_rope_rows", [big, big, None, big, big, big, big, tiny, big, big], pre)  # table short of 2 x 8 entries
    loc = [22, 11, 1024, 4096, 16, 2, eps, 1]  # tokens .. rope
    refused("local_norm", [big, big, big, big], [23] + loc[1:])  # tokens not whole sequences
    refused("local_norm", [big, big, big, big], loc[:2] + [2048] + loc[3:])  # a stack 2048 wide
    refused("local_partial", [big, big, big], loc + [1024, 1024, 5])  # parts
    refused("local_add_norm", [None, big, big, None, big, big], loc + [2])  # parts without partial
    refused("local_embed", [big, big, big, big, None, big, None, None], loc + [1, 64, 5, 7, 2, 1, 0, 0, 2])  # frames
    refused("local_embed", [big, big, big, big, big, big, None, None], loc + [1, 64, 4, 7, 2, 1, 0, 0, 2])  # gain alone
    refused("dit_euler", [big, big, big, big, big, big, big], loc + [1, 20, 4, 7, rt.f32_bits(0.1)])  # channels
    refused("dit_euler", [big, big, big, big, big, big, big], loc + [1, 64, 4, 7, rt.f32_bits(float("nan"))])  # dt
    refused("cfm_noise", [big, big, big], [0, 256])
    refused("gemv_linear", [big, None, big, big, big], [4, 1024, 1024, 256, 0, 256, 0, 0])  # K1 without x1
    refused("gemv_linear", [big, None, big, big, big], [4, 1024, 0, 256, 16, 256, 0, 0])  # out rows too narrow
    refused("select_rows", [big, big, big, big], [4, 6])  # K not a multiple of 4
    p.close()
    for m in (big, small, tiny):
        m.close()
