"""Benchmark of the MiniCPM-4 backbone's decode step on one MI355X.

Workload (the headline): the full backbone shape — 24 layers, hidden 1024, 16 query / 2 KV heads,
head_dim 64, SiLU-gated FFN 4096, bf16 weights drawn N(0, 0.02) from a seed — at batch 1, its
cache filled to position 256 (a 256-position prompt), then `--steps` decode steps (500 by default),
each at the next position, every input already in HBM. A step is one pass of the stack: 121
kernels launched as one recorded HIP graph. `value` is decode steps per second.

Beside it on the same JSON line:
- "batches": decode at 16 and 64 requests, contexts drawn U[64, 1024] (seeded), 200 steps;
- "roofline": the step's dominant kernel for HBM, the one whose launches move the most
  algorithmic bytes per step (gate/up: 56 % of the weights), its algorithmic bytes per launch over
  its average duration from per-dispatch HIP events (each recorded by the kernel's own dispatch);
  "roofline_longest" the same for the kernel with the most time per step;
- "cpu_baseline": the fp32 CPU path (the oracle, OpenMP over the host's cores) on a bounded
  sample of the same workload;
- "prefill": 8 runs of 2048 positions at once, tok/s and the GEMMs' share of bf16 MFMA peak;
- "tts_step": the full per-patch pipeline at 16 requests (LM side with both LMs, then the LocDiT
  sampler's 10 Euler steps with guidance), patch steps per second.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
for p in (ROOT / "tgtts-v4_amd", ROOT / "oracle"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

METRIC = "LM decode steps/s at batch 1/16/64; % of 8 TB/s HBM roofline; prefill tok/s"
HBM_PEAK = 8.0e12  # MI355X HBM3E, bytes/s
PROMPT = 256


def log(*a):
    print("[bench]", *a, file=sys.stderr, flush=True)


def spec_and_shape(capacity: int):
    import tgx
    from tgx.synth import StackSpec

    spec = StackSpec(layers=24, dtype="bf16", seed=0)
    shape = tgx.Shape(hidden=spec.hidden, inner=spec.inner, heads=spec.heads, kv_heads=spec.kv_heads,
                      head_dim=spec.head_dim, layers=spec.layers, capacity=capacity, eps=spec.eps,
                      rope_theta=spec.rope_theta)
    return spec, shape


def load(dec, weights):
    from tgx.synth import bf16_bits

    for name, v in weights.items():
        dec.load(name, bf16_bits(v))


def kernel_bytes(shape, label: str, rows: int, kv_positions: int) -> int:
    """Algorithmic HBM bytes of one launch: weights once, activations in and out, and for the
    attention the keys and values of every position read (kv_positions over the batch)."""
    h, i, H, KV, d = shape.hidden, shape.inner, shape.heads, shape.kv_heads, shape.head_dim
    qkv = (H + 2 * KV) * d
    if label == "gemv_qkv_rope":
        return qkv * h * 2 + rows * h * 4 + rows * qkv * 2
    if label == "attention_decode":
        return kv_positions * KV * d * 2 * 2 + rows * H * d * 2 * 2
    if label == "o_proj":
        return h * H * d * 2 + rows * H * d * 2 + rows * h * 4 * 2
    if label == "gemv_gate_up":
        return 2 * i * h * 2 + rows * h * 4 + rows * i * 2
    if label == "down_proj":
        return h * i * 2 + rows * i * 2 + rows * h * 4 * 2
    if label == "final_norm":
        return rows * h * 4 * 2 + h * 4
    return 0


def step_bytes(shape, positions) -> int:
    """A step's algorithmic bytes: every weight once, every cached key and value of each row read
    (positions 0..p), the new ones written."""
    kvpp = shape.kv_bytes_per_position()
    return shape.weight_bytes() + sum(kvpp * (p + 1) for p in positions) + kvpp * len(positions)


EAGER = False  # launch dispatch by dispatch instead of the recorded graph (for profilers)


def run_decode(ctx, weights, rows: int, contexts: list, steps: int, warmup: int, profile_steps: int = 4):
    """Decode `steps` steps of `rows` requests, request r from position contexts[r]; returns the
    timing record."""
    import tgx

    capacity = int(np.ceil((max(contexts) + steps + warmup + 1) / 256.0) * 256)
    spec, shape = spec_and_shape(capacity)
    dec = tgx.Decoder(ctx, shape, tgx.Batch(rows=rows, slots=rows))
    if EAGER:
        # Every dispatch of the run launched on its own with its own events, as the per-kernel
        # timings below are taken, so a profiler's averages over the run compare with them.
        dec.set_graph(False)
        dec.set_timed(True)
    load(dec, weights)
    from tgx.synth import embeddings

    x = embeddings(7, "bench.x", rows, shape.hidden)
    # Each request's prompt, prefilled at once into its slot.
    prompt = embeddings(8, "bench.prompt", int(sum(contexts)), shape.hidden)
    dec.prefill_runs([(r, 0, int(c)) for r, c in enumerate(contexts)], prompt)
    for r, c in enumerate(contexts):
        dec.reserve(r, c + steps + warmup + 1)
    start_rows = [tgx.Row(c, r) for r, c in enumerate(contexts)]
    if warmup:
        dec.set_rows(start_rows, x)
        dec.launch(warmup, advance=True)
        dec.wait()
    dec.set_rows(start_rows, x)
    t0 = time.perf_counter()
    dec.launch(steps, advance=True)
    dec.wait()
    wall = time.perf_counter() - t0
    gpu_ms = dec.elapsed_ms()
    # Per-dispatch times from a few steps in the middle of the run.
    mid = [tgx.Row(c + steps // 2, r) for r, c in enumerate(contexts)]
    dec.set_timed(True)
    per = {}
    for k in range(profile_steps):
        dec.set_rows([tgx.Row(m.position + k, m.slot) for m in mid], x)
        dec.start()
        dec.wait()
        for label, ms in dec.timings():
            per.setdefault(label, []).append(ms)
    dec.set_timed(EAGER)
    # Through the boundary with host arrays, as a caller of tgx_decoder_step_rows steps: each
    # step's inputs copied in, the step's graph launched and waited for, its outputs copied out,
    # from the same positions (inside the reserved blocks). Beside `value`, never it.
    # The wait sleeps between polls unless the context spins first (tgx_context_set_fence_spin, as
    # decode_timing.rs:505-511 sweeps it): both, the spin at 1 ms.
    host = None
    if not EAGER:
        n_host = min(100, steps // 2)
        host = {"steps": n_host}
        for spin_us in (0, 1000):
            ctx.set_fence_spin(spin_us * 1000)
            t0 = time.perf_counter()
            for k in range(n_host):
                dec.step_rows([tgx.Row(m.position + k, m.slot) for m in mid], x)
            host_wall = time.perf_counter() - t0
            key = "" if spin_us == 0 else f"_spin_{spin_us}us"
            host["steps_per_s" + key] = n_host / host_wall
            host["ms_per_step" + key] = host_wall * 1e3 / n_host
        ctx.set_fence_spin(0)
    dec.close()
    positions_mid = [c + steps // 2 for c in contexts]
    bytes_mid = step_bytes(shape, positions_mid)
    kernels = {}
    kv_positions = sum(p + 1 for p in positions_mid)
    for label, ms in per.items():
        avg = float(np.mean(ms))
        launches_per_step = len(ms) / profile_steps
        b = kernel_bytes(shape, label, rows, kv_positions)
        kernels[label] = {
            "avg_us": avg * 1e3,
            "per_step_us": avg * 1e3 * launches_per_step,
            "bytes_per_launch": b,
            "GB_s": b / (avg * 1e-3) / 1e9 if avg > 0 else None,
        }
    ms_per_step = wall * 1e3 / steps
    return {
        "rows": rows,
        "steps": steps,
        "steps_per_s": steps / wall,
        "ms_per_step": ms_per_step,
        "gpu_ms_per_step": gpu_ms / steps,
        "step_bytes_mid": bytes_mid,
        "hbm_fraction": bytes_mid / (ms_per_step * 1e-3) / HBM_PEAK,
        "kernels": kernels,
        "kernel_sum_us": sum(k["per_step_us"] for k in kernels.values()),
        "host_boundary": host,
        "shape": shape,
    }


MFMA_PEAK = 2.5e15  # MI355X dense bf16, FLOP/s


def prefill_flops(shape, count: int, length: int) -> tuple[int, int]:
    """Linear FLOPs (2 x every weight per position, norms aside) and causal attention FLOPs
    (4 L H d (t + 1) at position t) of `count` runs of `length` positions from 0."""
    linear_params = shape.weight_bytes(1) - shape.layers * 2 * shape.hidden - shape.hidden
    linear = 2 * linear_params * count * length
    attention = 4 * shape.layers * shape.heads * shape.head_dim * count * length * (length + 1) // 2
    return linear, attention


def gemm_flops(shape, label: str, rows: int) -> int:
    h, i, H, KV, d = shape.hidden, shape.inner, shape.heads, shape.kv_heads, shape.head_dim
    n_k = {"prefill_qkv": ((H + 2 * KV) * d, h), "prefill_o": (h, H * d), "prefill_gate_up": (2 * i, h),
           "prefill_down": (h, i)}.get(label)
    return 2 * rows * n_k[0] * n_k[1] if n_k else 0


def run_prefill(ctx, weights, count: int, length: int, times: int, decode_steps: int):
    """`count` runs of `length` positions prefilled at once, then `decode_steps` decode steps."""
    import tgx
    from tgx.synth import embeddings

    capacity = int(np.ceil((length + decode_steps + 1) / 256.0) * 256)
    spec, shape = spec_and_shape(capacity)
    dec = tgx.Decoder(ctx, shape, tgx.Batch(rows=count, slots=count))
    if EAGER:
        dec.set_graph(False)
        dec.set_timed(True)
    load(dec, weights)
    x = embeddings(9, "bench.prefill", count * length, shape.hidden)
    runs = [(s, 0, length) for s in range(count)]
    out = dec.prefill_runs(runs, x)
    finite = bool(np.all(np.isfinite(out)))
    dec.prefill_launch(1)
    dec.wait()
    t0 = time.perf_counter()
    dec.prefill_launch(times)
    dec.wait()
    wall = (time.perf_counter() - t0) / times
    gpu = dec.elapsed_ms() / times * 1e-3
    dec.set_timed(True)
    dec.prefill_launch(1)
    dec.wait()
    per = {}
    for label, ms in dec.timings():
        per.setdefault(label, []).append(ms)
    dec.set_timed(EAGER)
    # The decode steps that follow, every run at once.
    xs = embeddings(10, "bench.after", count, shape.hidden)
    for r in range(count):
        dec.reserve(r, length + decode_steps + 1)
    dec.set_rows([tgx.Row(length, r) for r in range(count)], xs)
    t1 = time.perf_counter()
    dec.launch(decode_steps, advance=True)
    dec.wait()
    dwall = time.perf_counter() - t1
    # Through the boundary with host arrays (tgx_prefill_runs: the inputs copied in from pageable
    # host memory, the outputs copied back), beside the resident rate, never it; last, so that the
    # GPU's idle time during the copies precedes none of the timings above.
    host_ms = None
    if not EAGER:
        t0 = time.perf_counter()
        for _ in range(2):
            dec.prefill_runs(runs, x)
        host_ms = (time.perf_counter() - t0) / 2 * 1e3
    dec.close()
    linear, attention = prefill_flops(shape, count, length)
    kernels = {}
    rows = count * length
    for label, ms in per.items():
        avg = float(np.mean(ms))
        f = gemm_flops(shape, label, rows)
        kernels[label] = {"avg_us": avg * 1e3, "launches": len(ms), "TFLOP_s": f / (avg * 1e-3) / 1e12 if f else None,
                          "flops": f}
    return {
        "tokens_per_s": rows / wall,
        "ms": wall * 1e3,
        "gpu_ms": gpu * 1e3,
        "flops": linear + attention,
        "mfma_fraction": (linear + attention) / wall / MFMA_PEAK,
        "kernels": kernels,
        "finite": finite,
        "decode_steps_per_s": decode_steps / dwall,
        "host_ms": host_ms,
        "rows": rows,
    }


def run_tts(ctx, rows: int, steps: int, warmup: int, context: int = 128):
    """The full per-patch pipeline at `rows` requests, on the device throughout: the local encoder
    (a 4-layer stack over the patch before), the LM side (the 24-layer backbone and the 8-layer
    residual LM without RoPE, with the heads between them) and the sampler (a 4-layer LocDiT, 10
    Euler steps with CFG-Zero* guidance 2.0 over both sequences of every row) on its mu, `steps`
    patch steps, each request's caches filled to `context` positions first."""
    import tgx
    from tgx.patch import Encoder, HeadsShape, LmSide, PatchShape, PatchStep, Sampler
    from tgx.synth import StackSpec, embeddings, encoder_weights, lm_side_weights, sampler_weights

    # Positions run on through the warm-up, the timed steps and the LM side's steps alone.
    reach = context + warmup + 2 * steps + 2
    capacity = int(np.ceil(reach / 256.0) * 256)
    base = tgx.Shape(layers=24, capacity=capacity)
    residual = tgx.Shape(layers=8, capacity=capacity, rope=False)
    heads = HeadsShape(1024, 1024, 256, 9)
    patch = PatchShape(64, 4, 10, rows)
    side = LmSide(ctx, base, residual, tgx.Batch(rows=rows, slots=rows), heads)
    side.load_all(lm_side_weights(StackSpec(layers=24, seed=0), StackSpec(layers=8, seed=1), 1024, 1024, 256))
    dit = StackSpec(layers=4, seed=2)
    sampler = Sampler(ctx, tgx.Shape(layers=4, capacity=16), patch)
    sampler.load_all(sampler_weights(dit, 64))
    local = StackSpec(layers=4, seed=3)
    encoder = Encoder(ctx, tgx.Shape(layers=4, capacity=16), patch)
    encoder.load_all(encoder_weights(local, 64))
    for which in (0, 1):
        d = side.decoder(which)
        d.prefill_runs([(r, 0, context) for r in range(rows)], embeddings(12 + which, "tts.prompt", rows * context, 1024))
        for r in range(rows):
            d.reserve(r, reach)
    rng = np.random.default_rng(5)
    sampling = np.array([[1.0, 2.0]] * rows, dtype=np.float32)
    cond = rng.standard_normal((rows, 64, 4)).astype(np.float32)
    noise = rng.standard_normal((rows, 64, 4)).astype(np.float32)
    mu = np.zeros((rows, 2, 1024), dtype=np.float32)
    sampler.sample(mu, cond, noise, sampling)  # inputs in place, the graph recorded
    side.set_rows([tgx.Row(context, r) for r in range(rows)], embeddings(14, "tts.enc", rows, 1024))
    step = PatchStep(encoder, side, sampler)
    step.launch(warmup)
    step.wait()
    t0 = time.perf_counter()
    step.launch(steps)
    step.wait()
    wall = time.perf_counter() - t0
    gpu = step.elapsed_ms()
    # The parts alone, for the split.
    side.launch(steps, advance=True)
    side.wait()
    side_ms = side.elapsed_ms() / steps
    sampler.launch(steps)
    sampler.wait()
    sampler_ms = sampler.elapsed_ms() / steps
    dispatches = encoder.dispatches() + side.dispatches() + sampler.dispatches()
    step.close()
    for o in (side, sampler, encoder):
        o.close()
    # Algorithmic bytes: every weight once a step (the DiT's once per Euler evaluation).
    layer = tgx.Shape(layers=1).weight_bytes() - 2 * 1024
    dit_bytes = dit.layers * layer + 2 * 1024
    enc_bytes = local.layers * layer + 2 * 1024 + 2 * 1024 * 64
    lm_bytes = base.weight_bytes() + residual.weight_bytes()
    return {
        "workload": f"{rows} requests: 4-layer local encoder over the patch before, 24-layer backbone + 8-layer "
                    f"residual LM (no RoPE) + heads, then a 4-layer LocDiT over 4 x 64 latents, 10 Euler steps "
                    f"(9 DiT evaluations) with CFG-Zero* 2.0; contexts from {context}",
        "rows": rows,
        "steps": steps,
        "steps_per_s": steps / wall,
        "ms_per_step": wall * 1e3 / steps,
        "gpu_ms_per_step": gpu / steps,
        "lm_side_ms": side_ms,
        "sampler_ms": sampler_ms,
        "encoder_and_copies_ms": gpu / steps - side_ms - sampler_ms,
        "dispatches_per_step": dispatches + 1,
        "weight_bytes_per_step": lm_bytes + 9 * dit_bytes + enc_bytes,
    }


def host_threads() -> int:
    """The host cores the CPU baseline uses: those the process may run on, at most 16. A job on
    one GPU of an 8-GPU host has 16 of the host's CPUs to itself (OMP_NUM_THREADS 16), whatever
    os.cpu_count() reports of the whole host; more threads than that would contend with the GPU's
    own feeding thread and with each other."""
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(16, n))


def host_info() -> dict:
    """The host the CPU baseline ran on: its CPU model, the CPUs the OS reports, those this process
    may run on, and OMP_NUM_THREADS as the environment sets it."""
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except AttributeError:
        affinity = None
    return {"cpu_model": model, "nproc": os.cpu_count(), "affinity": affinity,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "threads_used": host_threads(),
            "why_16": "a one-GPU job's share of an 8-GPU host is 16 CPUs; threads stop there"}


def cpu_baseline(weights, seconds: float):
    """The fp32 CPU path (the oracle in float32, OpenMP over the host's cores) on the same
    24-layer stack at batch 1, decode steps from position 256 of a zero-filled cache."""
    import oracle
    from tgx.synth import StackSpec, embeddings

    spec = StackSpec(layers=24, dtype="bf16", seed=0)
    oracle.set_threads(host_threads())
    st = oracle.Stack(spec, weights, PROMPT + 512, "f32")
    x = embeddings(7, "bench.cpu", 1, spec.hidden)[0]
    t0 = time.perf_counter()
    st.decode(PROMPT, x)
    first = time.perf_counter() - t0
    n = max(3, min(400, int(seconds / max(first, 1e-6))))
    t0 = time.perf_counter()
    for i in range(n):
        st.decode(PROMPT + 1 + i, x)
    dt = time.perf_counter() - t0
    return {
        "value": n / dt,
        "unit": "steps/s",
        "cores": oracle.threads(),
        "host": host_info(),
        "kind": "port",
        "sample": f"{n} fp32 decode steps of the 24-layer stack at batch 1, positions {PROMPT + 1}..{PROMPT + n} "
                  f"(keys and values below {PROMPT} zero), {dt:.1f} s on {oracle.threads()} OpenMP threads",
    }


def cpu_rows(weights, seconds: float) -> dict:
    """The other rows of the CPU path beside the GPU's, each on a bounded sample of its workload
    (the oracle in float32: decode row by row in C with OpenMP, prefill layer by layer with numpy's
    float32 BLAS; the patch step with its LocDiT in numpy float64): decode steps/s at 16 and 64
    requests, prefill tok/s of one 2048-position run, patch steps/s at 16 requests."""
    import oracle
    import patch_oracle as po
    from tgx.synth import StackSpec, embeddings, encoder_weights, lm_side_weights, sampler_weights

    spec = StackSpec(layers=24, dtype="bf16", seed=0)
    oracle.set_threads(host_threads())
    out = {}
    st = oracle.Stack(spec, weights, 2048 + 64, "f32")
    for rows in (16, 64):
        ctxs = [int(c) for c in np.random.default_rng(rows).integers(64, 1025, rows)]
        x = embeddings(7, "bench.cpu", rows, spec.hidden)
        t0, n = time.perf_counter(), 0
        while n == 0 or time.perf_counter() - t0 < seconds:
            for r in range(rows):  # a step: every request once, at its own position
                st.decode(ctxs[r] + n, x[r])
            n += 1
        dt = time.perf_counter() - t0
        out[f"decode_batch{rows}"] = {"value": n / dt, "unit": "steps/s", "tokens_per_s": n * rows / dt,
                                      "sample": f"{n} steps of {rows} requests (contexts U[64,1024]), {dt:.1f} s"}
    length = 2048
    x = embeddings(9, "bench.cpu.prefill", length, spec.hidden)
    t0 = time.perf_counter()
    st.prefill_rows(0, x)
    dt = time.perf_counter() - t0
    out["prefill"] = {"value": length / dt, "unit": "tok/s",
                      "sample": f"one {length}-position run (of the 8 x 2048 workload), float32 BLAS, {dt:.1f} s"}
    # The patch step at 16 requests: the encoder over the patch before, both LMs a position on, the
    # heads, the sampler's 9 evaluations over both sequences of every request.
    rows = 16
    base, res = StackSpec(layers=24, seed=0), StackSpec(layers=8, seed=1)
    w = lm_side_weights(base, res, 1024, 1024, 256)
    dw, ew = sampler_weights(StackSpec(layers=4, seed=2), 64), encoder_weights(StackSpec(layers=4, seed=3), 64)
    lms = [oracle.Stack(s_, {k[len(p_):]: v for k, v in w.items() if k.startswith(p_)}, 256, "f32", rope=(p_ == "base_lm."))
           for s_, p_ in ((base, "base_lm."), (res, "residual_lm."))]
    shape = po.StackShape(layers=4)
    rng = np.random.default_rng(5)
    cond = rng.standard_normal((rows, 64, 4))
    noise = rng.standard_normal((rows, 64, 4))
    sampling = np.array([[1.0, 2.0]] * rows)
    t0, n = time.perf_counter(), 0
    while n == 0 or time.perf_counter() - t0 < seconds:
        emb = po.encode(ew, shape, 64, 4, cond)
        embed = po.linear(w, "enc_to_lm_proj", emb)
        base_out = np.stack([lms[0].decode(128 + n, embed[r]) for r in range(rows)])
        _, lv = po.quantizer(w, base_out, 9)
        lm_hidden, residual_in, to_dit, _, _ = po.heads_after_levels(w, lv, embed)
        res_out = np.stack([lms[1].decode(128 + n, residual_in[r]) for r in range(rows)])
        mu = np.concatenate([to_dit, po.linear(w, "res_to_dit_proj", res_out)], axis=-1).reshape(rows, 2, 1024)
        _, cond = po.sample(dw, shape, 64, 4, 10, mu, cond, noise, sampling)
        n += 1
    dt = time.perf_counter() - t0
    out["patch_step"] = {"value": n / dt, "unit": "patch steps/s",
                         "sample": f"{n} patch steps of {rows} requests (encoder, 24 + 8 layers, heads, 4-layer LocDiT "
                                   f"x 9 evaluations; LocDiT in numpy float64), {dt:.1f} s"}
    return out


COPY_BYTES = 256 << 20


def copy_calibration() -> int:
    """A plain elementwise copy (torch.neg, out=) of COPY_BYTES, five times: the kernel whose
    FETCH_SIZE and WRITE_SIZE counters are known to be COPY_BYTES each."""
    import torch

    src = torch.ones(COPY_BYTES // 4, dtype=torch.float32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(5):
        torch.neg(src, out=dst)
    torch.cuda.synchronize()
    log(f"copied {COPY_BYTES} bytes 5 times, check {float(dst[0])}")
    return 0


def sampler_profile(rows: int, samples: int) -> int:
    """The sampler alone (a 4-layer LocDiT, 10 Euler steps over 4 x 64 latents, CFG-Zero* 2.0) at
    `rows` requests, launched dispatch by dispatch with events around each (what a kernel-trace
    profiler sees), `samples` times after one to warm up: each kernel's mean time a launch."""
    import collections

    import tgx
    from tgx.patch import PatchShape, Sampler
    from tgx.synth import StackSpec, sampler_weights

    ctx = tgx.Context(0)
    s = Sampler(ctx, tgx.Shape(layers=4, capacity=16), PatchShape(64, 4, 10, rows))
    s.load_all(sampler_weights(StackSpec(layers=4, seed=2), 64))
    rng = np.random.default_rng(5)
    mu = rng.standard_normal((rows, 2, 1024)).astype(np.float32)
    cond = rng.standard_normal((rows, 64, 4)).astype(np.float32)
    noise = rng.standard_normal((rows, 64, 4)).astype(np.float32)
    sampling = np.array([[1.0, 2.0]] * rows, dtype=np.float32)
    s.set_timed(True)
    s.sample(mu, cond, noise, sampling)
    total, count = collections.defaultdict(float), collections.Counter()
    for _ in range(samples):
        s.sample(mu, cond, noise, sampling)
        for label, ms in s.timings():
            total[label] += ms
            count[label] += 1
    log(f"sampler at {rows} rows: {sum(total.values()) / samples * 1e3:.1f} us a sample of dispatch-timed kernels")
    for label in sorted(total, key=lambda k: -total[k]):
        log(f"  {label:20s} {total[label] / count[label] * 1e3:8.2f} us a launch x {count[label] // samples:3d}")
    s.close()
    ctx.close()
    return 0


def trace_figure(label: str, workload: str):
    """The committed kernel trace's average duration of `label` on `workload` (a dispatch-by-dispatch
    run under rocprofv3, whose interception lengthens a short kernel by ~0.5 us), with the file and
    commit it comes from; None when none is on record."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None
    data = json.loads(path.read_text())
    for rec in (data.get(label), data.get(workload.replace(" ", ""), {}).get(label), data.get("prefill_8x2048", {}).get(label)):
        if isinstance(rec, dict) and rec.get("workload") == workload and rec.get("trace_avg_us"):
            return {"avg_us": rec["trace_avg_us"], "file": rec.get("trace_file"), "commit": rec.get("commit")}
    return None


def measured_traffic(label: str, workload: str):
    """HBM bytes per launch of `label` measured with rocprofv3's FETCH_SIZE and WRITE_SIZE on the
    same workload, each scaled by the counter's reading of a copy of known size, and where that
    figure comes from (not this run: the record's profile file and the commit it was measured at);
    (None, None) when no measurement of this kernel on this workload is on record."""
    path = ROOT / "profiles" / "traffic.json"
    if not path.exists():
        return None, None
    data = json.loads(path.read_text())
    # Batch 1's records at the top, other workloads' under their own key ("batch64").
    for rec in (data.get(label), data.get(workload.replace(" ", ""), {}).get(label)):
        if isinstance(rec, dict) and rec.get("workload") == workload:
            source = {"measured_in_this_run": False, "file": rec.get("source"), "commit": rec.get("commit"),
                      "counters": "FETCH_SIZE x fetch_scale + WRITE_SIZE x write_scale, KiB a dispatch"}
            return rec["bytes_per_launch"], source
    return None, None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=1, help="the batch the headline value is taken at")
    ap.add_argument("--no-extra", action="store_true", help="skip the batch-16/64 runs")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-prefill", action="store_true", help="skip the 8 x 2048 prefill")
    ap.add_argument("--no-tts", action="store_true", help="skip the full per-patch pipeline at 16 requests")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a plain device copy of 256 MiB five times (scales rocprofv3's HBM counters)")
    ap.add_argument("--eager", action="store_true",
                    help="launch each step dispatch by dispatch, not as the recorded graph (for profilers)")
    ap.add_argument("--sampler", action="store_true",
                    help="only the sampler at --batch rows, dispatch by dispatch, --steps samples (for profilers)")
    args = ap.parse_args()
    global EAGER
    EAGER = args.eager
    if args.copy_calibration:
        return copy_calibration()
    if args.sampler:
        return sampler_profile(args.batch, args.steps)
    if args.gpus != 1:
        print("bench.py runs on one GPU: tgx has no multi-GPU path (requests would be routed to GPUs "
              "at admission, with no collective); run with --gpus 1.", file=sys.stderr)
        return 2

    import tgx
    from tgx.synth import StackSpec, stack_weights

    t0 = time.perf_counter()
    weights = stack_weights(StackSpec(layers=24, dtype="bf16", seed=0))
    log(f"weights drawn in {time.perf_counter() - t0:.1f} s")
    ctx = tgx.Context(0)
    report = ctx.report()
    log(f"device {report['name']} {report['arch']} {report['compute_units']} CUs {report['clock_khz']} kHz")

    rng = np.random.default_rng(1234)
    headline_contexts = [PROMPT] * args.batch if args.batch == 1 else [int(c) for c in np.random.default_rng(args.batch).integers(64, 1025, args.batch)]
    head = run_decode(ctx, weights, args.batch, headline_contexts, args.steps, args.warmup)
    shape = head.pop("shape")
    log(f"batch {args.batch}: {head['steps_per_s']:.1f} steps/s, {head['ms_per_step']*1e3:.1f} us/step, "
        f"kernels sum {head['kernel_sum_us']:.1f} us")
    if head["host_boundary"]:
        log(f"batch {args.batch} through host arrays: {head['host_boundary']['steps_per_s']:.1f} steps/s, "
            f"{head['host_boundary']['steps_per_s_spin_1000us']:.1f} with the wait spinning")
    for label, k in sorted(head["kernels"].items(), key=lambda kv: -kv[1]["per_step_us"]):
        log(f"  {label:16s} {k['avg_us']:8.2f} us/launch {k['per_step_us']:8.1f} us/step {k['GB_s'] or 0:8.1f} GB/s")

    batches = {}
    if not args.no_extra:
        for rows in (16, 64):
            if rows == args.batch:
                continue
            ctxs = [int(c) for c in np.random.default_rng(rows).integers(64, 1025, rows)]
            r = run_decode(ctx, weights, rows, ctxs, 200, 10)
            r.pop("shape")
            for label, k in sorted(r["kernels"].items(), key=lambda kv: -kv[1]["per_step_us"]):
                log(f"  [{rows:2d}] {label:16s} {k['avg_us']:8.2f} us/launch {k['per_step_us']:8.1f} us/step {k['GB_s'] or 0:8.1f} GB/s")
            batches[str(rows)] = {k: r[k] for k in ("steps_per_s", "ms_per_step", "hbm_fraction", "kernel_sum_us", "step_bytes_mid", "host_boundary")}
            batches[str(rows)]["kernels_us"] = {k: round(v["avg_us"], 3) for k, v in r["kernels"].items()}
            batches[str(rows)]["tokens_per_s"] = r["steps_per_s"] * rows
            batches[str(rows)]["contexts"] = "U[64,1024] seeded, 200 steps"
            log(f"batch {rows}: {r['steps_per_s']:.1f} steps/s ({r['steps_per_s']*rows:.0f} tok/s), "
                f"{r['hbm_fraction']*100:.1f}% of HBM peak on algorithmic bytes"
                + (f"; through host arrays {r['host_boundary']['steps_per_s']:.1f} steps/s, "
                   f"{r['host_boundary']['steps_per_s_spin_1000us']:.1f} spinning" if r["host_boundary"] else ""))

    prefill = None
    if not args.no_prefill:
        pf = run_prefill(ctx, weights, 8, 2048, 3, 32)
        for label, k in sorted(pf["kernels"].items(), key=lambda kv: -kv[1]["avg_us"] * kv[1]["launches"]):
            log(f"  [prefill] {label:18s} {k['avg_us']:10.1f} us x {k['launches']:3d}"
                + (f"  {k['TFLOP_s']:8.1f} TFLOP/s" if k["TFLOP_s"] else ""))
        log(f"prefill 8 x 2048: {pf['tokens_per_s']:.0f} tok/s, {pf['ms']:.2f} ms, "
            f"{pf['mfma_fraction'] * 100:.1f}% of bf16 MFMA peak; then {pf['decode_steps_per_s']:.0f} steps/s at batch 8"
            + (f"; through host arrays {pf['host_ms']:.2f} ms" if pf["host_ms"] else ""))
        gemms = {k: v for k, v in pf["kernels"].items() if v["TFLOP_s"]}
        dom = max(gemms.items(), key=lambda kv: kv[1]["avg_us"] * kv[1]["launches"])
        prefill = {
            "workload": "8 runs x 2048 positions, causal, 24 layers, bf16; then 32 decode steps at batch 8",
            "tokens_per_s": round(pf["tokens_per_s"], 1),
            "ms": round(pf["ms"], 3),
            "flops": pf["flops"],
            "mfma_fraction": round(pf["mfma_fraction"], 4),
            "finite": pf["finite"],
            "decode_steps_per_s_after": round(pf["decode_steps_per_s"], 1),
            # tgx_prefill_runs with the inputs and outputs in (pageable) host memory.
            "host_boundary": None if pf["host_ms"] is None else
                {"ms": round(pf["host_ms"], 3), "tokens_per_s": round(pf["rows"] / (pf["host_ms"] * 1e-3), 1)},
            "roofline": {"bound": "mfma", "kernel": dom[0], "achieved": round(dom[1]["TFLOP_s"], 1),
                         "peak": MFMA_PEAK / 1e12, "unit": "TFLOP/s", "frac": round(dom[1]["TFLOP_s"] * 1e12 / MFMA_PEAK, 4),
                         "avg_us": round(dom[1]["avg_us"], 2),
                         "trace": trace_figure(dom[0], "8 x 2048 prefill")},
            "kernels_us": {k: round(v["avg_us"], 2) for k, v in pf["kernels"].items()},
        }

    tts = None
    if not args.no_tts:
        tts = run_tts(ctx, 16, 30, 3)
        log(f"tts step at 16 requests: {tts['steps_per_s']:.1f} patch steps/s ({tts['ms_per_step']:.2f} ms; LM side "
            f"{tts['lm_side_ms']:.2f} ms, sampler {tts['sampler_ms']:.2f} ms, encoder and copies "
            f"{tts['encoder_and_copies_ms']:.2f} ms)")
        tts = {k: (round(v, 4) if isinstance(v, float) else v) for k, v in tts.items()}

    # The roofline of the step's dominant kernel for HBM: the one whose launches move the most
    # algorithmic bytes per step; beside it, the kernel with the most time per step.
    def kernel_roofline(label, k):
        achieved = k["bytes_per_launch"] / (k["avg_us"] * 1e-6) / 1e9
        traffic, traffic_source = measured_traffic(label, f"batch {args.batch}")
        return {
            "bound": "hbm",
            "kernel": label,
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK / 1e9,
            "unit": "GB/s",
            "frac": round(achieved / (HBM_PEAK / 1e9), 4),
            "traffic": traffic,
            "traffic_source": traffic_source,
            "bytes_per_launch": k["bytes_per_launch"],
            "avg_us": round(k["avg_us"], 3),
            "trace": trace_figure(label, f"batch {args.batch}"),
            "of_stream_floor": round(achieved / floor_kernel["GB_s"], 4),
        }

    # The stream-read floor (stream_read.comp, as decode_timing.rs:430-441 reports it): the step's
    # weight bytes read once by a kernel that does nothing else, at its best of 20 launches; and
    # one gate/up projection's bytes, the size of the step's largest kernel.
    floor = ctx.stream_read(shape.weight_bytes(), 20)
    floor_kernel = ctx.stream_read(kernel_bytes(shape, "gemv_gate_up", args.batch, 0), 50)
    log(f"stream-read floor: {floor['GB_s']:.0f} GB/s over {floor['bytes']} bytes, "
        f"{floor_kernel['GB_s']:.0f} GB/s over {floor_kernel['bytes']} bytes ({floor_kernel['best_ms'] * 1e3:.2f} us)")

    kernels = head["kernels"]
    by_bytes = max(kernels.items(), key=lambda kv: kv[1]["bytes_per_launch"] * kv[1]["per_step_us"] / kv[1]["avg_us"])
    by_time = max(kernels.items(), key=lambda kv: kv[1]["per_step_us"])
    roofline = kernel_roofline(*by_bytes)
    roofline_longest = kernel_roofline(*by_time)

    cpu = None
    if not args.no_cpu:
        try:
            cpu = cpu_baseline(weights, args.cpu_seconds)
            log(f"cpu baseline: {cpu['value']:.2f} steps/s on {cpu['cores']} threads")
            cpu["rows"] = cpu_rows(weights, args.cpu_seconds / 2)
            for name, r in cpu["rows"].items():
                log(f"cpu baseline {name}: {r['value']:.3f} {r['unit']} ({r['sample']})")
        except Exception as e:  # the baseline is reported, never required
            log(f"cpu baseline failed: {e}")

    line = {
        "metric": METRIC,
        "value": round(head["steps_per_s"], 2),
        "unit": "steps/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,0.02) bf16 weights, N(0,1) inputs)",
        "config": {
            "workload": f"MiniCPM-4 backbone decode: 24 layers, hidden 1024, 16/2 GQA heads, head_dim 64, "
                        f"FFN 4096, bf16 weights; batch {args.batch}, from position {PROMPT} "
                        f"({'256-position prompt' if args.batch == 1 else 'contexts U[64,1024]'}), "
                        f"{args.steps} decode steps, paged KV cache (64-position blocks)",
            "batch": args.batch,
            "layers": 24,
            "hidden": 1024,
            "kernels_per_step": 121,
        },
        "hbm_fraction_step": round(head["hbm_fraction"], 4),
        "stream_read_floor": {"GB_s": round(floor["GB_s"], 1), "bytes": floor["bytes"], "best_ms": round(floor["best_ms"], 4),
                              "kernel_size_GB_s": round(floor_kernel["GB_s"], 1), "kernel_size_bytes": floor_kernel["bytes"],
                              "step_at_floor_ms": round(step_bytes(shape, [c + args.steps // 2 for c in headline_contexts]) / (floor["GB_s"] * 1e9) * 1e3, 4)},
        "gpu_ms_per_step": round(head["gpu_ms_per_step"], 4),
        # Steps through tgx_decoder_step_rows with host arrays (PCIe copies and a wait each step).
        "host_boundary": head["host_boundary"],
        "roofline": roofline,
        "roofline_longest": roofline_longest,
        "cpu_baseline": cpu,
        "batches": batches,
        "prefill": prefill,
        "tts_step": tts,
        "kernels_us": {k: round(v["avg_us"], 3) for k, v in head["kernels"].items()},
        "device": {"name": report["name"], "arch": report["arch"], "clock_khz": report["clock_khz"]},
    }
    print(json.dumps(line), flush=True)
    ctx.close()
    return 0


if __name__ == "__main__":
    sys.exit(main())
