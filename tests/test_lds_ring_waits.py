"""The waits of the kernels that stage operands through LDS by direct global-to-LDS loads
(prefill_gemm, prefill_attention, local_gemm_ring), checked on the compiler's own AMD assembly for
gfx950 by a replay of one workgroup's waves (tests/lds_replay.py): each kernel counts its loads in
issue order (s_waitcnt vmcnt(N)) and reads LDS through inline asm the compiler does not order
behind those loads, so the count is right only while the loads go out in the order the source
assumes. A compiler that reorders them (as it did the local ring's prelude before its scheduling
barriers) lets a wave read a slot one load early, which gives finite wrong values most of the time
(the batch-invariance contract of crates/graph/src/decode.rs:8-11 must hold on cold caches too).

Every instance the library builds is compiled here with the library's own flags
(tgtts-v4_amd/build_lib.py), its argument structs' layouts read from clang's record-layout dump,
and one or two workgroups replayed on arguments of the shapes the library launches (the backbone's
and VoxCPM2's widths, ragged position counts), with the uniform branches whose conditions depend
on data taken both ways. No LDS access may meet a load into its bytes still in flight. The local
ring with its prelude as it was before its scheduling barriers is a planted defect the check must
catch. Nothing here runs on a GPU."""

import re
import shutil
import struct
import subprocess
from functools import lru_cache
from pathlib import Path

import pytest

import lds_replay as lr

ROOT = Path(__file__).resolve().parent.parent
CSRC = ROOT / "tgtts-v4_amd" / "csrc"
HIPCC = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"

pytestmark = pytest.mark.skipif(not Path(HIPCC).exists(), reason="hipcc is needed to build the kernels' assembly")


def f32(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", x))[0]


def device_flags(source: str) -> list:
    import build_lib

    return [f for f in build_lib.SOURCES[source] if f != "-fPIC"]


@lru_cache(maxsize=None)
def assembly(source: str, text: str | None = None, tmp: str | None = None) -> dict:
    """The kernels of `source` (or of `text` in its place) as the library builds them, parsed."""
    path = CSRC / source
    if text is not None:
        path = Path(tmp) / source
        path.write_text(text)
    out = Path(tmp or "/tmp") / (source + ".replay.s")
    cmd = [HIPCC, *device_flags(source), "--cuda-device-only", "-S", "-I", str(CSRC), "-I", str(ROOT / "include"), str(path),
           "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return lr.parse(out.read_text())


@lru_cache(maxsize=None)
def layout(source: str) -> dict:
    cmd = [HIPCC, "-x", "hip", "--cuda-host-only", "-fsyntax-only", "-std=c++17", "-Xclang", "-fdump-record-layouts",
           "-I", str(CSRC), "-I", str(ROOT / "include"), str(CSRC / source)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr[-2000:]
    return lr.layouts(r.stdout)


def template_args(symbol: str) -> list:
    """The integer template arguments of a mangled kernel name, in order."""
    return [int(x) for x in re.findall(r"Li(\d+)E", symbol)]


def instances(kernels: dict, stem: str) -> list:
    return sorted(k for k in kernels if re.search(rf"\d{stem}I", k))


# Addresses of the buffers the kernels only stream (their contents never steer a branch) and of
# those whose contents the replay is given.
W, X, OUT, AUX, Q, KV, ATT, TILES, POS, SLOT, TABLE, COS, SIN = (0x1000000000 * (i + 1) for i in range(13))


def replay(kernel, explicit, grid, threads, memory, wgs):
    ka = lr.kernarg(kernel, explicit, grid=grid, block=(threads, 1, 1))
    runs = []
    for wg in wgs:
        r = lr.Replay(kernel, ka, memory, wg=wg, threads=threads, unknown_branch="fall").run()
        runs.append((wg, "fall", r))
        if r.unknown_branches:  # a uniform branch on data the replay does not know: the other way too
            runs.append((wg, "take", lr.Replay(kernel, ka, memory, wg=wg, threads=threads, unknown_branch="take").run()))
    return runs


def check(runs, name):
    for wg, policy, r in runs:
        s = r.summary()
        assert s["loads_into_lds"] > 0 and s["lds_accesses"] > 0, (name, wg, policy, s)
        hz = r.hazards()
        assert not hz, f"{name} workgroup {wg} ({policy} on unknown branches), {s}: {len(hz)} hazards, e.g. {hz[:3]}"
    print(f"{name}: {runs[0][2].summary()}", flush=True)


# ---- the prefill GEMM ----

GEMM_EPI = {0: "qkv", 1: "residual", 2: "silu", 3: "residual_in"}


def prefill_args(L, M, M_pad, hidden, inner, heads, kv_heads, head_dim, capacity, max_blocks, nblocks, nslots=1):
    return lr.pack(L, "PrefillArgs", dict(M=M, M_pad=M_pad, hidden=hidden, inner=inner, heads=heads, kv_heads=kv_heads,
                                          head_dim=head_dim, capacity=capacity, nslots=nslots, max_blocks=max_blocks,
                                          nblocks=nblocks, eps=f32(1e-5), scale=f32(head_dim ** -0.5), rope=1, tok_pos=POS,
                                          tok_slot=SLOT, table=TABLE, cos=COS, sin=SIN))


def rows_memory(M, M_pad, max_blocks, nslots=1):
    spare = 0xFFFFFFFF
    pos = b"".join(struct.pack("<I", m if m < M else spare) for m in range(M_pad))
    slot = b"".join(struct.pack("<I", 0 if m < M else spare) for m in range(M_pad))
    table = b"".join(struct.pack("<I", i) for i in range(nslots * max_blocks))
    return {POS: pos, SLOT: slot, TABLE: table}


def test_prefill_gemm_reads_no_stage_before_it_lands():
    symbols = instances(assembly("prefill_kernels.hip"), "prefill_gemm")
    assert len(symbols) >= 7, symbols  # q/k/v at both head widths, o and down at both strip heights, gate/up
    for symbol in symbols:
        prefill_gemm_case(symbol)


def prefill_gemm_case(symbol):
    epi, wr, tm, d = template_args(symbol)
    k = assembly("prefill_kernels.hip")[symbol]
    L = layout("prefill_kernels.hip")
    hidden, inner = (1024, 4096) if d == 64 else (2048, 6144)
    heads, kv = 16, 2
    M, M_pad = 200, 256
    K, N = {0: (hidden, (heads + 2 * kv) * d), 1: (inner, hidden), 2: (hidden, 2 * inner), 3: (heads * d, hidden)}[epi]
    # The main loop is the same code at every K (a multiple of 1024, the stages taken in pairs): K
    # 1024, its 32 stages, runs its prologue, steady state and tail as the longer K's do.
    K = 1024
    for scaled in (False, True):
        g = dict(w=W, x=X, K=K, N=N, residual=0, out=0, mlp=0, q=0, kv=0, row_sq=0, next_gain=0, out_n=0, out_sq=0)
        if epi == 0:
            g.update(q=Q, kv=KV, row_sq=AUX if scaled else 0)
        elif epi == 2:
            g.update(mlp=OUT, row_sq=AUX if scaled else 0)
        else:
            g.update(residual=AUX, out=OUT, next_gain=AUX + 0x100000 if scaled else 0, out_n=OUT + 0x1000000,
                     out_sq=OUT + 0x2000000)
        a = prefill_args(L, M, M_pad, hidden, inner, heads, kv, d, 512, 8, 8)
        grid = (N // 256, M_pad // tm, 1)
        last = (grid[0] - 1, grid[1] - 1, 0)
        runs = replay(k, [a, lr.pack(L, "GemmArgs", g)], grid, tm * 2, rows_memory(M, M_pad, 8), [(0, 0, 0), last])
        check(runs, f"prefill_gemm<{GEMM_EPI[epi]}, {wr}, {tm}, {d}> K {K} N {N}{' scaled' if scaled else ''}")


# ---- the prefill attention ----


def test_prefill_attention_reads_no_chunk_before_it_lands():
    symbols = instances(assembly("prefill_kernels.hip"), "prefill_attention")
    assert len(symbols) == 14, symbols  # column groups of 16, 8, 5, 4, 3, 2, 1 positions at head widths 64 and 128
    for symbol in symbols:
        prefill_attention_case(symbol)


def prefill_attention_case(symbol):
    tile, waves, cg, d = template_args(symbol)
    group = 16 // (tile // waves // cg)
    k = assembly("prefill_kernels.hip")[symbol]
    L = layout("prefill_kernels.hip")
    heads, kv = 16, 16 // group
    hidden, inner = (1024, 4096) if d == 64 else (2048, 6144)
    max_blocks = 16
    # Tiles: the run's first (every chunk masked: the first steps' path), one well inside a long
    # run (the unmasked phase, the ring turning several times), and a ragged last one.
    tiles = [(0, 0, tile, 0), (tile, 333, tile, 0), (2 * tile, 700, tile - 5, 0)]
    mem = rows_memory(3 * tile, 256, max_blocks)
    mem[TILES] = b"".join(struct.pack("<4I", *t) for t in tiles)
    a = prefill_args(L, 3 * tile, 256, hidden, inner, heads, kv, d, 1024, max_blocks, max_blocks)
    explicit = [a, struct.pack("<Q", Q), struct.pack("<Q", KV), struct.pack("<Q", ATT), struct.pack("<Q", TILES)]
    # Workgroup kv t + h takes tile t for KV head h: each tile for the last head.
    runs = replay(k, explicit, (len(tiles) * kv, 1, 1), waves * 64, mem, [(i * kv + kv - 1, 0, 0) for i in range(len(tiles))])
    check(runs, f"prefill_attention<{tile}, {waves}, {cg}, {d}> (group {group})")


# ---- the local stack's ring GEMM ----

LOCAL_EPI = {0: "qkv", 1: "partial", 2: "silu", 3: "add"}


def local_ring_runs(kernels, symbol):
    epi, sw, kbp, parts, tt = template_args(symbol)
    k = kernels[symbol]
    L = layout("local_kernels.hip")
    M, M_pad = 352, 384  # the 16-request sampler: 2 x 16 sequences of 11 tokens
    K = kbp * parts * 32
    N = {0: 1280, 2: 8192, 3: 1024}[epi]
    a = lr.pack(L, "LocalArgs", dict(M=M, M_pad=M_pad, T=11, hidden=1024, inner=4096, heads=16, kv_heads=2, eps=f32(1e-5),
                                     scale=f32(0.125), rope=1, cos=COS, sin=SIN))
    g = dict(w=W, x=X, K=K, N=N, partial=0, mlp=0, q=0, k=0, v=0, row_sq=0, residual=0, sum=0, next_gain=0, normed=0, sum_sq=0)
    if epi == 0:
        g.update(q=Q, k=Q + 0x1000000, v=Q + 0x2000000, row_sq=AUX)
    elif epi == 2:
        g.update(mlp=OUT, row_sq=AUX)
    else:
        g.update(residual=AUX, sum=OUT, next_gain=AUX + 0x100000, normed=OUT + 0x1000000, sum_sq=OUT + 0x2000000)
    units = N // 16 // sw
    grid = (N // 64, M_pad // 64, 1) if epi == 3 else (units // 4, M_pad // (16 * tt), 1)
    last = (grid[0] - 1, grid[1] - 1, 0)
    return replay(k, [a, lr.pack(L, "LocalGemm", g)], grid, 256, {}, [(0, 0, 0), last]), (epi, sw, kbp, parts, tt, K, N)


def test_local_ring_reads_no_slot_before_it_lands():
    kernels = assembly("local_kernels.hip")
    symbols = instances(kernels, "local_gemm_ring")
    assert len(symbols) >= 6, symbols
    for symbol in symbols:
        runs, (epi, sw, kbp, parts, tt, K, N) = local_ring_runs(kernels, symbol)
        check(runs, f"local_gemm_ring<{LOCAL_EPI[epi]}, {sw}, {kbp}, {parts}, {tt}> K {K} N {N}")


def test_the_local_rings_prelude_without_its_scheduling_barriers_is_caught(tmp_path):
    """Planted defect: the prelude as it was before its scheduling barriers (every group's loads
    issued in one stretch, which the compiler reorders), which let the first waits pass a slot's
    load still in flight: the check must report it."""
    text = (CSRC / "local_kernels.hip").read_text()
    fixed = """    all_issued();
#pragma unroll
    for (int kb = 0; kb < RING; ++kb) {
        fetch(kb);
        all_issued();
    }"""
    assert fixed in text, "the ring's prelude changed: plant the defect in its new form"
    planted = text.replace(fixed, """#pragma unroll
    for (int kb = 0; kb < RING; ++kb) fetch(kb);
    all_issued();""")
    kernels = assembly("local_kernels.hip", planted, str(tmp_path))
    caught = 0
    for symbol in instances(kernels, "local_gemm_ring"):
        runs, _ = local_ring_runs(kernels, symbol)
        hz = runs[0][2].hazards()
        caught += bool(hz)
        if hz:
            print(f"planted: {symbol}: {len(hz)} hazards, e.g. {hz[0]}", flush=True)
    assert caught > 0, "the planted prelude passed the check"


def test_a_last_step_reading_the_buffer_its_prefetch_writes_is_caught(tmp_path):
    """Planted defect: the prefill GEMM's last step reading (for fragments never used) the buffer
    of its own stage, into which the same step's prefetch of the last stage again is loading, as
    the ring once did. The read and the load meet between the same two barriers: the check must
    report it for the q/k/v GEMM."""
    text = (CSRC / "prefill_kernels.hip").read_text()
    fixed = "read(st + 1, next);  // its buffer: (st + 1) % NBUF"
    assert fixed in text, "the GEMM's step changed: plant the defect in its new form"
    kernels = assembly("prefill_kernels.hip", text.replace(fixed, "read(min(st + 1, stages - 1), next);"), str(tmp_path))
    symbol = next(s for s in instances(kernels, "prefill_gemm") if template_args(s) == [0, 16, 128, 64])
    L = layout("prefill_kernels.hip")
    g = dict(w=W, x=X, K=1024, N=1280, residual=0, out=0, mlp=0, q=Q, kv=KV, row_sq=0, next_gain=0, out_n=0, out_sq=0)
    a = prefill_args(L, 200, 256, 1024, 4096, 16, 2, 64, 512, 8, 8)
    runs = replay(kernels[symbol], [a, lr.pack(L, "GemmArgs", g)], (5, 2, 1), 256, rows_memory(200, 256, 8), [(0, 0, 0)])
    hz = runs[0][2].hazards()
    print(f"planted: {len(hz)} hazards, e.g. {hz[:1]}", flush=True)
    assert any("between barriers" in h for h in hz)
