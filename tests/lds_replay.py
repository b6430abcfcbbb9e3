"""A replay of a workgroup's waves over the compiler's AMD assembly for gfx950, to check the waits
that kernels staging operands through LDS by direct global-to-LDS loads (global_load_lds) make
by hand: such a kernel reads LDS through inline-asm ds_read, which the compiler does not order
behind those loads, and waits with s_waitcnt vmcnt(N) counts it chose, which hold only while the
loads go out in the order the source assumes.

The replay runs every wave of one workgroup instruction by instruction on concrete kernel
arguments: scalar registers and the vector registers' 64 lanes with their integer operations
exact (floating-point and matrix results are unknown, as is anything loaded from memory the
caller did not describe), branches followed, the exec mask kept, s_barrier as a meeting of the
waves. Each wave keeps its vector memory operations in issue order; s_waitcnt vmcnt(N) retires
the oldest until N are left, as gfx950's one vector memory counter does for loads and stores
alike. Every direct-to-LDS load is recorded with the LDS bytes it writes (M0 + 16 bytes a lane)
and every LDS access with the bytes its lanes reach, and `hazards` reports an access that a load
into the same bytes could still be in flight for:

- the wave's own load issued before the access and not yet retired by its waits;
- another wave's load issued before the barrier the access follows, and not retired before that
  wave reached that barrier;
- another wave's load issued between the same two barriers as the access (unordered with it).

It also reports a wave that ends with a direct-to-LDS load in flight. This is test
infrastructure: nothing in the library imports it.
"""

from __future__ import annotations

import re
from dataclasses import dataclass, field
from functools import lru_cache

import numpy as np
import yaml

M32 = 0xFFFFFFFF
M64 = (1 << 64) - 1
LANES = 64
LDS_BYTES = 160 * 1024  # a gfx950 workgroup's LDS
ALL = np.ones(LANES, dtype=bool)
NONE = np.zeros(LANES, dtype=bool)


class ReplayError(Exception):
    """The replay met something it cannot follow (an unknown branch past its budget, an LDS
    address it cannot resolve, an instruction form it does not model where it matters)."""


# ---- the assembly ----------------------------------------------------------------------------


@dataclass
class Kernel:
    name: str
    code: list  # (mnemonic, operands, modifiers, source line)
    labels: dict
    desc: dict
    meta: dict


_INLINE_F32 = {"0.5": 0x3F000000, "-0.5": 0xBF000000, "1.0": 0x3F800000, "-1.0": 0xBF800000, "2.0": 0x40000000,
               "-2.0": 0xC0000000, "4.0": 0x40800000, "-4.0": 0xC0800000, "0.15915494": 0x3E22F983}


def _split_operands(rest: str):
    """Operands (comma-separated) and the modifiers after them (offset:N, sc0, bitop3:0xNN ...)."""
    rest = rest.split(";", 1)[0].strip()
    if not rest:
        return [], {}
    parts = [p.strip() for p in rest.split(",")]
    mods = {}
    last = parts[-1].split()
    parts[-1] = last[0]
    for m in last[1:]:
        k, _, v = m.partition(":")
        mods[k] = v
    # A modifier may also follow an operand before the last (never with the forms modelled here).
    return parts, mods


def parse(asm: str) -> dict:
    """Every kernel of an assembly listing, by symbol."""
    meta = {}
    m = re.search(r"\.amdgpu_metadata\n(.*?)\.end_amdgpu_metadata", asm, re.S)
    if m:
        text = m.group(1)
        end = text.find("\n...")
        doc = yaml.safe_load(text[: end if end >= 0 else len(text)])
        for k in doc.get("amdhsa.kernels", []):
            meta[k[".name"]] = k
    kernels = {}
    for m in re.finditer(r"\.amdhsa_kernel (\S+)\n(.*?)\.end_amdhsa_kernel", asm, re.S):
        desc = {}
        for line in m.group(2).split("\n"):
            f = line.split()
            if len(f) == 2 and f[0].startswith(".amdhsa_"):
                desc[f[0][8:]] = int(f[1], 0)
        kernels[m.group(1)] = desc
    out = {}
    lines = asm.split("\n")
    i = 0
    while i < len(lines):
        m = re.match(r"^(_Z\S+):", lines[i])
        if not m or m.group(1) not in kernels:
            i += 1
            continue
        name = m.group(1)
        code, labels = [], {}
        i += 1
        while i < len(lines) and not lines[i].startswith(".Lfunc_end"):
            line = lines[i]
            lm = re.match(r"^(\.L\w+):", line)
            if lm:
                labels[lm.group(1)] = len(code)
            elif line.startswith("\t") and not line.startswith("\t.") and not line.lstrip().startswith(";"):
                text = line.strip()
                mn, _, rest = text.partition(" ")
                ops, mods = _split_operands(rest)
                code.append((mn, ops, mods, text))
            i += 1
        out[name] = Kernel(name, code, labels, kernels[name], meta.get(name, {}))
    return out


# ---- values --------------------------------------------------------------------------------------
# A scalar is (value, known bits); a vector is (values [64] uint64 holding 32 or 64 bits, known
# [64] bool).


@lru_cache(maxsize=None)
def _reg(op: str):
    """('s'|'v'|'a', first, count) for a register operand, else None."""
    m = re.fullmatch(r"([sva])(\d+)", op)
    if m:
        return m.group(1), int(m.group(2)), 1
    m = re.fullmatch(r"([sva])\[(\d+):(\d+)\]", op)
    if m:
        return m.group(1), int(m.group(2)), int(m.group(3)) - int(m.group(2)) + 1
    return None


_FLOAT_OPS = {"cvt_f32_u32", "cvt_f32_i32", "cvt_u32_f32", "cvt_i32_f32", "rcp_iflag_f32", "rcp_f32", "trunc_f32",
              "floor_f32", "mul_f32", "add_f32", "sub_f32", "subrev_f32", "max_f32", "min_f32", "fma_f32", "fmac_f32",
              "mac_f32"}


def _modified(op: str) -> bool:
    """An operand with a negation or absolute-value modifier (not a negative literal)."""
    return op.startswith("|") or re.match(r"-\|?[vsa]", op) is not None


def _literal(op: str):
    if op in _INLINE_F32:
        return _INLINE_F32[op]
    try:
        return int(op, 0) & M64
    except ValueError:
        return None


@dataclass
class Access:
    wave: int
    epoch: int
    pos: int
    lo: int
    hi: int
    what: str


@dataclass
class Dma:
    wave: int
    epoch: int
    pos: int
    lo: int
    hi: int
    what: str
    retired_epoch: int | None = None
    retired_pos: int | None = None


@dataclass
class Wave:
    index: int
    s: list = field(default_factory=lambda: [(0, 0)] * 128)
    v: np.ndarray = field(default_factory=lambda: np.zeros((1024, LANES), dtype=np.uint64))
    vk: np.ndarray = field(default_factory=lambda: np.zeros((1024, LANES), dtype=bool))
    special: dict = field(default_factory=dict)
    scc: tuple = (0, False)
    pc: int = 0
    pos: int = 0
    done: bool = False
    at_barrier: bool = False
    queue: list = field(default_factory=list)  # in flight: Dma or None (another vector memory operation)


class Replay:
    """One workgroup of `kernel` at workgroup id `wg` with `threads` threads: `kernarg` the argument
    bytes, `memory` {address: bytes} the buffers whose contents the kernel may branch on.
    `unknown_branch` chooses a uniform branch whose condition is not known: "fall" or "take"."""

    def __init__(self, kernel: Kernel, kernarg: bytes, memory: dict, wg=(0, 0, 0), threads=256,
                 unknown_branch="fall", budget=4_000_000, grid=(1, 1, 1)):
        self.k = kernel
        self.kernarg_at = 0x7F0000000000
        self.memory = dict(memory)
        self.memory[self.kernarg_at] = bytes(kernarg)
        self.unknown_branch = unknown_branch
        self.budget = budget
        self.epoch = 0
        self.dmas: list[Dma] = []
        self.accesses: list[Access] = []
        self.ended_in_flight: list[str] = []
        self.unknown_branches = 0
        self.steps = 0
        self._exec_memo = {}
        # LDS contents: what ds writes store is known, what direct-to-LDS loads bring is not.
        self.lds = np.zeros(LDS_BYTES + 64, dtype=np.uint8)
        self.lds_known = np.zeros(LDS_BYTES + 64, dtype=bool)
        self.unresolved_accesses = 0
        self.waves = [self._wave(w, wg, threads) for w in range((threads + LANES - 1) // LANES)]

    # -- state --

    def _wave(self, w, wg, threads):
        d = self.k.desc
        wave = Wave(w)
        n = 0
        for flag, size in (("user_sgpr_private_segment_buffer", 4), ("user_sgpr_dispatch_ptr", 2), ("user_sgpr_queue_ptr", 2)):
            if d.get(flag):
                for j in range(size):
                    wave.s[n + j] = (0, 0)
                n += size
        if d.get("user_sgpr_kernarg_segment_ptr"):
            wave.s[n] = (self.kernarg_at & M32, M32)
            wave.s[n + 1] = (self.kernarg_at >> 32, M32)
            n += 2
        if d.get("user_sgpr_kernarg_preload_length"):
            raise ReplayError("kernel arguments preloaded into SGPRs")
        n = d.get("user_sgpr_count", n)
        for axis, flag in enumerate(("system_sgpr_workgroup_id_x", "system_sgpr_workgroup_id_y", "system_sgpr_workgroup_id_z")):
            if d.get(flag):
                wave.s[n] = (wg[axis], M32)
                n += 1
        if d.get("system_vgpr_workitem_id", 0) != 0:
            raise ReplayError("workitem ids past x")
        tid = np.arange(LANES, dtype=np.uint64) + LANES * w
        wave.v[0] = tid
        wave.vk[0] = True
        live = min(LANES, threads - LANES * w)
        ex = (1 << live) - 1
        wave.special["exec"] = (ex, M64)
        wave.special["vcc"] = (0, 0)
        wave.special["m0"] = (0, 0)
        return wave

    # scalar registers

    def _sget(self, wv: Wave, op: str, width=32):
        """(value, known bits) of a scalar operand of 32 or 64 bits."""
        r = _reg(op)
        if r and r[0] == "s":
            lo = wv.s[r[1]]
            if width == 64 or r[2] == 2:
                hi = wv.s[r[1] + 1]
                return (lo[0] | hi[0] << 32, lo[1] | hi[1] << 32)
            return lo
        if op in ("vcc", "exec"):
            val, kn = wv.special[op]
            return (val, kn) if width == 64 else (val & M32, kn & M32)
        if op in ("vcc_lo", "exec_lo"):
            val, kn = wv.special[op[:-3]]
            return (val & M32, kn & M32)
        if op in ("vcc_hi", "exec_hi"):
            val, kn = wv.special[op[:-3]]
            return (val >> 32, kn >> 32)
        if op == "m0":
            return wv.special["m0"]
        if op == "scc":
            return (int(wv.scc[0]), 1 if wv.scc[1] else 0)
        lit = _literal(op)
        if lit is not None:
            if width == 32:
                return (lit & M32, M32)
            if lit >> 32 == 0 and op.startswith("-"):
                lit |= 0xFFFFFFFF00000000
            return (lit & M64, M64)
        return (0, 0)

    def _sset(self, wv: Wave, op: str, val: int, kn: int, width=32):
        r = _reg(op)
        if r and r[0] == "s":
            wv.s[r[1]] = (val & M32, kn & M32)
            if width == 64 or r[2] == 2:
                wv.s[r[1] + 1] = ((val >> 32) & M32, (kn >> 32) & M32)
            return
        if op in ("vcc", "exec"):
            if width == 32:
                pv, pk = wv.special[op]
                val = (pv & ~M32) | (val & M32)
                kn = (pk & ~M32) | (kn & M32)
            wv.special[op] = (val & M64, kn & M64)
            return
        if op in ("vcc_lo", "exec_lo", "vcc_hi", "exec_hi"):
            base = op[:-3]
            pv, pk = wv.special[base]
            sh = 0 if op.endswith("lo") else 32
            keep = ~(M32 << sh) & M64
            wv.special[base] = ((pv & keep) | ((val & M32) << sh), (pk & keep) | ((kn & M32) << sh))
            return
        if op == "m0":
            wv.special["m0"] = (val & M32, kn & M32)
            return
        if op in ("null", "off"):
            return
        raise ReplayError(f"scalar destination {op}")

    # vector registers

    def _vget(self, wv: Wave, op: str, width=32):
        """(values [64] uint64, known [64] bool) of a vector operand (a scalar broadcast)."""
        if _modified(op):
            return np.zeros(LANES, np.uint64), NONE.copy()
        r = _reg(op)
        if r and r[0] in "va":
            base = r[1] + (512 if r[0] == "a" else 0)
            if width == 64:
                val = wv.v[base] | (wv.v[base + 1] << np.uint64(32))
                return val, wv.vk[base] & wv.vk[base + 1]
            return wv.v[base].copy(), wv.vk[base].copy()
        val, kn = self._sget(wv, op, width)
        full = M64 if width == 64 else M32
        if (kn & full) == full:
            return np.full(LANES, val, dtype=np.uint64), ALL.copy()
        return np.full(LANES, val, dtype=np.uint64), NONE.copy()

    def _exec_lanes(self, wv: Wave):
        """(lanes surely active, lanes whose activity is unknown)."""
        key = wv.special["exec"]
        got = self._exec_memo.get(key)
        if got is None:
            bits, known = self._mask_lanes(*key)
            got = self._exec_memo[key] = (bits & known, ~known)
        return got

    def _vset(self, wv: Wave, op: str, val, known, width=32):
        r = _reg(op)
        if not r or r[0] not in "va":
            raise ReplayError(f"vector destination {op}")
        on, maybe = self._exec_lanes(wv)
        base = r[1] + (512 if r[0] == "a" else 0)
        val = np.asarray(val, dtype=np.uint64)
        regs = [(base, val & np.uint64(M32))]
        if width == 64:
            regs.append((base + 1, (val >> np.uint64(32)) & np.uint64(M32)))
        for reg, v in regs:
            wv.v[reg] = np.where(on | maybe, v, wv.v[reg])
            wv.vk[reg] = np.where(on, known, np.where(maybe, False, wv.vk[reg]))

    def _unknown_dest(self, wv: Wave, op: str):
        r = _reg(op)
        if r is None:
            if op in ("vcc", "vcc_lo", "vcc_hi", "exec", "exec_lo", "exec_hi", "m0"):
                self._sset(wv, op, 0, 0, 64 if op in ("vcc", "exec") else 32)
            return
        kind, first, count = r
        if kind == "s":
            for j in range(count):
                wv.s[first + j] = (0, 0)
        else:
            base = first + (512 if kind == "a" else 0)
            on, maybe = self._exec_lanes(wv)
            for j in range(count):
                wv.vk[base + j] = np.where(on | maybe, False, wv.vk[base + j])

    _WEIGHTS = np.uint64(1) << np.arange(LANES, dtype=np.uint64)

    def _lane_mask(self, bits: np.ndarray, known: np.ndarray):
        """A 64-bit lane mask (value, known bits) from per-lane bits."""
        kn = int(np.sum(self._WEIGHTS[known], dtype=np.uint64))
        val = int(np.sum(self._WEIGHTS[known & bits], dtype=np.uint64))
        return val, kn

    def _mask_lanes(self, val, kn):
        bits = (np.uint64(val) >> np.arange(LANES, dtype=np.uint64)) & np.uint64(1)
        known = (np.uint64(kn) >> np.arange(LANES, dtype=np.uint64)) & np.uint64(1)
        return bits.astype(bool), known.astype(bool)

    # memory

    def _read(self, addr: int, size: int):
        """The little-endian integer of `size` bytes at addr, or None outside the described memory."""
        for base, data in self.memory.items():
            if base <= addr and addr + size <= base + len(data):
                return int.from_bytes(data[addr - base : addr - base + size], "little")
        return None

    # -- running --

    def run(self):
        while True:
            runnable = [w for w in self.waves if not w.done and not w.at_barrier]
            if not runnable:
                waiting = [w for w in self.waves if w.at_barrier]
                if not waiting:
                    break
                self.epoch += 1
                for w in waiting:
                    w.at_barrier = False
                continue
            for w in runnable:
                while not w.done and not w.at_barrier:
                    self._step(w)
                    self.steps += 1
                    if self.steps > self.budget:
                        raise ReplayError(f"past {self.budget} instructions")
        return self

    def _retire(self, wv: Wave, keep: int):
        while len(wv.queue) > keep:
            d = wv.queue.pop(0)
            if d is not None:
                d.retired_epoch = self.epoch
                d.retired_pos = wv.pos

    def _issue(self, wv: Wave, dma: Dma | None):
        wv.queue.append(dma)
        if dma is not None:
            self.dmas.append(dma)

    def _branch(self, wv: Wave, target: str, taken):
        if taken is None:
            self.unknown_branches += 1
            taken = self.unknown_branch == "take"
        if taken:
            wv.pc = self.k.labels[target]

    def _step(self, wv: Wave):
        if wv.pc >= len(self.k.code):
            raise ReplayError("ran past the kernel's end")
        mn, ops, mods, text = self.k.code[wv.pc]
        wv.pc += 1
        wv.pos += 1
        try:
            self._execute(wv, mn, ops, mods, text)
        except ReplayError:
            raise
        except Exception as e:  # noqa: BLE001 - reported with the instruction
            raise ReplayError(f"{text}: {e!r}") from e

    def _execute(self, wv, mn, ops, mods, text):
        base = re.sub(r"_e(32|64)$", "", mn)
        if mn in ("s_nop", "s_setprio", "s_sleep") or mn.startswith("s_sched") or base == "s_waitcnt_lgkmcnt":
            return
        if mn == "s_endpgm":
            wv.done = True
            for d in wv.queue:
                if d is not None:
                    self.ended_in_flight.append(f"wave {wv.index}: {d.what}")
            return
        if mn == "s_barrier":
            wv.at_barrier = True
            return
        if mn == "s_waitcnt":
            m = re.search(r"vmcnt\((\d+)\)", " ".join(ops + [f"{k}:{v}" for k, v in mods.items()]) + " " + text)
            if m:
                self._retire(wv, int(m.group(1)))
            elif ops and _literal(ops[0]) is not None and "(" not in text:
                imm = _literal(ops[0])
                self._retire(wv, (imm & 0xF) | (((imm >> 14) & 3) << 4))
            return
        if base == "s_branch":
            wv.pc = self.k.labels[ops[0]]
            return
        if base.startswith("s_cbranch_"):
            cond = base[len("s_cbranch_"):]
            if cond in ("scc0", "scc1"):
                v, known = wv.scc
                self._branch(wv, ops[0], None if not known else (bool(v) == (cond == "scc1")))
            elif cond in ("vccz", "vccnz", "execz", "execnz"):
                val, kn = wv.special["vcc" if cond.startswith("vcc") else "exec"]
                if val & kn:
                    nonzero = True
                elif kn == M64:
                    nonzero = False
                else:
                    nonzero = None
                taken = None if nonzero is None else (nonzero if cond.endswith("nz") else not nonzero)
                self._branch(wv, ops[0], taken)
            else:
                raise ReplayError(f"branch {mn}")
            return
        if mn.startswith("s_load_dword"):
            self._s_load(wv, mn, ops)
            return
        if mn.startswith("s_buffer_load") or mn.startswith("s_memtime") or mn.startswith("s_getreg"):
            self._unknown_dest(wv, ops[0])
            return
        if mn.startswith("s_"):
            self._salu(wv, base, ops, text)
            return
        if mn.startswith("global_load_lds") or mn.startswith("buffer_load") and "lds" in mods:
            self._dma(wv, mn, ops, mods, text)
            return
        if mn.startswith(("global_load", "flat_load")):
            self._global_load(wv, mn, ops, mods)
            return
        if mn.startswith(("global_store", "flat_store", "global_atomic", "flat_atomic", "buffer_", "scratch_")):
            self._issue(wv, None)
            if mn.startswith(("buffer_load", "scratch_load", "buffer_atomic", "global_atomic", "flat_atomic")) and ops:
                if "glc" in mods or "sc0" in mods or mn.startswith(("buffer_load", "scratch_load")):
                    self._unknown_dest(wv, ops[0])
            return
        if mn.startswith("ds_"):
            self._lds(wv, mn, ops, mods, text)
            return
        if mn.startswith("v_"):
            self._valu(wv, base, mn, ops, mods, text)
            return
        raise ReplayError(f"instruction {text}")

    # -- scalar ALU --

    def _salu(self, wv, base, ops, text):
        op = base[2:]
        w64 = base.endswith("64")
        width = 64 if w64 else 32
        full = M64 if w64 else M32

        def g(i, wd=width):
            return self._sget(wv, ops[i], wd)

        def known(*xs, wd=width):
            f = M64 if wd == 64 else M32
            return all((x[1] & f) == f for x in xs)

        def setd(val, kn, wd=width):
            self._sset(wv, ops[0], val & (M64 if wd == 64 else M32), kn, wd)

        def setscc(v, k):
            wv.scc = (int(bool(v)), bool(k))

        def sx(v, bits=32):
            v &= (1 << bits) - 1
            return v - (1 << bits) if v >> (bits - 1) else v

        if op in ("mov_b32", "mov_b64", "movk_i32", "cmov_b32", "cmov_b64"):
            if op.startswith("cmov"):
                c, ck = wv.scc
                if not ck:
                    setd(0, 0)
                    return
                if not c:
                    return
            a = g(1)
            if op == "movk_i32":
                a = (sx(a[0], 16) & M32, M32)
            setd(*a)
            return
        if op in ("and_b32", "and_b64", "or_b32", "or_b64", "xor_b32", "xor_b64", "andn2_b32", "andn2_b64",
                  "orn2_b32", "orn2_b64", "nand_b64", "nor_b64", "xnor_b64"):
            a, b = g(1), g(2)
            if op.startswith(("andn2", "orn2")):
                b = ((~b[0]) & full, b[1])
            if op.startswith(("and", "nand")):
                val = a[0] & b[0]
                kn = (a[1] & b[1]) | (a[1] & ~a[0]) | (b[1] & ~b[0])
            elif op.startswith(("or", "nor")):
                val = a[0] | b[0]
                kn = (a[1] & b[1]) | (a[1] & a[0]) | (b[1] & b[0])
            else:
                val = a[0] ^ b[0]
                kn = a[1] & b[1]
            if op.startswith(("nand", "nor", "xnor")):
                val = ~val
            val &= full
            kn &= full
            setd(val, kn)
            setscc(val & kn != 0 or val != 0, kn == full or (val & kn) != 0)
            return
        if op in ("not_b32", "not_b64"):
            a = g(1)
            setd((~a[0]) & full, a[1])
            setscc(((~a[0]) & full) != 0, a[1] == full)
            return
        if op.endswith("saveexec_b64"):
            a = g(1, 64)
            ex = wv.special["exec"]
            self._sset(wv, ops[0], ex[0], ex[1], 64)
            kind = op[: -len("_saveexec_b64")]
            if kind == "and":
                val, kn = a[0] & ex[0], (a[1] & ex[1]) | (a[1] & ~a[0]) | (ex[1] & ~ex[0])
            elif kind == "or":
                val, kn = a[0] | ex[0], (a[1] & ex[1]) | (a[1] & a[0]) | (ex[1] & ex[0])
            elif kind == "andn2":
                nex = (~ex[0]) & M64
                val, kn = a[0] & nex, (a[1] & ex[1]) | (a[1] & ~a[0]) | (ex[1] & ex[0])
            elif kind == "xor":
                val, kn = a[0] ^ ex[0], a[1] & ex[1]
            else:
                raise ReplayError(f"instruction {text}")
            wv.special["exec"] = (val & M64, kn & M64)
            setscc(val != 0, kn == M64 or (val & kn) != 0)
            return
        if op in ("cselect_b32", "cselect_b64"):
            c, ck = wv.scc
            if not ck:
                setd(0, 0)
                return
            setd(*g(1 if c else 2))
            return
        if op.startswith("cmp_") or op.startswith("cmpk_"):
            m2 = re.match(r"cmpk?_(\w+)_(\w)(\d+)", op)
            rel, sign, bits = m2.group(1), m2.group(2), int(m2.group(3))
            a, b = g(0, bits), g(1, bits)
            if op.startswith("cmpk"):
                b = (sx(b[0], 16) & M32, M32) if sign == "i" else (b[0] & 0xFFFF, M32)
            if not known(a, b, wd=bits):
                setscc(0, False)
                return
            x, y = a[0], b[0]
            if sign == "i":
                x, y = sx(x, bits), sx(y, bits)
            r = {"eq": x == y, "lg": x != y, "gt": x > y, "ge": x >= y, "lt": x < y, "le": x <= y}[rel]
            setscc(r, True)
            return
        if op in ("bitset0_b32", "bitset1_b32", "bitset0_b64", "bitset1_b64"):
            d, b = g(0), g(1, 32)
            if (b[1] & M32) != M32:
                setd(0, 0)
                return
            bit = 1 << (b[0] & (63 if w64 else 31))
            setd((d[0] | bit) if op.startswith("bitset1") else (d[0] & ~bit), d[1] | bit)
            return
        if op in ("bitcmp0_b32", "bitcmp1_b32"):
            a, b = g(0), g(1)
            if not known(a, b):
                setscc(0, False)
                return
            bit = (a[0] >> (b[0] & 31)) & 1
            setscc(bit == (1 if op.startswith("bitcmp1") else 0), True)
            return
        # arithmetic: known only when every input is
        widths = [32] * (len(ops) - 1)
        if op in ("lshl_b64", "lshr_b64", "ashr_i64", "bcnt1_i32_b64"):
            widths[0] = 64
        srcs = [g(i + 1, wd) for i, wd in enumerate(widths)]
        if op in ("addc_u32", "subb_u32"):
            srcs.append((wv.scc[0], M32 if wv.scc[1] else 0))
            widths.append(32)
        if not all((k & (M64 if wd == 64 else M32)) == (M64 if wd == 64 else M32) for (_, k), wd in zip(srcs, widths)):
            self._unknown_dest(wv, ops[0])
            wv.scc = (0, False)
            return
        v = [s[0] for s in srcs]
        res = None
        scc = None
        if op in ("add_u32", "add_i32", "addk_i32"):
            if op == "addk_i32":
                a0 = g(0)
                if a0[1] != M32:
                    self._unknown_dest(wv, ops[0])
                    return
                v = [a0[0], sx(v[0], 16) & M32]
            t = v[0] + v[1]
            res = t & M32
            scc = t > M32 if op == "add_u32" else (sx(v[0]) + sx(v[1])) != sx(res)
        elif op == "addc_u32":
            t = v[0] + v[1] + v[2]
            res, scc = t & M32, t > M32
        elif op in ("sub_u32", "sub_i32"):
            res = (v[0] - v[1]) & M32
            scc = v[1] > v[0] if op == "sub_u32" else (sx(v[0]) - sx(v[1])) != sx(res)
        elif op == "subb_u32":
            t = v[0] - v[1] - v[2]
            res, scc = t & M32, t < 0
        elif op == "mul_i32":
            res = (v[0] * v[1]) & M32
        elif op == "mul_hi_u32":
            res = ((v[0] * v[1]) >> 32) & M32
        elif op == "mul_hi_i32":
            res = ((sx(v[0]) * sx(v[1])) >> 32) & M32
        elif op == "lshl_b32":
            res = (v[0] << (v[1] & 31)) & M32
            scc = res != 0
        elif op == "lshr_b32":
            res = (v[0] >> (v[1] & 31)) & M32
            scc = res != 0
        elif op == "ashr_i32":
            res = (sx(v[0]) >> (v[1] & 31)) & M32
            scc = res != 0
        elif op == "lshl_b64":
            r64 = (v[0] << (v[1] & 63)) & M64
            setd(r64, M64, 64)
            wv.scc = (int(r64 != 0), True)
            return
        elif op == "lshr_b64":
            r64 = (v[0] >> (v[1] & 63)) & M64
            setd(r64, M64, 64)
            wv.scc = (int(r64 != 0), True)
            return
        elif op == "ashr_i64":
            r64 = (sx(v[0], 64) >> (v[1] & 63)) & M64
            setd(r64, M64, 64)
            wv.scc = (int(r64 != 0), True)
            return
        elif op in ("lshl1_add_u32", "lshl2_add_u32", "lshl3_add_u32", "lshl4_add_u32"):
            t = (v[0] << int(op[4])) + v[1]
            res, scc = t & M32, t > M32
        elif op in ("min_i32", "max_i32"):
            f = min if op.startswith("min") else max
            res = f(sx(v[0]), sx(v[1])) & M32
            scc = res == v[0]
        elif op in ("min_u32", "max_u32"):
            f = min if op.startswith("min") else max
            res = f(v[0], v[1])
            scc = res == v[0]
        elif op == "abs_i32":
            res = abs(sx(v[0])) & M32
            scc = res != 0
        elif op in ("bfe_u32", "bfe_i32"):
            off, width_ = v[1] & 31, (v[1] >> 16) & 127
            x = (v[0] >> off) & ((1 << width_) - 1) if width_ else 0
            if op == "bfe_i32" and width_:
                x = sx(x, width_)
            res = x & M32
            scc = res != 0
        elif op in ("sext_i32_i8", "sext_i32_i16"):
            res = sx(v[0], 8 if op.endswith("i8") else 16) & M32
        elif op == "bcnt1_i32_b32":
            res = bin(v[0]).count("1")
            scc = res != 0
        elif op == "bcnt1_i32_b64":
            res = bin(v[0]).count("1")
            scc = res != 0
        elif op in ("ff1_i32_b32",):
            res = (v[0] & -v[0]).bit_length() - 1 if v[0] else M32
        elif op in ("pack_ll_b32_b16",):
            res = (v[0] & 0xFFFF) | ((v[1] & 0xFFFF) << 16)
        else:
            raise ReplayError(f"instruction {text}")
        setd(res, M32)
        if scc is not None:
            wv.scc = (int(bool(scc)), True)

    def _s_load(self, wv, mn, ops):
        count = {"s_load_dword": 1, "s_load_dwordx2": 2, "s_load_dwordx3": 3, "s_load_dwordx4": 4, "s_load_dwordx8": 8,
                 "s_load_dwordx16": 16}[mn]
        base = self._sget(wv, ops[1], 64)
        off = self._sget(wv, ops[2]) if len(ops) > 2 else (0, M32)
        dst = _reg(ops[0])
        if base[1] != M64 or off[1] != M32:
            for j in range(count):
                wv.s[dst[1] + j] = (0, 0)
            return
        addr = base[0] + off[0]
        for j in range(count):
            val = self._read(addr + 4 * j, 4)
            wv.s[dst[1] + j] = (val, M32) if val is not None else (0, 0)

    # -- vector memory --

    def _global_addr(self, wv, ops, mods):
        """Each lane's address of a global instruction whose address operands start at ops[0]
        (vaddr, then saddr or off)."""
        off = int(mods.get("offset", "0"), 0)
        if len(ops) >= 2 and ops[1] != "off" and _reg(ops[1]) and _reg(ops[1])[0] == "s":
            s = self._sget(wv, ops[1], 64)
            va, vk = self._vget(wv, ops[0], 32)
            return (va + np.uint64(s[0]) + np.uint64(off & M64)) & np.uint64(M64), vk & (s[1] == M64)
        va, vk = self._vget(wv, ops[0], 64)
        return (va + np.uint64(off & M64)) & np.uint64(M64), vk

    def _global_load(self, wv, mn, ops, mods):
        size = {"dword": 4, "dwordx2": 8, "dwordx3": 12, "dwordx4": 16, "ushort": 2, "sshort": 2, "ubyte": 1,
                "sbyte": 1}.get(mn.split("_", 2)[-1], None)
        dst = _reg(ops[0])
        addr, ak = self._global_addr(wv, ops[1:], mods)
        self._issue(wv, None)
        if size is None or dst is None:
            self._unknown_dest(wv, ops[0])
            return
        regs = max(1, size // 4)
        vals = np.zeros((regs, LANES), dtype=np.uint64)
        known = np.zeros((regs, LANES), dtype=bool)
        inside = np.zeros(LANES, dtype=bool)
        for b0, data in self.memory.items():
            inside |= (addr >= np.uint64(b0)) & (addr < np.uint64(b0 + len(data)))
        if not np.any(inside & ak):
            self._unknown_dest(wv, ops[0])
            return
        for lane in range(LANES):
            if not ak[lane]:
                continue
            for j in range(regs):
                x = self._read(int(addr[lane]) + 4 * j, min(4, size))
                if x is not None:
                    vals[j, lane] = x
                    known[j, lane] = True
        for j in range(regs):
            self._vset(wv, f"v{dst[1] + j}" if dst[0] == "v" else f"a{dst[1] + j}", vals[j], known[j])

    def _dma(self, wv, mn, ops, mods, text):
        size = {"dword": 4, "dwordx3": 12, "dwordx4": 16, "ubyte": 1, "sbyte": 1, "ushort": 2, "sshort": 2}[mn.split("_")[-1]]
        if mods.get("offset") and int(mods["offset"], 0):
            raise ReplayError(f"an instruction offset on a load into LDS: {text}")
        m0, kn = wv.special["m0"]
        if kn != M32:
            raise ReplayError(f"M0 unknown at {text}")
        on, maybe = self._exec_lanes(wv)
        lanes = np.nonzero(on | maybe)[0]
        if len(lanes) == 0:
            self._issue(wv, None)
            return
        lo, hi = m0 + size * int(lanes.min()), m0 + size * (int(lanes.max()) + 1)
        self._issue(wv, Dma(wv.index, self.epoch, wv.pos, lo, hi, f"{text} @ {wv.pc - 1} into [{lo:#x}, {hi:#x})"))
        self.lds_known[max(0, lo) : min(hi, LDS_BYTES)] = False

    def _lds(self, wv, mn, ops, mods, text):
        if mn in ("ds_bpermute_b32", "ds_permute_b32", "ds_swizzle_b32"):
            self._unknown_dest(wv, ops[0])
            return
        read = mn.startswith("ds_read")
        m = re.match(r"ds_(read|write)(2st64|2)?_([bui])(\d+)$", mn)
        if m:
            size = int(m.group(4)) // 8
            two = m.group(2)
        else:
            size, two = 4, None  # LDS atomics
        addr_op = ops[1] if read else ops[0]
        va, vk = self._vget(wv, addr_op, 32)
        on, maybe = self._exec_lanes(wv)
        live = on | maybe
        if not np.any(live):
            return
        if two:
            unit = size * (64 if two == "2st64" else 1)
            offs = [int(mods.get("offset0", "0"), 0) * unit, int(mods.get("offset1", "0"), 0) * unit]
        else:
            offs = [int(mods.get("offset", "0"), 0)]
        if not np.all(vk[live]):
            # An address the replay cannot resolve: the access may reach any byte of LDS.
            self.unresolved_accesses += 1
            self.accesses.append(Access(wv.index, self.epoch, wv.pos, 0, LDS_BYTES, f"{text} @ {wv.pc - 1} (address unknown)"))
            if read:
                self._unknown_dest(wv, ops[0])
            else:
                self.lds_known[:] = False
            return
        addrs = va[live].astype(np.int64)
        for o in offs:
            lo, hi = int(addrs.min()) + o, int(addrs.max()) + o + size
            self.accesses.append(Access(wv.index, self.epoch, wv.pos, lo, hi, f"{text} @ {wv.pc - 1}"))
        if not m or size not in (4, 8, 16) and not (read and size in (1, 2)):
            if read:
                self._unknown_dest(wv, ops[0])
            return
        lanes = np.nonzero(live)[0]
        words = max(1, size // 4)
        nb = min(4, size)
        shifts = (np.arange(nb, dtype=np.uint64) * np.uint64(8))
        if read:
            dst = _reg(ops[0])
            for j, o in enumerate(offs):
                for word in range(words):
                    at = va[lanes].astype(np.int64) + o + 4 * word
                    ok = (at >= 0) & (at + nb <= LDS_BYTES)
                    idx = np.where(ok, at, 0)[:, None] + np.arange(nb)
                    vals = np.zeros(LANES, np.uint64)
                    known = np.zeros(LANES, bool)
                    vals[lanes] = np.sum(self.lds[idx].astype(np.uint64) << shifts, axis=1, dtype=np.uint64)
                    known[lanes] = self.lds_known[idx].all(axis=1) & ok & on[lanes]
                    self._vset(wv, f"{dst[0]}{dst[1] + j * words + word}", vals, known)
        else:
            data = [_reg(o) for o in ops[1:]]
            for j, o in enumerate(offs):
                d = data[j] if j < len(data) else data[0]
                dbase = d[1] + (512 if d[0] == "a" else 0)
                for word in range(words):
                    at = va[lanes].astype(np.int64) + o + 4 * word
                    ok = (at >= 0) & (at + 4 <= LDS_BYTES)
                    at, ln = at[ok], lanes[ok]
                    idx = at[:, None] + np.arange(4)
                    vals = wv.v[dbase + word][ln] & np.uint64(M32)
                    self.lds[idx] = ((vals[:, None] >> (np.arange(4, dtype=np.uint64) * np.uint64(8))) & np.uint64(0xFF)).astype(np.uint8)
                    self.lds_known[idx] = (wv.vk[dbase + word][ln] & on[ln])[:, None]

    # -- vector ALU --

    def _valu(self, wv, base, mn, ops, mods, text):
        op = base[2:]
        u32 = np.uint64(M32)

        def g(i, wd=32):
            return self._vget(wv, ops[i], wd)

        def put(val, known, wd=32, dst=0):
            self._vset(wv, ops[dst], val, known, wd)

        def sx(a, bits=32):
            a = a.astype(np.int64) & ((1 << bits) - 1)
            return np.where(a >> (bits - 1) & 1, a - (1 << bits), a)

        if op in _FLOAT_OPS and not ("dpp" in mods or "row_shr" in mods or "quad_perm" in mods or mn.endswith("_sdwa")
                                     or "op_sel" in mods or "clamp" in mods or "mul" in mods or "div" in mods):
            self._float(wv, op, ops)
            return
        if "dpp" in mods or "row_shr" in mods or "quad_perm" in mods or "sdwa" in mn or mn.endswith("_sdwa") \
                or "op_sel" in mods or any(_modified(o) for o in ops[1:]):
            if op.startswith("cmp"):
                self._unknown_dest(wv, "vcc" if mn.endswith("e32") else ops[0])
            else:
                self._unknown_dest(wv, ops[0])
            return
        if op.startswith("cmpx"):
            raise ReplayError(f"instruction {text}")
        if op.startswith("cmp_"):
            m = re.match(r"cmp_(\w+)_([uif])(\d+)", op)
            dst, srcs = ops[0], ops[1:3]  # vcc (e32) or an SGPR pair (e64), then the two sources
            on, maybe = self._exec_lanes(wv)
            if m is None or m.group(2) == "f" or m.group(1) in ("class",):
                self._sset(wv, dst, *self._lane_mask(np.zeros(LANES, bool), ~(on | maybe)), 64)
                return
            rel, sign, bits_ = m.group(1), m.group(2), int(m.group(3))
            a, ak = self._vget(wv, srcs[0], bits_)
            b, bk = self._vget(wv, srcs[1], bits_)
            if sign == "i":
                a, b = sx(a, bits_), sx(b, bits_)
            else:
                a, b = a.astype(np.uint64), b.astype(np.uint64)
            r = {"eq": a == b, "ne": a != b, "lg": a != b, "lt": a < b, "le": a <= b, "gt": a > b, "ge": a >= b,
                 "f": np.zeros(LANES, bool), "t": np.ones(LANES, bool)}[rel]
            res = r & on
            kn = (on & ak & bk) | ~(on | maybe)
            self._sset(wv, dst, *self._lane_mask(res, kn), 64)
            return
        if op == "cndmask_b32":
            mask = ops[3] if len(ops) > 3 else "vcc"
            a, ak = g(1)
            b, bk = g(2)
            mv, mk = self._sget(wv, mask, 64)
            mb, mkn = self._mask_lanes(mv, mk)
            put(np.where(mb, b, a), np.where(mb, bk, ak) & mkn)
            return
        if op == "readfirstlane_b32":
            a, ak = g(1)
            on, maybe = self._exec_lanes(wv)
            first = None
            for i in range(LANES):
                if maybe[i]:
                    break
                if on[i]:
                    first = i
                    break
            if first is None or not ak[first]:
                self._sset(wv, ops[0], 0, 0)
            else:
                self._sset(wv, ops[0], int(a[first]), M32)
            return
        if op == "readlane_b32":
            a, ak = g(1)
            ln = self._sget(wv, ops[2])
            if ln[1] != M32 or not ak[ln[0] & 63]:
                self._sset(wv, ops[0], 0, 0)
            else:
                self._sset(wv, ops[0], int(a[ln[0] & 63]), M32)
            return
        if op == "writelane_b32":
            val = self._sget(wv, ops[1])
            ln = self._sget(wv, ops[2])
            r = _reg(ops[0])
            reg = r[1] + (512 if r[0] == "a" else 0)
            if ln[1] != M32:
                wv.vk[reg] = False
            else:
                wv.v[reg][ln[0] & 63] = val[0]
                wv.vk[reg][ln[0] & 63] = val[1] == M32
            return
        if op in ("mbcnt_lo_u32_b32", "mbcnt_hi_u32_b32"):
            mv, mk = self._sget(wv, ops[1])
            b, bk = g(2)
            lane = np.arange(LANES)
            shift = 0 if op.startswith("mbcnt_lo") else 32
            cnt = np.array([bin(mv & ((1 << max(0, min(32, l - shift))) - 1)).count("1") for l in lane], dtype=np.uint64)
            put((cnt + b) & u32, bk & (mk == M32))
            return
        if op in ("add_co_u32", "sub_co_u32", "subrev_co_u32", "addc_co_u32", "subb_co_u32", "subbrev_co_u32"):
            # d, carry-out, a, b[, carry-in]
            cdst = ops[1]
            a, ak = g(2)
            b, bk = g(3)
            cin, cink = np.zeros(LANES, np.uint64), ALL.copy()
            if op in ("addc_co_u32", "subb_co_u32", "subbrev_co_u32"):
                mv, mk = self._sget(wv, ops[4] if len(ops) > 4 else "vcc", 64)
                cb, ck = self._mask_lanes(mv, mk)
                cin, cink = cb.astype(np.uint64), ck
            if op.startswith("subrev") or op == "subbrev_co_u32":
                a, b = b, a
                ak, bk = bk, ak
            if op.startswith("add"):
                t = a + b + cin
                res, carry = t & u32, t > u32
            else:
                t = a.astype(np.int64) - b.astype(np.int64) - cin.astype(np.int64)
                res, carry = (t & M32).astype(np.uint64), t < 0
            known = ak & bk & cink
            on, maybe = self._exec_lanes(wv)
            put(res, known)
            self._sset(wv, cdst, *self._lane_mask(carry & on, (on & known) | ~(on | maybe)), 64)
            return
        if op in ("mad_u64_u32", "mad_i64_i32"):
            a, ak = g(2)
            b, bk = g(3)
            c, ck = g(4, 64)
            if op == "mad_i64_i32":
                p = (sx(a) * sx(b)).astype(np.int64)
                res = (p.astype(np.uint64) + c) & np.uint64(M64)
            else:
                res = (a * b + c) & np.uint64(M64)
            put(res, ak & bk & ck, 64)
            self._unknown_dest(wv, ops[1])
            return
        if op == "lshl_add_u64":
            a, ak = g(1, 64)
            s, sk = g(2)
            c, ck = g(3, 64)
            put(((a << (s & np.uint64(63))) + c) & np.uint64(M64), ak & sk & ck, 64)
            return
        if op in ("lshlrev_b64", "lshrrev_b64", "ashrrev_i64"):
            s, sk = g(1)
            a, ak = g(2, 64)
            sh = s & np.uint64(63)
            if op == "lshlrev_b64":
                res = (a << sh) & np.uint64(M64)
            elif op == "lshrrev_b64":
                res = a >> sh
            else:
                res = (sx(a, 64) >> sh.astype(np.int64)).astype(np.uint64)
            put(res, ak & sk, 64)
            return
        if op == "mov_b64":
            a, ak = g(1, 64)
            put(a, ak, 64)
            return
        two = {"add_u32": lambda a, b: a + b, "sub_u32": lambda a, b: a - b, "subrev_u32": lambda a, b: b - a,
               "and_b32": lambda a, b: a & b, "or_b32": lambda a, b: a | b, "xor_b32": lambda a, b: a ^ b,
               "lshlrev_b32": lambda a, b: b << (a & np.uint64(31)), "lshrrev_b32": lambda a, b: b >> (a & np.uint64(31)),
               "ashrrev_i32": lambda a, b: (sx(b) >> (a & np.uint64(31)).astype(np.int64)).astype(np.uint64),
               "mul_lo_u32": lambda a, b: a * b, "mul_hi_u32": lambda a, b: (a * b) >> np.uint64(32),
               "mul_u32_u24": lambda a, b: (a & np.uint64(0xFFFFFF)) * (b & np.uint64(0xFFFFFF)),
               "mul_i32_i24": lambda a, b: (sx(a & np.uint64(0xFFFFFF), 24) * sx(b & np.uint64(0xFFFFFF), 24)).astype(np.uint64),
               "min_u32": np.minimum, "max_u32": np.maximum,
               "min_i32": lambda a, b: np.minimum(sx(a), sx(b)).astype(np.uint64),
               "max_i32": lambda a, b: np.maximum(sx(a), sx(b)).astype(np.uint64),
               "add_u16": lambda a, b: (a + b) & np.uint64(0xFFFF), "sub_u16": lambda a, b: (a - b) & np.uint64(0xFFFF)}
        if op in two and len(ops) == 3:
            a, ak = g(1)
            b, bk = g(2)
            with np.errstate(over="ignore"):
                put(two[op](a, b).astype(np.uint64) & u32, ak & bk)
            return
        three = {"and_or_b32": lambda a, b, c: (a & b) | c, "or3_b32": lambda a, b, c: a | b | c,
                 "xor3_b32": lambda a, b, c: a ^ b ^ c, "add3_u32": lambda a, b, c: a + b + c,
                 "lshl_add_u32": lambda a, b, c: (a << (b & np.uint64(31))) + c,
                 "add_lshl_u32": lambda a, b, c: (a + b) << (c & np.uint64(31)),
                 "lshl_or_b32": lambda a, b, c: (a << (b & np.uint64(31))) | c,
                 "mad_u32_u24": lambda a, b, c: (a & np.uint64(0xFFFFFF)) * (b & np.uint64(0xFFFFFF)) + c,
                 "bfe_u32": lambda a, b, c: (a >> (b & np.uint64(31))) & ((np.uint64(1) << (c & np.uint64(31))) - np.uint64(1)),
                 "bfi_b32": lambda a, b, c: (a & b) | (~a & c),
                 "alignbit_b32": lambda a, b, c: (((a << np.uint64(32)) | b) >> (c & np.uint64(31))),
                 "perm_b32": None}
        if op in three and three[op] is not None and len(ops) == 4:
            a, ak = g(1)
            b, bk = g(2)
            c, ck = g(3)
            with np.errstate(over="ignore"):
                put(three[op](a, b, c).astype(np.uint64) & u32, ak & bk & ck)
            return
        if op == "bfe_i32":
            a, ak = g(1)
            b, bk = g(2)
            c, ck = g(3)
            res = np.zeros(LANES, np.uint64)
            for i in range(LANES):
                w_ = int(c[i]) & 31
                x = (int(a[i]) >> (int(b[i]) & 31)) & ((1 << w_) - 1) if w_ else 0
                if w_ and x >> (w_ - 1):
                    x -= 1 << w_
                res[i] = x & M32
            put(res, ak & bk & ck)
            return
        if op == "bitop3_b32":
            a, ak = g(1)
            b, bk = g(2)
            c, ck = g(3)
            table = int(mods.get("bitop3", "0"), 0)
            res = np.zeros(LANES, np.uint64)
            for t in range(8):
                if table >> t & 1:
                    sa = a if t & 4 else ~a
                    sb = b if t & 2 else ~b
                    sc = c if t & 1 else ~c
                    res |= sa & sb & sc
            put(res & u32, ak & bk & ck)
            return
        if op in ("mov_b32", "not_b32"):
            a, ak = g(1)
            put((~a if op == "not_b32" else a) & u32, ak)
            return
        # anything else (floating point, matrix, conversions, packing): its destination unknown
        if ops:
            if op.startswith("mfma") or op.startswith("accvgpr") or op.startswith("smfmac"):
                self._unknown_dest(wv, ops[0])
                return
            if op in ("div_scale_f32", "div_scale_f64"):
                self._unknown_dest(wv, ops[0])
                self._unknown_dest(wv, ops[1])
                return
            if op in ("readfirstlane_b32",):
                self._unknown_dest(wv, ops[0])
                return
            self._unknown_dest(wv, ops[0])

    def _float(self, wv, op, ops):
        """Single-precision arithmetic on every lane, as IEEE float32 (the integer division
        sequences the compiler emits start from a reciprocal estimate and correct it exactly)."""

        def fget(i):
            o = ops[i]
            neg = o.startswith("-") and _modified(o)
            o = o[1:] if neg else o
            ab = o.startswith("|")
            o = o.strip("|")
            v, k = self._vget(wv, o, 32)
            x = (v & np.uint64(M32)).astype(np.uint32).view(np.float32)
            if ab:
                x = np.abs(x)
            if neg:
                x = -x
            return x, k

        with np.errstate(all="ignore"):
            if op in ("cvt_f32_u32", "cvt_f32_i32"):
                v, k = self._vget(wv, ops[1], 32)
                x = (v & np.uint64(M32)).astype(np.uint32)
                r = x.astype(np.float32) if op.endswith("u32") else x.view(np.int32).astype(np.float32)
                self._vset(wv, ops[0], r.view(np.uint32).astype(np.uint64), k)
                return
            if op in ("cvt_u32_f32", "cvt_i32_f32"):
                x, k = fget(1)
                x = np.nan_to_num(np.trunc(x.astype(np.float64)), nan=0.0)
                if op == "cvt_u32_f32":
                    r = np.clip(x, 0, M32).astype(np.uint64)
                else:
                    r = (np.clip(x, -(2**31), 2**31 - 1).astype(np.int64) & M32).astype(np.uint64)
                self._vset(wv, ops[0], r, k)
                return
            unary = {"rcp_iflag_f32": lambda a: np.float32(1.0) / a, "rcp_f32": lambda a: np.float32(1.0) / a,
                     "trunc_f32": np.trunc, "floor_f32": np.floor, "mov_b32": lambda a: a}
            binary = {"mul_f32": lambda a, b: a * b, "add_f32": lambda a, b: a + b, "sub_f32": lambda a, b: a - b,
                      "subrev_f32": lambda a, b: b - a, "max_f32": np.maximum, "min_f32": np.minimum}
            if op in unary:
                a, ak = fget(1)
                r = unary[op](a).astype(np.float32)
                k = ak
            elif op in binary:
                a, ak = fget(1)
                b, bk = fget(2)
                r = binary[op](a, b).astype(np.float32)
                k = ak & bk
            elif op in ("fma_f32", "fmac_f32", "mac_f32"):
                a, ak = fget(1)
                b, bk = fget(2)
                c, ck = fget(3) if op == "fma_f32" else fget(0)
                r = (a.astype(np.float64) * b.astype(np.float64) + c.astype(np.float64)).astype(np.float32)
                k = ak & bk & ck
            else:
                raise ReplayError(f"float op {op}")
            self._vset(wv, ops[0], r.view(np.uint32).astype(np.uint64), k)

    # -- the check --

    def hazards(self) -> list[str]:
        """Every LDS access a direct-to-LDS load into its bytes could still be in flight for, and
        every wave that ended with such a load in flight."""
        out = []
        grain = 1024
        index = {}
        for d in self.dmas:
            for g in range(d.lo // grain, (d.hi - 1) // grain + 1):
                index.setdefault(g, []).append(d)
        for a in self.accesses:
            seen = set()
            for g in range(a.lo // grain, (a.hi - 1) // grain + 1):
                for d in index.get(g, ()):
                    if id(d) in seen or d.hi <= a.lo or a.hi <= d.lo:
                        continue
                    seen.add(id(d))
                    if d.wave == a.wave:
                        if d.pos < a.pos and (d.retired_pos is None or d.retired_pos > a.pos):
                            out.append(f"wave {a.wave} reads before its own load landed: {a.what} / {d.what}")
                    elif d.epoch < a.epoch:
                        if d.retired_epoch is None or d.retired_epoch >= a.epoch:
                            out.append(f"wave {a.wave} (between barriers {a.epoch} and {a.epoch + 1}) reads before wave "
                                       f"{d.wave}'s load landed: {a.what} / {d.what}")
                    elif d.epoch == a.epoch:
                        out.append(f"wave {a.wave} and wave {d.wave}'s load into the same bytes between barriers "
                                   f"{a.epoch} and {a.epoch + 1}: {a.what} / {d.what}")
        out += [f"ended with a load into LDS in flight: {e}" for e in self.ended_in_flight]
        return out

    def summary(self) -> dict:
        return {"waves": len(self.waves), "barriers": self.epoch, "loads_into_lds": len(self.dmas),
                "lds_accesses": len(self.accesses), "instructions": self.steps, "unknown_branches": self.unknown_branches,
                "unresolved_lds_addresses": self.unresolved_accesses}


# ---- kernel arguments ------------------------------------------------------------------------------


def kernarg(kernel: Kernel, explicit: list[bytes], grid=(1, 1, 1), block=(256, 1, 1)) -> bytes:
    """The kernel's argument segment: the explicit arguments' bytes in order at the offsets the
    metadata gives, then the hidden arguments the kernel reads (grid and block sizes)."""
    args = kernel.meta.get(".args", [])
    size = kernel.desc.get("kernarg_size", max((a[".offset"] + a[".size"] for a in args), default=0))
    seg = bytearray(size)
    ex = [a for a in args if not a[".value_kind"].startswith("hidden_")]
    if len(ex) != len(explicit):
        raise ReplayError(f"{len(explicit)} arguments for {len(ex)}")
    for a, b in zip(ex, explicit):
        if len(b) != a[".size"]:
            raise ReplayError(f"argument at {a['.offset']}: {len(b)} bytes for {a['.size']}")
        seg[a[".offset"] : a[".offset"] + a[".size"]] = b
    hidden = {"hidden_block_count_x": grid[0], "hidden_block_count_y": grid[1], "hidden_block_count_z": grid[2],
              "hidden_group_size_x": block[0], "hidden_group_size_y": block[1], "hidden_group_size_z": block[2],
              "hidden_remainder_x": 0, "hidden_remainder_y": 0, "hidden_remainder_z": 0, "hidden_grid_dims": 2}
    for a in args:
        kind = a[".value_kind"]
        if kind in hidden:
            seg[a[".offset"] : a[".offset"] + a[".size"]] = int(hidden[kind]).to_bytes(a[".size"], "little")
    return bytes(seg)


def layouts(dump: str) -> dict:
    """Struct layouts from clang's record layout dump (-Xclang -fdump-record-layouts): for each
    struct by its unqualified name, {"sizeof": n, field: [offset, size]} (int, float and 32-bit
    integer fields 4 bytes, pointers 8)."""
    out = {}
    for block in dump.split("*** Dumping AST Record Layout")[1:]:
        lines = block.strip("\n").split("\n")
        m = re.match(r"\s*0 \| (?:struct|class) (.+)$", lines[0])
        if not m or "<" in m.group(1) or "std::" in m.group(1):
            continue
        name = m.group(1).split("::")[-1].strip()
        fields = {}
        for line in lines[1:]:
            sm = re.search(r"\[sizeof=(\d+)", line)
            if sm:
                fields["sizeof"] = int(sm.group(1))
                break
            fm = re.match(r"\s*(\d+) \|   (\S.*?) (\w+)$", line)
            if fm and not line.split("|", 1)[1].startswith("    "):
                typ = fm.group(2)
                fields[fm.group(3)] = [int(fm.group(1)), 8 if "*" in typ else 4]
        out.setdefault(name, fields)
    return out


def pack(layout: dict, struct: str, values: dict) -> bytes:
    """A struct's bytes from its fields' offsets and sizes (`layout`[struct] = {"sizeof": n,
    field: [offset, size]}), each field's value an int (a float is given as its bits)."""
    desc = layout[struct]
    out = bytearray(desc["sizeof"])
    for name, v in values.items():
        off, size = desc[name]
        out[off : off + size] = int(v & ((1 << (8 * size)) - 1)).to_bytes(size, "little")
    return bytes(out)
