"""TEST INFRASTRUCTURE -- GPU-free virtual machine for the gfx950 SGEMM kernels.

Only tests/ (and __graft_entry__.smoke) use it, as a checker; the product never
imports it.

It executes, on the CPU, the AMD assembly that hipcc produces for this
project's own HIP kernel (``GpuContext.assembly()`` of generator.py), so the
kernel's indexing, LDS traffic, K loop, MFMA operand layout and epilogue can be
checked against numpy without a GPU.  The public surface keeps the reference
VM's (/root/reference/vm/gcn_virtual_machine.py:53-582):
``GcnVirtualMachine(nsgpr, nvgpr, wavefront_size)`` with register files
``s``, ``v``, ``a``, memories ``smem`` (kernel arguments, read by ``s_load``),
``vmem`` (global memory, byte offsets are addresses) and ``lds``, ``run(context)``
for one wave, and ``accvgpr_to_ndarray`` / ``vgpr_to_ndarray`` for the MFMA
layouts.  On top of that ``run_kernel`` dispatches a whole grid: every
work-group in turn, its waves interleaved at ``s_barrier``.

Semantics that make it a checker rather than a simulator:

* 32-bit wrap-around integer arithmetic, EXEC masking, SCC/VCC;
* loads snapshot memory when issued and write their destination registers only
  when an ``s_waitcnt`` retires them (in order per counter), so a missing wait
  reads stale registers and shows up as a wrong result;
* every global/LDS/kernarg access is bounds-checked: an out-of-range address
  raises ``MemoryError`` naming the instruction;
* an unknown mnemonic or operand form raises ``NotImplementedError``.

MFMA layouts (CDNA3/CDNA4 ISA, v_mfma_f32_32x32x2_f32 and _16x16x4_f32): lane l
supplies A[l % M][l // M] and B[l // N][l % N]; accumulator slot q of lane l is
D[(q % 4) + 8 (q // 4) + 4 (l // 32)][l % 32] (32x32) or D[q + 4 (l // 16)][l % 16]
(16x16).  Products are accumulated in float64 and rounded to float32 once per
instruction.
"""
from __future__ import annotations

import re
import struct
from collections import deque
from typing import Callable, Dict, List, Optional, Sequence, Tuple

import numpy as np

MASK32 = 0xFFFFFFFF
MASK64 = (1 << 64) - 1
WAVE = 64


# ------------------------------------------------------------------ memory
class Memory:
    """Byte-addressed, bounds-checked memory; ``.mem`` is the backing array."""

    def __init__(self, num_bytes: int, name: str):
        self.mem = bytearray(int(num_bytes))
        self._u8 = np.frombuffer(self.mem, dtype=np.uint8)  # writable view of the same bytes
        self.name = name
        # optional list of (start, end) byte ranges that kernels may touch; an
        # access must lie entirely inside one of them (host accesses are free)
        self.regions: Optional[List[Tuple[int, int]]] = None

    @property
    def size(self) -> int:
        return len(self.mem)

    def allocate_region(self, start: int, nbytes: int, label: str = ""):
        if self.regions is None:
            self.regions = []
        self.regions.append((int(start), int(start) + int(nbytes), label))

    def _check(self, addr: np.ndarray, nbytes: int, where: str):
        n = len(self.mem)
        if addr.size and (int(addr.min()) < 0 or int(addr.max()) + nbytes > n):
            bad = int(addr.max()) if int(addr.max()) + nbytes > n else int(addr.min())
            raise MemoryError(f"{where}: {self.name} access at byte {bad} (+{nbytes}) outside [0, {n})")
        if self.regions is not None and where not in ("host write", "host read") and addr.size:
            ok = np.zeros(addr.shape, dtype=bool)
            for lo, hi, _ in self.regions:
                ok |= (addr >= lo) & (addr + nbytes <= hi)
            if not ok.all():
                bad = int(addr[~ok][0])
                raise MemoryError(f"{where}: {self.name} access at byte {bad} (+{nbytes}) is outside every "
                                  f"allocated buffer {[(lo, hi, l) for lo, hi, l in self.regions]}")

    def read_u32(self, addr: np.ndarray, ndwords: int, where: str) -> np.ndarray:
        """addr: (L,) byte addresses; returns (ndwords, L) uint32."""
        addr = np.asarray(addr, dtype=np.int64)
        self._check(addr, 4 * ndwords, where)
        idx = addr[None, :] + 4 * np.arange(ndwords, dtype=np.int64)[:, None]
        b = self._u8[idx[..., None] + np.arange(4)]
        return (b[..., 0].astype(np.uint32) | (b[..., 1].astype(np.uint32) << 8)
                | (b[..., 2].astype(np.uint32) << 16) | (b[..., 3].astype(np.uint32) << 24))

    def write_u32(self, addr: np.ndarray, data: np.ndarray, where: str):
        """addr: (L,), data: (ndwords, L) uint32; lanes written in order."""
        addr = np.asarray(addr, dtype=np.int64)
        nd = data.shape[0]
        self._check(addr, 4 * nd, where)
        for lane in range(addr.size):
            a = int(addr[lane])
            self.mem[a:a + 4 * nd] = data[:, lane].astype("<u4").tobytes()

    def write_bytes(self, offset: int, raw: bytes):
        self._check(np.array([offset]), len(raw), "host write")
        self.mem[offset:offset + len(raw)] = raw

    def read_bytes(self, offset: int, nbytes: int) -> bytes:
        self._check(np.array([offset]), nbytes, "host read")
        return bytes(self.mem[offset:offset + nbytes])


# ------------------------------------------------------------------ parsing
_REG = re.compile(r"^([sva])(\d+)$")
_RANGE = re.compile(r"^([sva])\[(\d+):(\d+)\]$")
_SPECIAL = {"vcc": ("vcc", 2), "exec": ("exec", 2), "vcc_lo": ("vcc_lo", 1), "vcc_hi": ("vcc_hi", 1),
            "exec_lo": ("exec_lo", 1), "exec_hi": ("exec_hi", 1), "m0": ("m0", 1), "scc": ("scc", 1)}
_INLINE_FLOATS = {"0.5": 0x3F000000, "-0.5": 0xBF000000, "1.0": 0x3F800000, "-1.0": 0xBF800000,
                  "2.0": 0x40000000, "-2.0": 0xC0000000, "4.0": 0x40800000, "-4.0": 0xC0800000,
                  "0.15915494": 0x3E22F983}


class Operand:
    __slots__ = ("kind", "index", "count", "value", "text")

    def __init__(self, kind, index=0, count=1, value=0, text=""):
        self.kind, self.index, self.count, self.value, self.text = kind, index, count, value, text

    def __repr__(self):
        return self.text


def parse_operand(tok: str) -> Operand:
    tok = tok.strip()
    m = _REG.match(tok)
    if m:
        return Operand(m.group(1), int(m.group(2)), 1, text=tok)
    m = _RANGE.match(tok)
    if m:
        lo, hi = int(m.group(2)), int(m.group(3))
        return Operand(m.group(1), lo, hi - lo + 1, text=tok)
    if tok in _SPECIAL:
        kind, cnt = _SPECIAL[tok]
        return Operand(kind, 0, cnt, text=tok)
    if tok == "off":
        return Operand("off", text=tok)
    if tok in _INLINE_FLOATS:
        return Operand("imm", value=_INLINE_FLOATS[tok], text=tok)
    try:
        if tok.lower().startswith(("0x", "-0x")):
            v = int(tok, 16)
        else:
            v = int(tok, 10)
        return Operand("imm", value=v, text=tok)
    except ValueError:
        pass
    if re.match(r"^-?\d+\.\d*(e-?\d+)?$", tok):
        return Operand("imm", value=struct.unpack("<I", struct.pack("<f", float(tok)))[0], text=tok)
    if re.match(r"^[.A-Za-z_][\w.$]*$", tok):
        return Operand("label", text=tok, value=tok)
    raise NotImplementedError(f"operand form {tok!r}")


class Instruction:
    __slots__ = ("mnemonic", "ops", "mods", "text", "line")

    def __init__(self, mnemonic: str, ops: List[Operand], mods: Dict[str, int], text: str, line: int):
        self.mnemonic, self.ops, self.mods, self.text, self.line = mnemonic, ops, mods, text, line

    def __repr__(self):
        return f"{self.line}: {self.text}"


def _split_operands(rest: str) -> Tuple[List[str], List[str]]:
    parts = [p.strip() for p in rest.split(",")] if rest.strip() else []
    mods: List[str] = []
    if parts:
        last = parts[-1].split()
        parts[-1] = last[0] if last else ""
        mods = last[1:]
        if parts[-1] == "":
            parts.pop()
    return parts, mods


def parse_assembly(asm: str, kernel: str = "generated_gemm") -> "Program":
    """Instructions of ``kernel`` plus the kernel-descriptor fields the VM needs."""
    lines = asm.splitlines()
    start = None
    for i, line in enumerate(lines):
        if line.split(";")[0].strip() == f"{kernel}:":
            start = i + 1
            break
    if start is None:
        raise ValueError(f"kernel {kernel} not found in assembly")
    insts: List[Instruction] = []
    labels: Dict[str, int] = {}
    for i in range(start, len(lines)):
        raw = lines[i].split(";")[0].rstrip()
        t = raw.strip()
        if not t:
            continue
        if t.startswith(".Lfunc_end") or t == "s_code_end":
            break
        if t.endswith(":"):
            labels[t[:-1]] = len(insts)
            continue
        if t.startswith("."):
            continue
        mn, _, rest = t.partition(" ")
        if mn == "s_waitcnt":
            mods = {}
            for m in re.finditer(r"(vmcnt|lgkmcnt|expcnt)\((\d+)\)", rest):
                mods[m.group(1)] = int(m.group(2))
            insts.append(Instruction(mn, [], mods, t, i + 1))
            continue
        toks, modtoks = _split_operands(rest)
        mods: Dict[str, int] = {}
        for mt in modtoks:
            if ":" in mt:
                k, v = mt.split(":", 1)
                mods[k] = int(v, 0)
            else:
                mods[mt] = 1
        ops = [parse_operand(x) for x in toks]
        insts.append(Instruction(mn, ops, mods, t, i + 1))
    # the descriptor block of this kernel only (a code object may hold several)
    m = re.search(r"\.amdhsa_kernel\s+" + re.escape(kernel) + r"\b(.*?)\.end_amdhsa_kernel", asm, re.S)
    block = m.group(1) if m else asm
    desc = {}
    for key in ("amdhsa_group_segment_fixed_size", "amdhsa_user_sgpr_count", "amdhsa_user_sgpr_kernarg_segment_ptr",
                "amdhsa_system_sgpr_workgroup_id_x", "amdhsa_system_sgpr_workgroup_id_y",
                "amdhsa_system_sgpr_workgroup_id_z", "amdhsa_user_sgpr_dispatch_ptr", "amdhsa_user_sgpr_queue_ptr",
                "amdhsa_user_sgpr_dispatch_id", "amdhsa_user_sgpr_private_segment_size",
                "amdhsa_system_vgpr_workitem_id", "amdhsa_next_free_sgpr", "amdhsa_next_free_vgpr",
                "amdhsa_accum_offset", "amdhsa_kernarg_size"):
        m = re.search(r"\." + key + r"\s+(\d+)", block)
        if m:
            desc[key] = int(m.group(1))
    return Program(insts, labels, desc)


class Program:
    def __init__(self, insts, labels, desc):
        self.insts = insts
        self.labels = labels
        self.desc = desc


def _f32(u: np.ndarray) -> np.ndarray:
    return np.asarray(u, dtype=np.uint32).view(np.float32)


def _u32(f: np.ndarray) -> np.ndarray:
    return np.asarray(f, dtype=np.float32).view(np.uint32)


def _sext(v: int, bits: int) -> int:
    v &= (1 << bits) - 1
    return v - (1 << bits) if v >> (bits - 1) else v


class BarrierReached(Exception):
    pass


class Yielded(Exception):
    """A wave gave up its turn (``s_sleep``, or a preemption point) without
    reaching a barrier: the other waves of its work-group run next."""


# ---------------------------------------------------------------- the VM
class GcnVirtualMachine:
    """One wave's architectural state plus the memories it sees."""

    def __init__(self, nsgpr: int = 104, nvgpr: int = 512, wavefront_size: int = WAVE,
                 vmem_bytes: int = 1 << 20, smem_bytes: int = 4096, lds_bytes: int = 160 * 1024):
        if wavefront_size != WAVE:
            raise ValueError("gfx950 waves are 64 lanes")
        self.wavefront_size = wavefront_size
        self.s = np.zeros(nsgpr, dtype=np.uint32)
        self.v = np.zeros((nvgpr, WAVE), dtype=np.uint32)
        self.a = np.zeros((256, WAVE), dtype=np.uint32)
        self.vcc = 0
        self.exec = MASK64
        self.scc = 0
        self.m0 = 0
        self.vmem = Memory(vmem_bytes, "vmem")
        self.smem = Memory(smem_bytes, "smem")
        self.lds = Memory(lds_bytes, "lds")
        self.pending: Dict[str, deque] = {"vmcnt": deque(), "lgkmcnt": deque()}
        self.pc = 0
        self.done = False
        self.executed = 0
        self.trace: Optional[Callable[[Instruction], None]] = None

    # ---------------------------------------------------------- helpers
    def exec_mask(self) -> np.ndarray:
        return ((self.exec >> np.arange(WAVE, dtype=np.uint64)) & np.uint64(1)).astype(bool)

    @staticmethod
    def _bits(mask: np.ndarray) -> int:
        out = 0
        for i in np.nonzero(mask)[0]:
            out |= 1 << int(i)
        return out

    def rs32(self, op: Operand) -> int:
        k = op.kind
        if k == "s":
            return int(self.s[op.index])
        if k == "imm":
            return op.value & MASK32
        if k in ("vcc", "vcc_lo"):
            return self.vcc & MASK32
        if k == "vcc_hi":
            return self.vcc >> 32
        if k in ("exec", "exec_lo"):
            return self.exec & MASK32
        if k == "exec_hi":
            return self.exec >> 32
        if k == "m0":
            return self.m0
        raise NotImplementedError(f"scalar read of {op}")

    def rs64(self, op: Operand) -> int:
        k = op.kind
        if k == "s":
            return int(self.s[op.index]) | (int(self.s[op.index + 1]) << 32)
        if k == "imm":
            return op.value & MASK64 if op.value >= 0 else (op.value & MASK64)
        if k == "vcc":
            return self.vcc
        if k == "exec":
            return self.exec
        raise NotImplementedError(f"64-bit scalar read of {op}")

    def ws32(self, op: Operand, val: int):
        val &= MASK32
        k = op.kind
        if k == "s":
            self.s[op.index] = val
        elif k == "vcc_lo":
            self.vcc = (self.vcc & ~MASK32 & MASK64) | val
        elif k == "vcc_hi":
            self.vcc = (self.vcc & MASK32) | (val << 32)
        elif k == "exec_lo":
            self.exec = (self.exec & ~MASK32 & MASK64) | val
        elif k == "exec_hi":
            self.exec = (self.exec & MASK32) | (val << 32)
        elif k == "m0":
            self.m0 = val
        else:
            raise NotImplementedError(f"scalar write of {op}")

    def ws64(self, op: Operand, val: int):
        val &= MASK64
        if op.kind == "s":
            self.s[op.index] = val & MASK32
            self.s[op.index + 1] = val >> 32
        elif op.kind == "vcc":
            self.vcc = val
        elif op.kind == "exec":
            self.exec = val
        else:
            raise NotImplementedError(f"64-bit scalar write of {op}")

    def rv32(self, op: Operand) -> np.ndarray:
        if op.kind == "v":
            return self.v[op.index].copy()
        if op.kind == "a":
            return self.a[op.index].copy()
        return np.full(WAVE, self.rs32(op), dtype=np.uint32)

    def rv64(self, op: Operand) -> np.ndarray:
        if op.kind == "v":
            return self.v[op.index].astype(np.uint64) | (self.v[op.index + 1].astype(np.uint64) << np.uint64(32))
        return np.full(WAVE, self.rs64(op), dtype=np.uint64)

    def wv32(self, op: Operand, val: np.ndarray, mask: Optional[np.ndarray] = None):
        mask = self.exec_mask() if mask is None else mask
        val = np.asarray(val).astype(np.uint32) if np.asarray(val).dtype != np.uint32 else np.asarray(val)
        if op.kind == "v":
            self.v[op.index][mask] = val[mask] if val.shape else val
        elif op.kind == "a":
            self.a[op.index][mask] = val[mask] if val.shape else val
        else:
            raise NotImplementedError(f"vector write of {op}")

    def wv64(self, op: Operand, val: np.ndarray):
        mask = self.exec_mask()
        val = np.asarray(val, dtype=np.uint64)
        self.v[op.index][mask] = (val & np.uint64(MASK32)).astype(np.uint32)[mask]
        self.v[op.index + 1][mask] = (val >> np.uint64(32)).astype(np.uint32)[mask]

    def regfile(self, op: Operand) -> np.ndarray:
        """The vector register file a memory instruction's data operand names:
        VGPRs, or AGPRs (gfx90a and later load and store them directly)."""
        if op.kind == "v":
            return self.v
        if op.kind == "a":
            return self.a
        raise NotImplementedError(f"vector memory data operand {op}")

    def reg_block(self, op: Operand) -> np.ndarray:
        """(count, 64) view of a v/a register range."""
        f = self.v if op.kind == "v" else self.a if op.kind == "a" else None
        if f is None:
            raise NotImplementedError(f"register block {op}")
        return f[op.index:op.index + op.count]

    # ---------------------------------------------- reference-style views
    def vgpr_to_ndarray(self, reg, rows: int, k: int) -> np.ndarray:
        """MFMA source operand as a (k, rows) float32 array: [kk][i] = lane i + rows*kk."""
        idx = reg.index if hasattr(reg, "index") else int(reg)
        return _f32(self.v[idx]).reshape(k, rows).copy()

    def accvgpr_to_ndarray(self, reg, m: int, n: int, k: int = 0) -> np.ndarray:
        """MFMA accumulator as D transposed, (n, m): [j][i] = D[i][j]."""
        idx = reg.index if hasattr(reg, "index") else int(reg)
        out = np.zeros((n, m), dtype=np.float32)
        slots = 16 if m == 32 else 4
        rows, cols = _ACC_INDEX[m]
        out[cols, rows] = _f32(self.a[idx:idx + slots].copy())
        return out

    # ----------------------------------------------------------- running
    def reset_wave(self):
        self.pending = {"vmcnt": deque(), "lgkmcnt": deque()}
        self.pc = 0
        self.done = False

    def run(self, context, max_instructions: int = 10_000_000):
        """Runs one wave of ``context`` (a Program, assembly text, or a
        generator GpuContext) from the current register state to s_endpgm."""
        prog = as_program(context)
        self.reset_wave()
        while not self.done:
            try:
                self.step(prog, max_instructions)
            except (BarrierReached, Yielded):
                continue  # a lone wave passes its barriers and keeps its turns
        return self

    def step(self, prog: "Program", max_instructions: int = 10_000_000,
             preempt: Optional[Callable[[], bool]] = None):
        """Executes until s_endpgm (sets done), an s_barrier (raises
        BarrierReached) or an s_sleep (raises Yielded).  ``preempt``, called
        after every instruction, can end the turn early (raises Yielded): a
        seeded random one explores interleavings of the waves' LDS accesses."""
        insts = prog.insts
        while True:
            if self.pc >= len(insts):
                raise RuntimeError("ran past the end of the kernel without s_endpgm")
            ins = insts[self.pc]
            self.pc += 1
            self.executed += 1
            if self.executed > max_instructions:
                raise RuntimeError("instruction budget exhausted (infinite loop?)")
            if self.trace:
                self.trace(ins)
            fn = _DISPATCH.get(ins.mnemonic)
            if fn is None:
                raise NotImplementedError(f"mnemonic {ins.mnemonic} ({ins})")
            r = fn(self, ins, prog)
            if r == "end":
                self.drain()
                self.done = True
                return
            if r == "barrier":
                raise BarrierReached()
            if r == "yield" or (preempt is not None and preempt()):
                raise Yielded()

    def drain(self):
        for q in self.pending.values():
            while q:
                q.popleft()()

    def retire(self, counter: str, keep: int):
        q = self.pending[counter]
        while len(q) > keep:
            q.popleft()()


def _acc_pos(m: int, q: int, lane: int) -> Tuple[int, int]:
    if m == 32:
        return (q % 4) + 8 * (q // 4) + 4 * (lane // 32), lane % 32
    return q + 4 * (lane // 16), lane % 16


def _acc_index(m: int) -> Tuple[np.ndarray, np.ndarray]:
    """(rows, cols) arrays of shape (slots, 64): where each accumulator slot lives in D."""
    slots = 16 if m == 32 else 4
    q = np.arange(slots)[:, None]
    lane = np.arange(WAVE)[None, :]
    if m == 32:
        return (q % 4) + 8 * (q // 4) + 4 * (lane // 32), np.broadcast_to(lane % 32, (slots, WAVE))
    return q + 4 * (lane // 16), np.broadcast_to(lane % 16, (slots, WAVE))


_ACC_INDEX = {32: _acc_index(32), 16: _acc_index(16)}


def as_program(context, kernel: Optional[str] = None) -> Program:
    """The parsed kernel of a Program, an assembly text or a generator context
    (``kernel`` defaults to the context's kernel name, else generated_gemm)."""
    if isinstance(context, Program):
        return context
    if isinstance(context, str):
        return parse_assembly(context, kernel or "generated_gemm")
    if hasattr(context, "assembly"):
        name = kernel or getattr(context, "name", None) or "generated_gemm"
        cache = getattr(context, "_vm_programs", None)
        if cache is None:
            cache = context._vm_programs = {}
        if name not in cache:
            cache[name] = parse_assembly(context.assembly(), name)
        return cache[name]
    raise TypeError(f"cannot run {type(context)}")


# ------------------------------------------------------------ semantics
_DISPATCH: Dict[str, Callable] = {}


def op(*names):
    def deco(fn):
        for n in names:
            _DISPATCH[n] = fn
        return fn
    return deco


# scalar ALU -----------------------------------------------------------
def _salu2(name, fn, scc=None):
    @op(name)
    def _impl(vm, ins, prog):
        a, b = vm.rs32(ins.ops[1]), vm.rs32(ins.ops[2])
        r = fn(a, b)
        vm.ws32(ins.ops[0], r)
        if scc is not None:
            vm.scc = int(scc(a, b, r))


_salu2("s_add_i32", lambda a, b: a + b,
       lambda a, b, r: (_sext(a, 32) + _sext(b, 32)) != _sext(r, 32))
_salu2("s_sub_i32", lambda a, b: a - b,
       lambda a, b, r: (_sext(a, 32) - _sext(b, 32)) != _sext(r, 32))
_salu2("s_mul_i32", lambda a, b: (_sext(a, 32) * _sext(b, 32)))
_salu2("s_mul_hi_u32", lambda a, b: (a * b) >> 32)
_salu2("s_and_b32", lambda a, b: a & b, lambda a, b, r: (r & MASK32) != 0)
_salu2("s_or_b32", lambda a, b: a | b, lambda a, b, r: (r & MASK32) != 0)
_salu2("s_xor_b32", lambda a, b: a ^ b, lambda a, b, r: (r & MASK32) != 0)
_salu2("s_andn2_b32", lambda a, b: a & ~b & MASK32, lambda a, b, r: (r & MASK32) != 0)
_salu2("s_orn2_b32", lambda a, b: (a | ~b) & MASK32, lambda a, b, r: (r & MASK32) != 0)
_salu2("s_lshl_b32", lambda a, b: a << (b & 31), lambda a, b, r: (r & MASK32) != 0)
_salu2("s_lshr_b32", lambda a, b: a >> (b & 31), lambda a, b, r: (r & MASK32) != 0)
_salu2("s_ashr_i32", lambda a, b: _sext(a, 32) >> (b & 31), lambda a, b, r: (r & MASK32) != 0)
_salu2("s_min_i32", lambda a, b: a if _sext(a, 32) < _sext(b, 32) else b, lambda a, b, r: _sext(a, 32) < _sext(b, 32))
_salu2("s_min_u32", lambda a, b: min(a, b), lambda a, b, r: a < b)
_salu2("s_max_i32", lambda a, b: a if _sext(a, 32) > _sext(b, 32) else b, lambda a, b, r: _sext(a, 32) > _sext(b, 32))
_salu2("s_max_u32", lambda a, b: max(a, b), lambda a, b, r: a > b)


@op("s_add_u32")
def _s_add_u32(vm, ins, prog):
    a, b = vm.rs32(ins.ops[1]), vm.rs32(ins.ops[2])
    r = a + b
    vm.ws32(ins.ops[0], r)
    vm.scc = int(r > MASK32)


@op("s_addc_u32")
def _s_addc_u32(vm, ins, prog):
    a, b = vm.rs32(ins.ops[1]), vm.rs32(ins.ops[2])
    r = a + b + vm.scc
    vm.ws32(ins.ops[0], r)
    vm.scc = int(r > MASK32)


@op("s_sub_u32")
def _s_sub_u32(vm, ins, prog):
    a, b = vm.rs32(ins.ops[1]), vm.rs32(ins.ops[2])
    vm.ws32(ins.ops[0], a - b)
    vm.scc = int(b > a)


@op("s_subb_u32")
def _s_subb_u32(vm, ins, prog):
    a, b = vm.rs32(ins.ops[1]), vm.rs32(ins.ops[2])
    vm.ws32(ins.ops[0], a - b - vm.scc)
    vm.scc = int(b + vm.scc > a)


@op("s_abs_i32")
def _s_abs(vm, ins, prog):
    r = abs(_sext(vm.rs32(ins.ops[1]), 32))
    vm.ws32(ins.ops[0], r)
    vm.scc = int((r & MASK32) != 0)


@op("s_mov_b32")
def _s_mov_b32(vm, ins, prog):
    vm.ws32(ins.ops[0], vm.rs32(ins.ops[1]))


@op("s_mov_b64")
def _s_mov_b64(vm, ins, prog):
    vm.ws64(ins.ops[0], vm.rs64(ins.ops[1]))


@op("s_movk_i32")
def _s_movk(vm, ins, prog):
    vm.ws32(ins.ops[0], _sext(ins.ops[1].value, 16))


@op("s_mulk_i32")
def _s_mulk(vm, ins, prog):
    vm.ws32(ins.ops[0], _sext(vm.rs32(ins.ops[0]), 32) * _sext(ins.ops[1].value, 16))


@op("s_addk_i32")
def _s_addk(vm, ins, prog):
    a = vm.rs32(ins.ops[0])
    b = _sext(ins.ops[1].value, 16) & MASK32
    r = a + b
    vm.ws32(ins.ops[0], r)
    vm.scc = int((_sext(a, 32) + _sext(b, 32)) != _sext(r, 32))


@op("s_cselect_b32")
def _s_cselect_b32(vm, ins, prog):
    vm.ws32(ins.ops[0], vm.rs32(ins.ops[1]) if vm.scc else vm.rs32(ins.ops[2]))


@op("s_cselect_b64")
def _s_cselect_b64(vm, ins, prog):
    vm.ws64(ins.ops[0], vm.rs64(ins.ops[1]) if vm.scc else vm.rs64(ins.ops[2]))


def _salu64(name, fn):
    @op(name)
    def _impl(vm, ins, prog):
        r = fn(vm.rs64(ins.ops[1]), vm.rs64(ins.ops[2])) & MASK64
        vm.ws64(ins.ops[0], r)
        vm.scc = int(r != 0)


_salu64("s_and_b64", lambda a, b: a & b)
_salu64("s_or_b64", lambda a, b: a | b)
_salu64("s_xor_b64", lambda a, b: a ^ b)
_salu64("s_andn2_b64", lambda a, b: a & ~b)
_salu64("s_orn2_b64", lambda a, b: a | ~b)


@op("s_lshl_b64")
def _s_lshl_b64(vm, ins, prog):
    r = (vm.rs64(ins.ops[1]) << (vm.rs32(ins.ops[2]) & 63)) & MASK64
    vm.ws64(ins.ops[0], r)
    vm.scc = int(r != 0)


@op("s_lshr_b64")
def _s_lshr_b64(vm, ins, prog):
    r = vm.rs64(ins.ops[1]) >> (vm.rs32(ins.ops[2]) & 63)
    vm.ws64(ins.ops[0], r)
    vm.scc = int(r != 0)


@op("s_ashr_i64")
def _s_ashr_i64(vm, ins, prog):
    r = (_sext(vm.rs64(ins.ops[1]), 64) >> (vm.rs32(ins.ops[2]) & 63)) & MASK64
    vm.ws64(ins.ops[0], r)
    vm.scc = int(r != 0)


@op("s_bfe_i64")
def _s_bfe_i64(vm, ins, prog):
    src = vm.rs64(ins.ops[1])
    ctl = vm.rs32(ins.ops[2])
    off, width = ctl & 63, (ctl >> 16) & 127
    r = 0 if width == 0 else _sext(src >> off, width) & MASK64
    vm.ws64(ins.ops[0], r)
    vm.scc = int(r != 0)


@op("s_bfe_u32")
def _s_bfe_u32(vm, ins, prog):
    src, ctl = vm.rs32(ins.ops[1]), vm.rs32(ins.ops[2])
    off, width = ctl & 31, (ctl >> 16) & 127
    r = (src >> off) & ((1 << width) - 1) if width else 0
    vm.ws32(ins.ops[0], r)
    vm.scc = int(r != 0)


@op("s_and_saveexec_b64")
def _s_and_saveexec(vm, ins, prog):
    old = vm.exec
    vm.exec = vm.rs64(ins.ops[1]) & old
    vm.ws64(ins.ops[0], old)
    vm.scc = int(vm.exec != 0)


@op("s_andn2_saveexec_b64")
def _s_andn2_saveexec(vm, ins, prog):
    # EXEC = S0 & ~EXEC (the else-branch mask); the old EXEC goes to D
    old = vm.exec
    vm.exec = vm.rs64(ins.ops[1]) & ~old & MASK64
    vm.ws64(ins.ops[0], old)
    vm.scc = int(vm.exec != 0)


@op("s_or_saveexec_b64")
def _s_or_saveexec(vm, ins, prog):
    # the source is read before the destination (often the same pair) is written
    old = vm.exec
    vm.exec = (vm.rs64(ins.ops[1]) | old) & MASK64
    vm.ws64(ins.ops[0], old)
    vm.scc = int(vm.exec != 0)


def _scmp(name, fn, signed=False):
    @op(name)
    def _impl(vm, ins, prog):
        a, b = vm.rs32(ins.ops[0]), vm.rs32(ins.ops[1])
        if signed:
            a, b = _sext(a, 32), _sext(b, 32)
        vm.scc = int(fn(a, b))


def _scmpk(name, fn, signed=False):
    """s_cmpk_*: SOPK compare of an SGPR with a 16-bit immediate."""
    @op(name)
    def _impl(vm, ins, prog):
        a, imm = vm.rs32(ins.ops[0]), ins.ops[1].value & 0xFFFF
        if signed:
            a, imm = _sext(a, 32), _sext(imm, 16)
        vm.scc = int(fn(a, imm))


def _scmp64(name, fn):
    @op(name)
    def _impl(vm, ins, prog):
        vm.scc = int(fn(vm.rs64(ins.ops[0]), vm.rs64(ins.ops[1])))


for _n, _f in (("eq", lambda a, b: a == b), ("lg", lambda a, b: a != b), ("gt", lambda a, b: a > b),
               ("ge", lambda a, b: a >= b), ("lt", lambda a, b: a < b), ("le", lambda a, b: a <= b)):
    _scmp(f"s_cmp_{_n}_u32", _f)
    _scmp(f"s_cmp_{_n}_i32", _f, signed=True)
    _scmpk(f"s_cmpk_{_n}_u32", _f)
    _scmpk(f"s_cmpk_{_n}_i32", _f, signed=True)
_scmp64("s_cmp_eq_u64", lambda a, b: a == b)
_scmp64("s_cmp_lg_u64", lambda a, b: a != b)
# s_bitcmp{0,1}_b32: SCC = (bit S1[4:0] of S0) == 0 / == 1
_scmp("s_bitcmp0_b32", lambda a, b: (a >> (b & 31)) & 1 == 0)
_scmp("s_bitcmp1_b32", lambda a, b: (a >> (b & 31)) & 1 == 1)


# control flow ------------------------------------------------------------
def _jump(vm, ins, prog):
    target = ins.ops[0].value
    if target not in prog.labels:
        raise RuntimeError(f"unknown label {target}")
    vm.pc = prog.labels[target]


@op("s_branch")
def _s_branch(vm, ins, prog):
    _jump(vm, ins, prog)


for _n, _cond in (("s_cbranch_scc0", lambda vm: vm.scc == 0), ("s_cbranch_scc1", lambda vm: vm.scc == 1),
                  ("s_cbranch_vccz", lambda vm: vm.vcc == 0), ("s_cbranch_vccnz", lambda vm: vm.vcc != 0),
                  ("s_cbranch_execz", lambda vm: vm.exec == 0), ("s_cbranch_execnz", lambda vm: vm.exec != 0)):
    def _mk(cond):
        def _impl(vm, ins, prog):
            if cond(vm):
                _jump(vm, ins, prog)
        return _impl
    _DISPATCH[_n] = _mk(_cond)


@op("s_endpgm")
def _s_endpgm(vm, ins, prog):
    return "end"


@op("s_barrier")
def _s_barrier(vm, ins, prog):
    return "barrier"


@op("s_nop", "s_setprio", "s_sched_barrier", "s_code_end")
def _s_nop(vm, ins, prog):
    return None


@op("s_sleep")
def _s_sleep(vm, ins, prog):
    return "yield"  # a polling wave lets the others of its work-group run


@op("s_waitcnt")
def _s_waitcnt(vm, ins, prog):
    if "vmcnt" in ins.mods:
        vm.retire("vmcnt", ins.mods["vmcnt"])
    if "lgkmcnt" in ins.mods:
        vm.retire("lgkmcnt", ins.mods["lgkmcnt"])


# scalar memory -----------------------------------------------------------
def _s_load(nd):
    def _impl(vm, ins, prog):
        base = vm.rs64(ins.ops[1])
        off = vm.rs32(ins.ops[2]) if len(ins.ops) > 2 else 0
        addr = base + off
        data = vm.smem.read_u32(np.array([addr]), nd, str(ins))[:, 0].copy()
        dst = ins.ops[0]

        def land():
            for i in range(nd):
                vm.s[dst.index + i] = data[i]
        vm.pending["lgkmcnt"].append(land)
    return _impl


for _nd, _name in ((1, "s_load_dword"), (2, "s_load_dwordx2"), (4, "s_load_dwordx4"), (8, "s_load_dwordx8"),
                   (16, "s_load_dwordx16")):
    _DISPATCH[_name] = _s_load(_nd)


# vector ALU -------------------------------------------------------------
def _vop(name, fn, nsrc=2, clamped=None):
    """VOP1/2/3 op without carry.  ``clamped`` (optional) computes the exact
    result as int64 for the VOP3 ``clamp`` modifier, which saturates an
    unsigned integer result to [0, 2^32 - 1]; any other op with ``clamp``, or
    an op with another modifier, is not modelled and fails loudly."""
    def _impl(vm, ins, prog):
        srcs = [vm.rv32(o) for o in ins.ops[1:1 + nsrc]]
        unknown = set(ins.mods) - {"clamp"}
        if unknown:
            raise NotImplementedError(f"modifiers {sorted(unknown)} of {ins}")
        if "clamp" in ins.mods:
            if clamped is None:
                raise NotImplementedError(f"clamp modifier of {ins}")
            vm.wv32(ins.ops[0], np.clip(clamped(*srcs), 0, MASK32).astype(np.uint32))
        else:
            vm.wv32(ins.ops[0], fn(*srcs))
    for suffix in ("", "_e32", "_e64"):
        _DISPATCH[name + suffix] = _impl


_u64 = lambda x: x.astype(np.uint64)  # noqa: E731
_i64 = lambda x: x.astype(np.int64)  # noqa: E731
_vop("v_mov_b32", lambda a: a, 1)
_vop("v_add_u32", lambda a, b: (_u64(a) + _u64(b)).astype(np.uint32), clamped=lambda a, b: _i64(a) + _i64(b))
_vop("v_sub_u32", lambda a, b: (_u64(a) - _u64(b)).astype(np.uint32), clamped=lambda a, b: _i64(a) - _i64(b))
_vop("v_subrev_u32", lambda a, b: (_u64(b) - _u64(a)).astype(np.uint32), clamped=lambda a, b: _i64(b) - _i64(a))
_vop("v_and_b32", lambda a, b: a & b)
_vop("v_or_b32", lambda a, b: a | b)
_vop("v_xor_b32", lambda a, b: a ^ b)
_vop("v_lshlrev_b32", lambda s, a: (_u64(a) << _u64(s & 31)).astype(np.uint32))
_vop("v_lshrrev_b32", lambda s, a: a >> (s & 31))
_vop("v_ashrrev_i32", lambda s, a: (a.view(np.int32) >> (s & 31).astype(np.int32)).view(np.uint32))
_vop("v_mul_u32_u24", lambda a, b: ((_u64(a) & 0xFFFFFF) * (_u64(b) & 0xFFFFFF)).astype(np.uint32))
_vop("v_mul_lo_u32", lambda a, b: (_u64(a) * _u64(b)).astype(np.uint32))
_vop("v_mul_hi_u32", lambda a, b: ((_u64(a) * _u64(b)) >> np.uint64(32)).astype(np.uint32))
_vop("v_mad_u32_u24", lambda a, b, c: ((_u64(a) & 0xFFFFFF) * (_u64(b) & 0xFFFFFF) + _u64(c)).astype(np.uint32), 3)
_vop("v_add3_u32", lambda a, b, c: (_u64(a) + _u64(b) + _u64(c)).astype(np.uint32), 3)
_vop("v_or3_b32", lambda a, b, c: a | b | c, 3)
_vop("v_lshl_or_b32", lambda a, s, c: ((_u64(a) << _u64(s & 31)).astype(np.uint32)) | c, 3)
_vop("v_lshl_add_u32", lambda a, s, c: ((_u64(a) << _u64(s & 31)) + _u64(c)).astype(np.uint32), 3)
_vop("v_add_lshl_u32", lambda a, b, s: ((_u64(a) + _u64(b)).astype(np.uint32).astype(np.uint64)
                                        << _u64(s & 31)).astype(np.uint32), 3)
_vop("v_and_or_b32", lambda a, b, c: (a & b) | c, 3)
_vop("v_min_u32", np.minimum)
_vop("v_max_u32", np.maximum)
_vop("v_min_i32", lambda a, b: np.minimum(a.view(np.int32), b.view(np.int32)).view(np.uint32))
_vop("v_max_i32", lambda a, b: np.maximum(a.view(np.int32), b.view(np.int32)).view(np.uint32))
_vop("v_not_b32", lambda a: ~a, 1)
_vop("v_mul_i32_i24", lambda a, b: ((((a.astype(np.int64) << 40) >> 40) * ((b.astype(np.int64) << 40) >> 40))
                                    & MASK32).astype(np.uint32))
_vop("v_bfe_u32", lambda a, o, w: ((a.astype(np.uint64) >> (o & 31).astype(np.uint64))
                                   & ((np.uint64(1) << (w & 31).astype(np.uint64)) - np.uint64(1))).astype(np.uint32), 3)
_vop("v_bfi_b32", lambda m, a, b: (m & a) | (~m & b), 3)


def _v_bitop3_b32(vm, ins, prog):
    """gfx950 V_BITOP3_B32 D, S0, S1, S2 bitop3:T: bit i of D is bit
    (S0_i << 2 | S1_i << 1 | S2_i) of the 8-bit truth table T -- the
    convention under which S0, S1 and S2 alone are the tables 0xF0, 0xCC and
    0xAA (LLVM's AMDGPU backend builds T that way)."""
    unknown = set(ins.mods) - {"bitop3"}
    if unknown:
        raise NotImplementedError(f"modifiers {sorted(unknown)} of {ins}")
    table = ins.mods.get("bitop3", 0)
    a, b, c = (vm.rv32(o) for o in ins.ops[1:4])
    out = np.zeros_like(a)
    for idx in range(8):
        if (table >> idx) & 1:
            out |= (a if idx & 4 else ~a) & (b if idx & 2 else ~b) & (c if idx & 1 else ~c)
    vm.wv32(ins.ops[0], out)


for _suffix in ("", "_e64"):
    _DISPATCH["v_bitop3_b32" + _suffix] = _v_bitop3_b32


def _vop_carry(name, fn):
    """VOP2/VOP3b ops with a carry: vdst, [sdst,] src0, src1[, carry-in]."""
    def _impl(vm, ins, prog):
        ops = ins.ops
        if len(ops) >= 4 and ops[1].kind in ("s", "vcc"):
            dst, sdst, srcs = ops[0], ops[1], ops[2:]
        else:
            dst, sdst, srcs = ops[0], Operand("vcc", text="vcc"), ops[1:]
        a, b = vm.rv32(srcs[0]).astype(np.int64), vm.rv32(srcs[1]).astype(np.int64)
        cin = None
        if len(srcs) > 2:
            m = vm.rs64(srcs[2])
            cin = ((m >> np.arange(WAVE, dtype=np.uint64)) & np.uint64(1)).astype(np.int64)
        elif name.startswith(("v_addc", "v_subb")):
            cin = ((vm.vcc >> np.arange(WAVE, dtype=np.uint64)) & np.uint64(1)).astype(np.int64)
        r, carry = fn(a, b, cin if cin is not None else 0)
        vm.wv32(dst, (r & MASK32).astype(np.uint32))
        vm.ws64(sdst, GcnVirtualMachine._bits(carry & vm.exec_mask()))
    for suffix in ("", "_e32", "_e64"):
        _DISPATCH[name + suffix] = _impl


_vop_carry("v_add_co_u32", lambda a, b, c: (a + b, (a + b) > MASK32))
_vop_carry("v_addc_co_u32", lambda a, b, c: (a + b + c, (a + b + c) > MASK32))
_vop_carry("v_sub_co_u32", lambda a, b, c: (a - b, b > a))
_vop_carry("v_subrev_co_u32", lambda a, b, c: (b - a, a > b))
_vop_carry("v_subb_co_u32", lambda a, b, c: (a - b - c, (b + c) > a))
_vop_carry("v_subbrev_co_u32", lambda a, b, c: (b - a - c, (a + c) > b))
_vop("v_mul_f32", lambda a, b: _u32(_f32(a) * _f32(b)))
_vop("v_add_f32", lambda a, b: _u32(_f32(a) + _f32(b)))
_vop("v_sub_f32", lambda a, b: _u32(_f32(a) - _f32(b)))
_vop("v_cvt_f32_u32", lambda a: _u32(a.astype(np.float32)), 1)
_vop("v_cvt_f32_i32", lambda a: _u32(a.view(np.int32).astype(np.float32)), 1)


def _cvt_u32_f32(a):
    f = _f32(a).astype(np.float64)
    f = np.where(np.isnan(f), 0.0, f)
    f = np.clip(np.trunc(f), 0.0, float(MASK32))
    return f.astype(np.uint64).astype(np.uint32)


_vop("v_cvt_u32_f32", _cvt_u32_f32, 1)


def _rcp(a):
    with np.errstate(divide="ignore"):
        return _u32(np.float32(1.0) / _f32(a))


_vop("v_rcp_iflag_f32", _rcp, 1)
_vop("v_rcp_f32", _rcp, 1)


def _fma32(a, b, c):
    return _u32((_f32(a).astype(np.float64) * _f32(b).astype(np.float64) + _f32(c).astype(np.float64))
                .astype(np.float32))


_vop("v_fma_f32", _fma32, 3)


@op("v_fmac_f32_e32", "v_fmac_f32_e64", "v_fmac_f32")
def _v_fmac(vm, ins, prog):
    vm.wv32(ins.ops[0], _fma32(vm.rv32(ins.ops[1]), vm.rv32(ins.ops[2]), vm.rv32(ins.ops[0])))


@op("v_cndmask_b32_e64", "v_cndmask_b32_e32", "v_cndmask_b32")
def _v_cndmask(vm, ins, prog):
    src0, src1 = vm.rv32(ins.ops[1]), vm.rv32(ins.ops[2])
    mask = vm.rs64(ins.ops[3]) if len(ins.ops) > 3 else vm.vcc
    sel = ((mask >> np.arange(WAVE, dtype=np.uint64)) & np.uint64(1)).astype(bool)
    vm.wv32(ins.ops[0], np.where(sel, src1, src0).astype(np.uint32))


@op("v_mbcnt_lo_u32_b32", "v_mbcnt_lo_u32_b32_e64")
def _v_mbcnt_lo(vm, ins, prog):
    """Per lane: popcount of mask bits 0..min(lane, 32)-1 plus src1."""
    mask = vm.rv32(ins.ops[1]).astype(np.uint64)
    lane = np.arange(WAVE, dtype=np.uint64)
    below = np.where(lane >= 32, np.uint64(0xFFFFFFFF), (np.uint64(1) << lane) - np.uint64(1))
    cnt = np.array([bin(int(x)).count("1") for x in (mask & below)], dtype=np.uint64)
    vm.wv32(ins.ops[0], ((cnt + vm.rv32(ins.ops[2]).astype(np.uint64)) & np.uint64(MASK32)).astype(np.uint32))


@op("v_mbcnt_hi_u32_b32", "v_mbcnt_hi_u32_b32_e64")
def _v_mbcnt_hi(vm, ins, prog):
    """Per lane: popcount of mask bits 0..lane-33 (lanes 32..63) plus src1."""
    mask = vm.rv32(ins.ops[1]).astype(np.uint64)
    lane = np.arange(WAVE, dtype=np.uint64)
    below = np.where(lane < 32, np.uint64(0), (np.uint64(1) << np.maximum(lane, np.uint64(32)) - np.uint64(32))
                     - np.uint64(1))
    cnt = np.array([bin(int(x)).count("1") for x in (mask & below)], dtype=np.uint64)
    vm.wv32(ins.ops[0], ((cnt + vm.rv32(ins.ops[2]).astype(np.uint64)) & np.uint64(MASK32)).astype(np.uint32))


@op("s_bcnt1_i32_b64")
def _s_bcnt1_i32_b64(vm, ins, prog):
    r = bin(vm.rs64(ins.ops[1])).count("1")
    vm.ws32(ins.ops[0], r)
    vm.scc = int(r != 0)


@op("v_readfirstlane_b32")
def _v_readfirstlane(vm, ins, prog):
    src = vm.rv32(ins.ops[1])
    mask = vm.exec_mask()
    lane = int(np.argmax(mask)) if mask.any() else 0
    vm.ws32(ins.ops[0], int(src[lane]))


@op("v_readlane_b32")
def _v_readlane(vm, ins, prog):
    """sdst = vsrc[lane]; the lane select is an SGPR or a constant (its low 6
    bits), and EXEC does not apply."""
    lane = vm.rs32(ins.ops[2]) & (WAVE - 1)
    vm.ws32(ins.ops[0], int(vm.regfile(ins.ops[1])[ins.ops[1].index][lane]))


@op("v_writelane_b32")
def _v_writelane(vm, ins, prog):
    """vdst[lane] = ssrc; the other lanes keep their value, EXEC does not apply
    (the compiler uses it to park scalar registers in vector lanes)."""
    lane = vm.rs32(ins.ops[2]) & (WAVE - 1)
    dst = ins.ops[0]
    vm.regfile(dst)[dst.index][lane] = np.uint32(vm.rs32(ins.ops[1]))


@op("v_lshl_add_u64")
def _v_lshl_add_u64(vm, ins, prog):
    a = vm.rv64(ins.ops[1])
    sh = vm.rv32(ins.ops[2]).astype(np.uint64) & np.uint64(63)
    c = vm.rv64(ins.ops[3])
    vm.wv64(ins.ops[0], (a << sh) + c)


@op("v_mov_b64", "v_mov_b64_e32", "v_mov_b64_e64")
def _v_mov_b64(vm, ins, prog):
    vm.wv64(ins.ops[0], vm.rv64(ins.ops[1]))


@op("v_lshlrev_b64", "v_lshlrev_b64_e64")
def _v_lshlrev_b64(vm, ins, prog):
    sh = vm.rv32(ins.ops[1]).astype(np.uint64) & np.uint64(63)
    vm.wv64(ins.ops[0], vm.rv64(ins.ops[2]) << sh)


@op("v_mad_u64_u32")
def _v_mad_u64_u32(vm, ins, prog):
    a = vm.rv32(ins.ops[2]).astype(object)
    b = vm.rv32(ins.ops[3]).astype(object)
    c = vm.rv64(ins.ops[4]).astype(object)
    full = a * b + c
    res = np.array([int(x) & MASK64 for x in full], dtype=np.uint64)
    carry = np.array([int(x) >> 64 for x in full]) != 0
    vm.wv64(ins.ops[0], res)
    if ins.ops[1].kind in ("s", "vcc"):
        vm.ws64(ins.ops[1], GcnVirtualMachine._bits(carry & vm.exec_mask()))


def _vcmp(name, fn, is_float=False, signed=False):
    def _impl(vm, ins, prog):
        if len(ins.ops) == 3:
            dst, a, b = ins.ops
        else:
            dst, (a, b) = Operand("vcc", text="vcc"), ins.ops
        x, y = vm.rv32(a), vm.rv32(b)
        if is_float:
            x, y = _f32(x), _f32(y)
        elif signed:
            x, y = x.view(np.int32), y.view(np.int32)
        with np.errstate(invalid="ignore"):
            res = fn(x, y) & vm.exec_mask()
        bits = GcnVirtualMachine._bits(res)
        if dst.kind in ("s", "vcc", "exec"):
            vm.ws64(dst, bits)
        else:
            raise NotImplementedError(f"compare destination {dst}")
    for suffix in ("_e32", "_e64"):
        _DISPATCH[name + suffix] = _impl


for _n, _f in (("eq", np.equal), ("ne", np.not_equal), ("lt", np.less), ("le", np.less_equal),
               ("gt", np.greater), ("ge", np.greater_equal)):
    _vcmp(f"v_cmp_{_n}_u32", _f)
    _vcmp(f"v_cmp_{_n}_i32", _f, signed=True)
def _vcmp64(name, fn, signed=False):
    def _impl(vm, ins, prog):
        if len(ins.ops) == 3:
            dst, a, b = ins.ops
        else:
            dst, (a, b) = Operand("vcc", text="vcc"), ins.ops
        x, y = vm.rv64(a), vm.rv64(b)
        if signed:
            x, y = x.view(np.int64), y.view(np.int64)
        res = fn(x, y) & vm.exec_mask()
        vm.ws64(dst, GcnVirtualMachine._bits(res))
    for suffix in ("_e32", "_e64"):
        _DISPATCH[name + suffix] = _impl


for _n, _f in (("eq", np.equal), ("ne", np.not_equal), ("lt", np.less), ("le", np.less_equal),
               ("gt", np.greater), ("ge", np.greater_equal)):
    _vcmp64(f"v_cmp_{_n}_u64", _f)
    _vcmp64(f"v_cmp_{_n}_i64", _f, signed=True)
_vcmp("v_cmp_eq_f32", np.equal, True)
_vcmp("v_cmp_lt_f32", np.less, True)
_vcmp("v_cmp_gt_f32", np.greater, True)
_vcmp("v_cmp_neq_f32", lambda x, y: ~(x == y), True)  # unordered-or-not-equal
_vcmp("v_cmp_lg_f32", lambda x, y: (x < y) | (x > y), True)


# accumulation registers ----------------------------------------------------
@op("v_accvgpr_write_b32", "v_accvgpr_write")
def _acc_write(vm, ins, prog):
    vm.wv32(ins.ops[0], vm.rv32(ins.ops[1]))


@op("v_accvgpr_read_b32", "v_accvgpr_read")
def _acc_read(vm, ins, prog):
    vm.wv32(ins.ops[0], vm.rv32(ins.ops[1]))


@op("v_accvgpr_mov_b32")
def _acc_mov(vm, ins, prog):
    vm.wv32(ins.ops[0], vm.rv32(ins.ops[1]))


def _mfma(m, n, kk, slots):
    def _impl(vm, ins, prog):
        dst, sa, sb, sc = ins.ops[:4]
        if any(k in ins.mods for k in ("cbsz", "abid", "blgp")):
            raise NotImplementedError(f"MFMA broadcast modifiers in {ins}")
        av = _f32(vm.rv32(sa)).astype(np.float64)
        bv = _f32(vm.rv32(sb)).astype(np.float64)
        A = av.reshape(kk, m).T          # A[i][k] = lane i + m*k
        B = bv.reshape(kk, n)            # B[k][j] = lane j + n*k
        rows, cols = _ACC_INDEX[m]
        if sc.kind == "imm":
            C = np.full((m, n), _f32(np.array([sc.value & MASK32], dtype=np.uint32))[0], dtype=np.float64)
        else:
            C = np.zeros((m, n))
            C[rows, cols] = _f32(vm.reg_block(sc)[:slots].copy())
        D = (A @ B + C).astype(np.float32)
        out = _u32(np.ascontiguousarray(D[rows, cols]))
        mask = vm.exec_mask()
        blk = vm.reg_block(dst)
        if not mask.all():
            raise NotImplementedError("MFMA under a partial EXEC mask")
        blk[:, :] = out
    return _impl


_DISPATCH["v_mfma_f32_32x32x2_f32"] = _DISPATCH["v_mfma_f32_32x32x2f32"] = _mfma(32, 32, 2, 16)
_DISPATCH["v_mfma_f32_16x16x4_f32"] = _DISPATCH["v_mfma_f32_16x16x4f32"] = _mfma(16, 16, 4, 4)


# global memory -------------------------------------------------------------
def _global_addr(vm, ins, vaddr_op, saddr_op):
    """Per-lane 64-bit address: vaddr (64-bit), or saddr (64-bit SGPR pair) plus
    the zero-extended 32-bit vaddr, plus the signed instruction offset, all
    modulo 2^64 as in the hardware.  A base outside the memory (a K tile's base
    before the matrix, say) is fine as long as the active lanes' sums land
    inside; the memory's range check judges those."""
    off = np.uint64(_sext(ins.mods.get("offset", 0), 32) & MASK64)
    if saddr_op is None or saddr_op.kind == "off":
        addr = vm.rv64(vaddr_op).astype(np.uint64)
    else:
        addr = np.uint64(vm.rs64(saddr_op) & MASK64) + vm.rv32(vaddr_op).astype(np.uint64)
    with np.errstate(over="ignore"):
        return (addr + off).astype(np.uint64)


def _global_load(nd):
    def _impl(vm, ins, prog):
        dst, vaddr = ins.ops[0], ins.ops[1]
        saddr = ins.ops[2] if len(ins.ops) > 2 else None
        mask = vm.exec_mask()
        addr = _global_addr(vm, ins, vaddr, saddr)
        data = np.zeros((nd, WAVE), dtype=np.uint32)
        if mask.any():
            data[:, mask] = vm.vmem.read_u32(addr[mask], nd, str(ins))

        def land():
            for i in range(nd):
                vm.regfile(dst)[dst.index + i][mask] = data[i][mask]
        vm.pending["vmcnt"].append(land)
    return _impl


def _global_store(nd):
    def _impl(vm, ins, prog):
        vaddr, src = ins.ops[0], ins.ops[1]
        saddr = ins.ops[2] if len(ins.ops) > 2 else None
        mask = vm.exec_mask()
        if not mask.any():
            return
        addr = _global_addr(vm, ins, vaddr, saddr)
        data = np.stack([vm.regfile(src)[src.index + i] for i in range(nd)])
        vm.vmem.write_u32(addr[mask], data[:, mask], str(ins))
    return _impl


for _nd, _sfx in ((1, "dword"), (2, "dwordx2"), (3, "dwordx3"), (4, "dwordx4")):
    _DISPATCH[f"global_load_{_sfx}"] = _global_load(_nd)
    _DISPATCH[f"global_store_{_sfx}"] = _global_store(_nd)


# scratch (private) memory: register spills --------------------------------
PRIVATE_BYTES = 1 << 16  # per lane; far above any spill area the kernels use


def _scratch_offsets(vm, ins, vaddr_op, saddr_op):
    """Per-lane byte offset into the lane's private memory: the 32-bit vaddr
    and/or saddr when given (not ``off``) plus the instruction offset."""
    off = np.full(WAVE, ins.mods.get("offset", 0), dtype=np.int64)
    if vaddr_op is not None and vaddr_op.kind != "off":
        off = off + vm.rv32(vaddr_op).astype(np.int64)
    if saddr_op is not None and saddr_op.kind != "off":
        off = off + np.int64(vm.rs32(saddr_op))
    return off


def _private(vm):
    if getattr(vm, "private", None) is None:
        vm.private = np.zeros((WAVE, PRIVATE_BYTES // 4), dtype=np.uint32)
    return vm.private


def _scratch_check(off, nd, ins):
    if (off % 4).any() or (off < 0).any() or (off + 4 * nd > PRIVATE_BYTES).any():
        raise MemoryError(f"{ins}: scratch access outside [0, {PRIVATE_BYTES}) or unaligned")


def _scratch_load(nd):
    def _impl(vm, ins, prog):
        dst, vaddr, saddr = ins.ops[0], ins.ops[1], ins.ops[2]
        mask = vm.exec_mask()
        off = _scratch_offsets(vm, ins, vaddr, saddr)
        _scratch_check(off[mask], nd, ins)
        mem = _private(vm)
        lanes = np.nonzero(mask)[0]
        data = np.zeros((nd, WAVE), dtype=np.uint32)
        for i in range(nd):
            data[i, lanes] = mem[lanes, off[lanes] // 4 + i]

        def land():
            for i in range(nd):
                vm.regfile(dst)[dst.index + i][mask] = data[i][mask]
        vm.pending["vmcnt"].append(land)
    return _impl


def _scratch_store(nd):
    def _impl(vm, ins, prog):
        vaddr, src, saddr = ins.ops[0], ins.ops[1], ins.ops[2]
        mask = vm.exec_mask()
        off = _scratch_offsets(vm, ins, vaddr, saddr)
        _scratch_check(off[mask], nd, ins)
        mem = _private(vm)
        lanes = np.nonzero(mask)[0]
        for i in range(nd):
            mem[lanes, off[lanes] // 4 + i] = vm.regfile(src)[src.index + i][lanes]
        vm.pending["vmcnt"].append(lambda: None)
    return _impl


for _nd, _sfx in ((1, "dword"), (2, "dwordx2"), (3, "dwordx3"), (4, "dwordx4")):
    _DISPATCH[f"scratch_load_{_sfx}"] = _scratch_load(_nd)
    _DISPATCH[f"scratch_store_{_sfx}"] = _scratch_store(_nd)


@op("global_atomic_add")
def _global_atomic_add(vm, ins, prog):
    """32-bit atomic add, lanes in ascending order.  With sc0 (glc) the first
    operand is the destination of the pre-add values, which land at vmcnt."""
    ret = bool(ins.mods.get("sc0", 0) or ins.mods.get("glc", 0))
    ops = ins.ops[1:] if ret else ins.ops
    vaddr, src = ops[0], ops[1]
    saddr = ops[2] if len(ops) > 2 else None
    mask = vm.exec_mask()
    addr = _global_addr(vm, ins, vaddr, saddr)
    data = vm.rv32(src)
    old = np.zeros(WAVE, dtype=np.uint32)
    for lane in np.nonzero(mask)[0]:
        a = addr[lane:lane + 1]
        cur = vm.vmem.read_u32(a, 1, str(ins))[0, 0]
        old[lane] = cur
        vm.vmem.write_u32(a, np.array([[(int(cur) + int(data[lane])) & MASK32]], dtype=np.uint32), str(ins))
    if ret:
        dst = ins.ops[0]

        def land():
            vm.regfile(dst)[dst.index][mask] = old[mask]
        vm.pending["vmcnt"].append(land)
    else:
        vm.pending["vmcnt"].append(lambda: None)


def _buffer_addr(vm, ins, vaddr_op, srd_op, soff_op):
    """Byte addresses and offsets of a raw (stride 0) MUBUF access:
    base + (offen ? vaddr : 0) + soffset + offset.  The range check against
    num_records (word 2 of the resource) is per dword, as measured on gfx950:
    a multi-dword load returns its in-range dwords and 0 for the others, a
    store writes only its in-range dwords."""
    if ins.mods.get("idxen", 0):
        raise NotImplementedError(f"indexed buffer access {ins}")
    w = [int(vm.s[srd_op.index + i]) for i in range(4)]
    base = w[0] | ((w[1] & 0xFFFF) << 32)
    if (w[1] >> 16) & 0x3FFF:
        raise NotImplementedError(f"strided buffer resource in {ins}")
    num_records = w[2]
    off = vm.rv32(vaddr_op).astype(np.int64) if ins.mods.get("offen", 0) else np.zeros(WAVE, dtype=np.int64)
    off = off + np.int64(vm.rs32(soff_op)) + np.int64(ins.mods.get("offset", 0))
    # A sum past 32 bits (a "negative" register offset plus the instruction's
    # offset field) is not modelled: which of the wrapped and the unwrapped
    # offset the range check sees is not part of this machine's contract.
    if (off[vm.exec_mask()] >= (1 << 32)).any():
        raise NotImplementedError(f"{ins}: buffer offset sum past 32 bits")
    return np.int64(base) + off, off, num_records


def _buffer_load(nd):
    def _impl(vm, ins, prog):
        dst, vaddr, srd, soff = ins.ops[:4]
        addr, off, num = _buffer_addr(vm, ins, vaddr, srd, soff)
        data = np.zeros((nd, WAVE), dtype=np.uint32)
        for i in range(nd):  # per-dword range check
            mask = vm.exec_mask() & (off + 4 * (i + 1) <= num)
            if mask.any():
                data[i, mask] = vm.vmem.read_u32(addr[mask] + 4 * i, 1, str(ins))[0]
        emask = vm.exec_mask()

        def land():
            for i in range(nd):
                vm.regfile(dst)[dst.index + i][emask] = data[i][emask]
        vm.pending["vmcnt"].append(land)
    return _impl


def _buffer_store(nd):
    def _impl(vm, ins, prog):
        src, vaddr, srd, soff = ins.ops[:4]
        addr, off, num = _buffer_addr(vm, ins, vaddr, srd, soff)
        for i in range(nd):  # per-dword range check
            mask = vm.exec_mask() & (off + 4 * (i + 1) <= num)
            if mask.any():
                vm.vmem.write_u32(addr[mask] + 4 * i, vm.regfile(src)[src.index + i][mask][None, :], str(ins))
        vm.pending["vmcnt"].append(lambda: None)
    return _impl


for _nd, _sfx in ((1, "dword"), (2, "dwordx2"), (3, "dwordx3"), (4, "dwordx4")):
    _DISPATCH[f"buffer_load_{_sfx}"] = _buffer_load(_nd)
    _DISPATCH[f"buffer_store_{_sfx}"] = _buffer_store(_nd)


@op("buffer_wbl2", "buffer_inv")
def _cache_maintenance(vm, ins, prog):
    """L2 write-back / invalidate of the device-scope fences: the VM has one
    coherent memory, so they only count as outstanding vector-memory work."""
    vm.pending["vmcnt"].append(lambda: None)


# LDS -------------------------------------------------------------------------
def _ds_read(nd):
    def _impl(vm, ins, prog):
        dst, addr_op = ins.ops[0], ins.ops[1]
        mask = vm.exec_mask()
        addr = vm.rv32(addr_op).astype(np.int64) + ins.mods.get("offset", 0)
        data = np.zeros((nd, WAVE), dtype=np.uint32)
        if mask.any():
            data[:, mask] = vm.lds.read_u32(addr[mask], nd, str(ins))

        def land():
            for i in range(nd):
                vm.regfile(dst)[dst.index + i][mask] = data[i][mask]
        vm.pending["lgkmcnt"].append(land)
    return _impl


def _ds_read2(dwords_each, scale):
    def _impl(vm, ins, prog):
        dst, addr_op = ins.ops[0], ins.ops[1]
        mask = vm.exec_mask()
        base = vm.rv32(addr_op).astype(np.int64)
        unit = 4 * dwords_each * scale
        parts = []
        for key in ("offset0", "offset1"):
            a = base + ins.mods.get(key, 0) * unit
            d = np.zeros((dwords_each, WAVE), dtype=np.uint32)
            if mask.any():
                d[:, mask] = vm.lds.read_u32(a[mask], dwords_each, str(ins))
            parts.append(d)
        data = np.concatenate(parts, axis=0)

        def land():
            for i in range(2 * dwords_each):
                vm.regfile(dst)[dst.index + i][mask] = data[i][mask]
        vm.pending["lgkmcnt"].append(land)
    return _impl


def _ds_write(nd):
    def _impl(vm, ins, prog):
        addr_op, src = ins.ops[0], ins.ops[1]
        mask = vm.exec_mask()
        if not mask.any():
            return
        addr = vm.rv32(addr_op).astype(np.int64) + ins.mods.get("offset", 0)
        data = np.stack([vm.regfile(src)[src.index + i] for i in range(nd)])
        vm.lds.write_u32(addr[mask], data[:, mask], str(ins))
        vm.pending["lgkmcnt"].append(lambda: None)
    return _impl


def _ds_write2(dwords_each, scale):
    def _impl(vm, ins, prog):
        addr_op, s0, s1 = ins.ops[0], ins.ops[1], ins.ops[2]
        mask = vm.exec_mask()
        if not mask.any():
            return
        base = vm.rv32(addr_op).astype(np.int64)
        unit = 4 * dwords_each * scale
        for key, src in (("offset0", s0), ("offset1", s1)):
            a = base + ins.mods.get(key, 0) * unit
            data = np.stack([vm.regfile(src)[src.index + i] for i in range(dwords_each)])
            vm.lds.write_u32(a[mask], data[:, mask], str(ins))
        vm.pending["lgkmcnt"].append(lambda: None)
    return _impl


for _nd, _sfx in ((1, "b32"), (2, "b64"), (3, "b96"), (4, "b128")):
    _DISPATCH[f"ds_read_{_sfx}"] = _ds_read(_nd)
    _DISPATCH[f"ds_write_{_sfx}"] = _ds_write(_nd)


@op("ds_add_u32")
def _ds_add_u32(vm, ins, prog):
    """LDS atomic add without return: the active lanes' values are added in
    lane order (32-bit wrap-around), visible to later accesses at once."""
    addr_op, src = ins.ops[0], ins.ops[1]
    mask = vm.exec_mask()
    if mask.any():
        addr = vm.rv32(addr_op).astype(np.int64) + ins.mods.get("offset", 0)
        vals = vm.regfile(src)[src.index]
        for lane in np.nonzero(mask)[0]:
            a = np.array([addr[lane]])
            cur = int(vm.lds.read_u32(a, 1, str(ins))[0, 0])
            vm.lds.write_u32(a, np.array([[(cur + int(vals[lane])) & MASK32]], dtype=np.uint32), str(ins))
    vm.pending["lgkmcnt"].append(lambda: None)
_DISPATCH["ds_read2_b32"] = _ds_read2(1, 1)
_DISPATCH["ds_read2_b64"] = _ds_read2(2, 1)
_DISPATCH["ds_read2st64_b32"] = _ds_read2(1, 64)
_DISPATCH["ds_read2st64_b64"] = _ds_read2(2, 64)
_DISPATCH["ds_write2_b32"] = _ds_write2(1, 1)
_DISPATCH["ds_write2_b64"] = _ds_write2(2, 1)
_DISPATCH["ds_write2st64_b32"] = _ds_write2(1, 64)
_DISPATCH["ds_write2st64_b64"] = _ds_write2(2, 64)


# ------------------------------------------------------------ dispatching
def run_kernel(program, grid: Tuple[int, ...], workgroup_size: int, kernargs: bytes, vmem: Memory,
               max_instructions: int = 50_000_000, on_workgroup: Optional[Callable] = None,
               order: Optional[Sequence[Tuple[int, int, int]]] = None,
               preempt_seed: Optional[int] = None, preempt_rate: float = 1.0 / 16) -> int:
    """Runs every work-group of a grid (x fastest, then y, then z), each with
    its waves taking turns: a wave runs until it reaches a barrier (released
    once every live wave of the work-group waits there), yields at an
    ``s_sleep`` or ends; returns the number of instructions executed.
    ``order`` lists the (x, y, z) work-groups in the order to run them
    instead (each exactly once).  With ``preempt_seed`` a wave also loses its
    turn after any instruction with probability ``preempt_rate`` (seeded),
    so that waves synchronising through LDS are checked under many
    interleavings, not just the one the turn order gives."""
    rng = np.random.default_rng(preempt_seed) if preempt_seed is not None else None
    preempt = (lambda: rng.random() < preempt_rate) if rng is not None else None
    prog = as_program(program)
    desc = prog.desc
    if not desc.get("amdhsa_user_sgpr_kernarg_segment_ptr", 0):
        raise NotImplementedError("kernel without a kernarg segment pointer")
    for key in ("amdhsa_user_sgpr_dispatch_ptr", "amdhsa_user_sgpr_queue_ptr", "amdhsa_user_sgpr_dispatch_id",
                "amdhsa_system_vgpr_workitem_id"):
        if desc.get(key, 0):
            raise NotImplementedError(f"kernel descriptor field {key} = {desc[key]}")
    gx, gy = grid[0], grid[1]
    gz = grid[2] if len(grid) > 2 else 1
    every = [(x, y, z) for z in range(gz) for y in range(gy) for x in range(gx)]
    if order is None:
        order = every
    elif sorted(order) != sorted(every):
        raise ValueError("order must list every work-group of the grid exactly once")
    user = desc.get("amdhsa_user_sgpr_count", 2)
    lds_size = desc.get("amdhsa_group_segment_fixed_size", 0)
    nwaves = (workgroup_size + WAVE - 1) // WAVE
    total = 0
    for (wx, wy, wz) in order:
        lds = Memory(max(lds_size, 4), "lds")
        # the kernel's whole declared kernarg segment, as the runtime allocates
        # it: bytes past the given image read as zeros
        smem = Memory(max(len(kernargs), desc.get("amdhsa_kernarg_size", 0), 8), "smem")
        smem.write_bytes(0, kernargs)
        waves = []
        for w in range(nwaves):
            vm = GcnVirtualMachine(nsgpr=max(desc.get("amdhsa_next_free_sgpr", 104) + 8, 104), nvgpr=512,
                                   vmem_bytes=8)
            vm.vmem, vm.smem, vm.lds = vmem, smem, lds
            vm.s[0] = 0
            vm.s[1] = 0
            sid = user
            if desc.get("amdhsa_system_sgpr_workgroup_id_x", 1):
                vm.s[sid] = wx
                sid += 1
            if desc.get("amdhsa_system_sgpr_workgroup_id_y", 0):
                vm.s[sid] = wy
                sid += 1
            if desc.get("amdhsa_system_sgpr_workgroup_id_z", 0):
                vm.s[sid] = wz
                sid += 1
            tid = np.arange(WAVE, dtype=np.uint32) + w * WAVE
            vm.v[0] = tid
            active = tid < workgroup_size
            vm.exec = GcnVirtualMachine._bits(active)
            vm.reset_wave()
            waves.append(vm)
        budget = max_instructions
        at_barrier = [False] * len(waves)
        while not all(vm.done for vm in waves):
            for i, vm in enumerate(waves):
                if vm.done or at_barrier[i]:
                    continue
                try:
                    vm.step(prog, budget, preempt)
                except BarrierReached:
                    at_barrier[i] = True
                except Yielded:
                    pass
            live = [i for i, vm in enumerate(waves) if not vm.done]
            waiting = [i for i in live if at_barrier[i]]
            if waiting and len(live) != len(waves):
                raise RuntimeError("a wave ended while others wait at a barrier")
            if live and len(waiting) == len(live):
                at_barrier = [False] * len(waves)  # every live wave arrived: release
        total += sum(vm.executed for vm in waves)
        if on_workgroup:
            on_workgroup(wx, wy, waves)
    return total


def pack_kernargs(a: int, b: int, c: int, d: int, m: int, n: int, k: int, lda: int, ldb: int, ldc: int, ldd: int,
                  alpha: float, beta: float, nwgx: int, nwgy: int) -> bytes:
    """The reference's 15-argument image (generator_runner.cpp:132-148), padded to 80 bytes."""
    raw = struct.pack("<QQQQIIIIIIIffii", a, b, c, d, m, n, k, lda, ldb, ldc, ldd, alpha, beta, nwgx, nwgy)
    return raw + b"\0" * (80 - len(raw))


def pack_splitk_kernargs(base: bytes, ws: int, tickets: int, splits: int) -> bytes:
    """The split-K kernel's image: the 15 arguments (80 bytes), then ws at 80,
    tickets at 88 and splits at 96, padded to 104 bytes."""
    raw = base[:80] + struct.pack("<QQI", ws, tickets, splits)
    return raw + b"\0" * (104 - len(raw))


def pack_streamk_kernargs(base: bytes, ws: int, tickets: int, sk_tiles: int, groups: int) -> bytes:
    """The stream-K kernel's image: the 15 arguments (80 bytes), then ws at 80,
    tickets at 88, sk_tiles at 96 and groups at 100: 104 bytes."""
    return base[:80] + struct.pack("<QQII", ws, tickets, sk_tiles, groups)


def run_sgemm(program, tile: Tuple[int, int], workitems: int, A: np.ndarray, B: np.ndarray,
              C: Optional[np.ndarray] = None, alpha: float = 1.0, beta: float = 0.0,
              mnk: Optional[Tuple[int, int, int]] = None, ldd: Optional[int] = None,
              splits: int = 0, order: Optional[Sequence[Tuple[int, int, int]]] = None,
              misalign: int = 0, stream_k: Optional[Tuple[int, int]] = None,
              preempt_seed: Optional[int] = None) -> Tuple[np.ndarray, Dict]:
    """Runs a compiled SGEMM kernel on column-major A, B, C.

    Without ``mnk`` the problem is A (m x k) @ B (k x n) with tight leading
    dimensions.  With ``mnk = (m, n, k)`` the arrays are the full column-major
    storage: A is lda x (>= k), B is ldb x (>= n), C is ldc x (>= n), so
    lda = A.shape[0] etc.; D gets ``ldd`` rows (default m).  Returns D as the
    full ldd x n storage when ``mnk`` is given, else m x n.

    ``splits >= 1`` runs ``generated_gemm_splitk`` instead, over a grid of
    ``splits`` K ranges, with its workspace and zeroed tickets;
    ``stream_k = (groups, sk_tiles)`` runs ``generated_gemm_streamk`` over
    ``groups`` work-groups with ``sk_tiles`` stream-K tiles, its workspace of
    2 * groups partial tiles and ``groups`` zeroed tickets; ``order`` is the
    work-group order (see run_kernel).  The returned info holds the tickets
    after the launch.  ``misalign`` (a multiple of 4 below 16) moves the start
    of every buffer that many bytes past a 4 KiB boundary."""
    if misalign % 4 or not 0 <= misalign < 16:
        raise ValueError("misalign must be 0, 4, 8 or 12 bytes")
    A = np.asfortranarray(A, dtype=np.float32)
    B = np.asfortranarray(B, dtype=np.float32)
    if mnk is None:
        m, k = A.shape
        n = B.shape[1]
        lda, ldb = m, k
    else:
        m, n, k = mnk
        lda, ldb = A.shape[0], B.shape[0]
    Cm = np.zeros((m, n), dtype=np.float32, order="F") if C is None else np.asfortranarray(C, dtype=np.float32)
    ldc = Cm.shape[0]
    ldd = ldd or m
    nwgx, nwgy = (m + tile[0] - 1) // tile[0], (n + tile[1] - 1) // tile[1]
    blobs = [A.ravel(order="F"), B.ravel(order="F"), Cm.ravel(order="F"),
             np.zeros(ldd * n, dtype=np.float32)]
    if splits and stream_k:
        raise ValueError("a launch is split-K or stream-K, not both")
    if splits:
        blobs.append(np.full(nwgx * nwgy * splits * tile[0] * tile[1], np.nan, dtype=np.float32))
        blobs.append(np.zeros(nwgx * nwgy, dtype=np.uint32))
    if stream_k:
        blobs.append(np.full(stream_k[0] * 2 * tile[0] * tile[1], np.nan, dtype=np.float32))
        blobs.append(np.zeros(stream_k[0], dtype=np.uint32))
    # every buffer gets exactly its own bytes as an allocated region, with
    # unallocated gaps between them: any access past a buffer raises
    offs, pos = [], 4096
    for bl in blobs:
        offs.append(pos + misalign)
        pos += (bl.nbytes + misalign + 4095) // 4096 * 4096 + 4096
    mem = Memory(pos, "vmem")
    for o, bl, label in zip(offs, blobs, ["A", "B", "C", "D", "ws", "tickets"]):
        mem.write_bytes(o, bl.tobytes())
        mem.allocate_region(o, bl.nbytes, label)
    ka = pack_kernargs(offs[0], offs[1], offs[2], offs[3], m, n, k, lda, ldb, ldc, ldd, alpha, beta, nwgx, nwgy)
    info: Dict = {}
    if splits:
        ka = pack_splitk_kernargs(ka, offs[4], offs[5], splits)
        grid: Tuple[int, ...] = (nwgx, nwgy, splits)
        prog = as_program(program, "generated_gemm_splitk")
    elif stream_k:
        ka = pack_streamk_kernargs(ka, offs[4], offs[5], stream_k[1], stream_k[0])
        grid = (stream_k[0], 1, 1)
        prog = as_program(program, "generated_gemm_streamk")
    else:
        grid = (nwgx, nwgy)
        prog = as_program(program)
    count = run_kernel(prog, grid, workitems, ka, mem, order=order, preempt_seed=preempt_seed)
    D = np.frombuffer(mem.read_bytes(offs[3], ldd * n * 4), dtype=np.float32).reshape(n, ldd).T.copy()
    if mnk is None:
        D = D[:m, :]
    if splits:
        info["tickets"] = np.frombuffer(mem.read_bytes(offs[5], nwgx * nwgy * 4), dtype=np.uint32).copy()
    if stream_k:
        info["tickets"] = np.frombuffer(mem.read_bytes(offs[5], stream_k[0] * 4), dtype=np.uint32).copy()
    info.update({"instructions": count, "grid": grid, "d_offset": offs[3], "memory": mem})
    return D, info
