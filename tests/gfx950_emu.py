"""An instruction-level emulator of the gfx950 code the library's kernels compile to, for tests on machines without
a GPU.  It runs the assembly hipcc emits (tests/isa_waits.compile_asm) for one workgroup after another; within a
workgroup the waves run in turn, each until it reaches a barrier or ends.

What it models, and why that is enough for the kernels it runs here:
  * 64-lane waves: scalar registers (with VCC, EXEC, M0, SCC), vector registers, per-lane private memory (scratch),
    the workgroup's LDS, and a flat device address space of the buffers the test allocates;
  * vector-memory operations complete out of program order with respect to everything else: a load, an atomic with
    return, or a buffer-to-LDS copy stays pending until an `s_waitcnt vmcnt(n)` retires it (oldest first, the
    counter's order).  Touching a pending load's destination register, or LDS bytes a pending copy will write, is an
    error (EmuError): the emulator finds the missing waits that the hardware would turn into wrong results.  Stores
    take effect at once and occupy their place in the counter's order;
  * workgroups run one after another, each to its end.  Kernels whose workgroups hand work to whichever arrives last
    (counters and partial results in device memory) are correct under this order as under any other;
  * arithmetic is exact where the hardware's is: integer ops bit for bit, fp32/fp64 with IEEE round-to-nearest-even
    and denormals kept (the library is built with denormals on), fused multiply-adds rounded once.  The reciprocal
    instructions return the correctly rounded reciprocal, which is within the hardware's documented error; they
    appear only in the compiler's integer-division sequences, whose final correction steps make the quotient exact
    for any reciprocal within that error.
  * MFMA v_mfma_i32_32x32x32_i8 with the operand and result layouts of the CDNA3/CDNA4 instruction set reference:
    A and B lane l hold row / column l % 32 and k bytes 16 (l / 32) .. + 15; D[i][j] sits in lane j + 32 ((i / 4) % 2),
    register 4 (i / 8) + i % 4.
  * buffer instructions with raw (stride 0) resources: the per-lane offset plus the instruction offset is checked
    against num_records per dword (out of range: loads return 0, stores are dropped); the scalar offset is added
    unchecked.  A copy into LDS writes lane l's bytes at M0 + instruction offset + l * size.
Only the instructions the library's kernels use are implemented; any other raises EmuError, so that a kernel that
compiles to something new fails loudly rather than running on a guess.
"""
import re
from fractions import Fraction

import os

import numpy as np

MASK32 = 0xFFFFFFFF
MASK64 = (1 << 64) - 1
LANES = np.arange(64)
INLINE_F32 = {'0.5': 0x3F000000, '-0.5': 0xBF000000, '1.0': 0x3F800000, '-1.0': 0xBF800000, '2.0': 0x40000000,
              '-2.0': 0xC0000000, '4.0': 0x40800000, '-4.0': 0xC0800000, '0.15915494': 0x3E22F983}
INLINE_F64 = {'0.5': 0x3FE0000000000000, '-0.5': 0xBFE0000000000000, '1.0': 0x3FF0000000000000,
              '-1.0': 0xBFF0000000000000, '2.0': 0x4000000000000000, '-2.0': 0xC000000000000000,
              '4.0': 0x4010000000000000, '-4.0': 0xC010000000000000, '0.15915494': 0x3FC45F306DC9C882}
SPECIAL = {'vcc': (106, 2), 'vcc_lo': (106, 1), 'vcc_hi': (107, 1), 'exec': (126, 2), 'exec_lo': (126, 1),
           'exec_hi': (127, 1), 'm0': (124, 1)}


class EmuError(Exception):
    pass


_LANE_MASKS = {}            # EXEC value -> per-lane bools (read-only, shared)


# ------------------------------------------------------------------------------------------------ device memory
class Memory:
    """The device address space: numpy byte buffers, each at its own host address (so addresses never collide, and
    host code that copies into a buffer through its address -- the emulated runtime's memcpy -- is seen by the
    kernels)."""

    def __init__(self):
        self.bufs = []              # (base, array)

    def alloc(self, nbytes, data=None):
        """A zeroed buffer of nbytes at a 256-byte aligned address (filled from data when given)."""
        n = max(int(nbytes), 1)
        raw_arr = np.zeros(n + 256, np.uint8)
        shift = (-raw_arr.ctypes.data) % 256
        arr = raw_arr[shift:shift + n]
        if data is not None:
            raw = np.frombuffer(np.ascontiguousarray(data).tobytes(), np.uint8)
            arr[:raw.size] = raw
        base = arr.ctypes.data
        self.bufs.append((base, arr))
        return base

    def release(self, base):
        self.bufs = [b for b in self.bufs if b[0] != base]

    def find(self, addr, n):
        for base, arr in self.bufs:
            if base <= addr and addr + n <= base + arr.size:
                return arr, addr - base
        raise EmuError(f'device access of {n} bytes at {addr:#x} outside every allocation')

    def read(self, addr, n):
        arr, off = self.find(addr, n)
        return arr[off:off + n].copy()

    def write(self, addr, data):
        data = np.asarray(data, np.uint8)
        arr, off = self.find(addr, data.size)
        arr[off:off + data.size] = data

    def gather(self, addr, size, mask):
        """(64, size) bytes at addr[l] .. + size for the lanes in mask (others 0)."""
        out = np.zeros((64, size), np.uint8)
        lanes = np.nonzero(mask)[0]
        if lanes.size == 0:
            return out
        a = addr[lanes].astype(np.int64)
        lo, hi = int(a.min()), int(a.max()) + size
        try:
            arr, off = self.find(lo, hi - lo)
        except EmuError:                       # lanes in different buffers (Parts outputs): one at a time
            for l in lanes:
                out[l] = self.read(int(addr[l]), size)
            return out
        out[lanes] = arr[(a - lo + off)[:, None] + np.arange(size)]
        return out

    def scatter(self, addr, data, mask):
        lanes = np.nonzero(mask)[0]
        if lanes.size == 0:
            return
        size = data.shape[1]
        a = addr[lanes].astype(np.int64)
        lo, hi = int(a.min()), int(a.max()) + size
        try:
            arr, off = self.find(lo, hi - lo)
        except EmuError:
            for l in lanes:
                self.write(int(addr[l]), data[l])
            return
        arr[(a - lo + off)[:, None] + np.arange(size)] = data[lanes]

    def array(self, base, dtype, count):
        arr, off = self.find(base, np.dtype(dtype).itemsize * count)
        return arr[off:off + np.dtype(dtype).itemsize * count].view(dtype)


# ------------------------------------------------------------------------------------------------ parsing
def split_operands(text):
    """Comma-separated operands (brackets kept whole) and the space-separated modifiers after the last one."""
    parts, depth, cur = [], 0, ''
    for ch in text:
        if ch in '([':
            depth += 1
        elif ch in ')]':
            depth -= 1
        if ch == ',' and depth == 0:
            parts.append(cur.strip())
            cur = ''
        else:
            cur += ch
    if cur.strip():
        parts.append(cur.strip())
    mods = {}
    if parts:
        toks = parts[-1].split()
        # a lone modifier list (s_waitcnt vmcnt(0) lgkmcnt(0)) has no operand
        first_is_mod = re.match(r'^(vmcnt|lgkmcnt|expcnt)\(', toks[0]) is not None
        if first_is_mod:
            parts = parts[:-1]
            rest = toks
        else:
            parts[-1] = toks[0]
            rest = toks[1:]
        for t in rest:
            if ':' in t:
                k, v = t.split(':', 1)
                mods[k] = v
            else:
                m = re.match(r'^(\w+)\((\d+)\)$', t)
                if m:
                    mods[m.group(1)] = int(m.group(2))
                else:
                    mods[t] = True
    return parts, mods


def parse_int(s):
    s = s.strip()
    neg = s.startswith('-')
    if neg:
        s = s[1:]
    v = int(s, 16) if s.lower().startswith('0x') else int(s)
    return -v if neg else v


class Op:
    """A decoded operand: kind 'v' / 's' (register base and count), 'lit' (integer bits or inline float name),
    'off', with neg / abs float modifiers."""
    __slots__ = ('kind', 'base', 'n', 'value', 'neg', 'abs', 'text')

    def __init__(self, text):
        self.text = text
        self.neg = self.abs = False
        t = text
        if t.startswith('neg(') and t.endswith(')'):
            self.neg, t = True, t[4:-1]
        if t.startswith('abs(') and t.endswith(')'):
            self.abs, t = True, t[4:-1]
        if t.startswith('-') and re.match(r'^-[vs\[|]', t):
            self.neg, t = True, t[1:]
        if t.startswith('|') and t.endswith('|'):
            self.abs, t = True, t[1:-1]
        self.base = self.n = self.value = None
        m = re.match(r'^([vsa])(?:\[(\d+):(\d+)\]|(\d+))$', t)
        if m:
            self.kind = 'v' if m.group(1) == 'v' else ('s' if m.group(1) == 's' else 'a')
            if m.group(4) is not None:
                self.base, self.n = int(m.group(4)), 1
            else:
                self.base, self.n = int(m.group(2)), int(m.group(3)) - int(m.group(2)) + 1
            if self.kind == 'a':
                raise EmuError('AGPR operands are not modelled')
        elif t in SPECIAL:
            self.kind = 's'
            self.base, self.n = SPECIAL[t]
        elif t in ('src_shared_base', 'src_private_base'):
            # apertures of LDS and scratch in the flat address space: the high word identifies the segment
            self.kind, self.value = 'lit', 0x1000000000000 if t == 'src_shared_base' else 0x2000000000000
        elif t == 'scc':
            self.kind = 'scc'
        elif t == 'off':
            self.kind = 'off'
        elif t in INLINE_F32:
            self.kind, self.value = 'flt', t
        elif re.match(r'^-?(0x[0-9a-fA-F]+|\d+)$', t):
            self.kind, self.value = 'lit', parse_int(t)
        else:
            raise EmuError(f'operand {text!r} not understood')


class Instr:
    __slots__ = ('mn', 'ops', 'mods', 'text', 'fn', 'target')

    def __init__(self, mn, rest):
        self.mn = re.sub(r'_e(32|64)$', '', mn)          # the encoding size does not change what an op does
        self.text = (mn + ' ' + rest).strip()
        parts, self.mods = split_operands(rest) if rest else ([], {})
        self.ops = parts
        self.fn = None
        self.target = None


class Program:
    """One kernel's instructions, labels and dispatch metadata, from hipcc's assembly."""

    @classmethod
    def from_lines(cls, lines, lds_bytes=0, private_bytes=0):
        """A program from bare instruction lines (tests of the emulator itself): no arguments, the kernarg pointer in
        s[0:1] and the workgroup id in s2 as for the library's kernels."""
        p = cls.__new__(cls)
        p.name, p.lds_bytes, p.private_bytes = 'snippet', lds_bytes, private_bytes
        p.user_sgprs, p.kernarg_size, p.args, p.hidden, p.wg_id_y, p.wg_id_z = 2, 8, [], [], 0, 0
        p.instrs, labels = [], {}
        for line in lines:
            s = line.split(';')[0].strip()
            if not s:
                continue
            if re.match(r'^\.?L\w+:$', s):
                labels[s[:-1]] = len(p.instrs)
                continue
            parts = s.split(None, 1)
            p.instrs.append(Instr(parts[0], parts[1] if len(parts) > 1 else ''))
        p.finish(labels)
        return p

    def finish(self, labels):
        for ins in self.instrs:
            if ins.mn.startswith(('s_branch', 's_cbranch')):
                ins.target = labels[ins.ops[0]]
            elif ins.mn == 's_set_gpr_idx_on':
                ins.ops = [Op(ins.ops[0])]          # the gpr_idx(...) list is read from the text
            else:
                ins.ops = [Op(o) for o in ins.ops]
            ins.fn = handler(ins.mn)

    def __init__(self, asm, name_part):
        names = [n for n in re.findall(r'^([A-Za-z_][\w.$]*):', asm, re.M) if name_part in n and not n.startswith('.')]
        if len(names) != 1:
            raise EmuError(f'kernel {name_part!r}: {names}')
        self.name = names[0]
        body = asm.split(self.name + ':', 1)[1].split('.Lfunc_end', 1)[0]
        self.instrs, labels = [], {}
        for line in body.splitlines():
            s = line.split(';')[0].strip()
            if not s:
                continue
            if re.match(r'^\.?L\w+:$', s):
                labels[s[:-1]] = len(self.instrs)
                continue
            if s.startswith('.'):
                continue
            p = s.split(None, 1)
            self.instrs.append(Instr(p[0], p[1] if len(p) > 1 else ''))
        self.finish(labels)
        kd = asm.split('.amdhsa_kernel ' + self.name, 1)[1].split('.end_amdhsa_kernel', 1)[0]
        d = dict(re.findall(r'\.(amdhsa_\w+)\s+(\S+)', kd))
        self.lds_bytes = int(d['amdhsa_group_segment_fixed_size'])
        self.private_bytes = int(d['amdhsa_private_segment_fixed_size'])
        self.user_sgprs = int(d['amdhsa_user_sgpr_count'])
        self.wg_id_y = int(d.get('amdhsa_system_sgpr_workgroup_id_y', 0))
        self.wg_id_z = int(d.get('amdhsa_system_sgpr_workgroup_id_z', 0))
        for k in ('amdhsa_user_sgpr_dispatch_ptr', 'amdhsa_user_sgpr_queue_ptr', 'amdhsa_user_sgpr_dispatch_id',
                  'amdhsa_user_sgpr_kernarg_preload_length', 'amdhsa_system_sgpr_workgroup_info'):
            if int(d.get(k, 0)):
                raise EmuError(f'{k} is not modelled')
        if not int(d['amdhsa_user_sgpr_kernarg_segment_ptr']) or self.user_sgprs != 2:
            raise EmuError('expected the kernarg pointer as the only user SGPRs')
        self.kernarg_size = int(d['amdhsa_kernarg_size'])
        self.args, self.hidden = kernel_args(asm, self.name)

    def pack_args(self, values):
        """The kernarg segment for the kernel's explicit arguments in order: ints, addresses, or bytes for structs."""
        if len(values) != len(self.args):
            raise EmuError(f'{len(values)} arguments for {len(self.args)}')
        buf = bytearray(self.kernarg_size)
        for (off, size), v in zip(self.args, values):
            raw = bytes(v) if isinstance(v, (bytes, bytearray)) else int(v).to_bytes(size, 'little', signed=int(v) < 0)
            if len(raw) != size:
                raise EmuError(f'argument at {off}: {len(raw)} bytes for {size}')
            buf[off:off + size] = raw
        return bytes(buf)


def kernel_args(asm, name):
    """[(offset, size)] of a kernel's explicit arguments, from the code object metadata in the assembly."""
    import yaml
    m = re.search(r'\.amdgpu_metadata\n(.*?)\.end_amdgpu_metadata', asm, re.S)
    text = '\n'.join(l for l in m.group(1).replace('\t', '    ').splitlines() if l.strip() not in ('---', '...'))
    for k in yaml.safe_load(text)['amdhsa.kernels']:
        if k['.name'] == name:
            args = [a for a in k['.args'] if not a['.value_kind'].startswith('hidden_')]
            hidden = [(a['.offset'], a['.size'], a['.value_kind']) for a in k['.args']
                      if a['.value_kind'].startswith('hidden_')]
            return [(a['.offset'], a['.size']) for a in args], hidden
    raise EmuError(f'no metadata for {name}')


# ------------------------------------------------------------------------------------------------ wave state
class Wave:
    serials = 0

    def __init__(self, wg, wid, program):
        self.wg, self.wid, self.prog = wg, wid, program
        Wave.serials += 1
        self.serial = Wave.serials
        self.s = [0] * 128
        self.scc = 0
        self.v = np.zeros((512, 64), np.uint32)
        self.pc = 0
        self.done = False
        self.at_barrier = False
        self.queue = []                 # pending vector-memory operations, oldest first
        self.pending_v = {}             # vgpr -> count of pending writes
        self.priv = np.zeros((64, max(program.private_bytes, 4) + 64), np.uint8)
        self.gpr_idx = None

    # --- scalar access
    def sget(self, op, width=1):
        if op.kind == 's':
            if width == 1:
                return self.s[op.base]
            return self.s[op.base] | (self.s[op.base + 1] << 32)
        if op.kind == 'lit':
            return op.value & (MASK32 if width == 1 else MASK64)
        if op.kind == 'flt':
            return INLINE_F32[op.value] if width == 1 else INLINE_F64[op.value]
        if op.kind == 'scc':
            return self.scc
        raise EmuError(f'scalar operand {op.text}')

    def sset(self, op, val, width=1):
        if op.kind != 's':
            raise EmuError(f'scalar destination {op.text}')
        if width == 1:
            self.s[op.base] = val & MASK32
        else:
            self.s[op.base] = val & MASK32
            self.s[op.base + 1] = (val >> 32) & MASK32

    @property
    def exec(self):
        return self.s[126] | (self.s[127] << 32)

    @exec.setter
    def exec(self, v):
        self.s[126], self.s[127] = v & MASK32, (v >> 32) & MASK32

    def lanes(self):
        e = self.exec
        m = _LANE_MASKS.get(e)
        if m is None:
            m = ((np.uint64(e) >> LANES.astype(np.uint64)) & np.uint64(1)).astype(bool)
            m.flags.writeable = False
            if len(_LANE_MASKS) < 4096:
                _LANE_MASKS[e] = m
        return m

    # --- vector access
    def check_v(self, base, n, what):
        for r in range(base, base + n):
            if self.pending_v.get(r):
                raise EmuError(f'wave {self.wid} pc {self.pc} ({self.prog.instrs[self.pc].text}): {what} v{r} '
                               f'while a load into it is pending')

    def vget(self, op, width=1):
        """(64,) uint32 for width 1, (64,) uint64 for width 2; abs / neg source modifiers act on the sign bit, as
        for the float operands they are defined on (VOP3 bit moves such as v_cndmask take them too)."""
        if op.kind == 'v':
            self.check_v(op.base, width, 'reads')
            if width == 1:
                x = self.v[op.base].copy()
            else:
                x = self.v[op.base].astype(np.uint64) | (self.v[op.base + 1].astype(np.uint64) << np.uint64(32))
        else:
            val = self.sget(op, width) if op.kind != 'lit' else (
                op.value & MASK32 if width == 1 else op.value & MASK64)
            x = np.full(64, val, np.uint32 if width == 1 else np.uint64)
        if op.abs or op.neg:
            sign = np.uint32(0x80000000) if width == 1 else np.uint64(1 << 63)
            if op.abs:
                x = x & ~sign
            if op.neg:
                x = x ^ sign
        return x

    def vset(self, op, val, width=1, mask=None):
        if op.kind != 'v':
            raise EmuError(f'vector destination {op.text}')
        self.check_v(op.base, width, 'writes')
        m = self.lanes() if mask is None else mask
        if width == 1:
            self.v[op.base][m] = np.asarray(val, np.uint32)[m] if np.ndim(val) else np.uint32(val)
        else:
            val = np.asarray(val, np.uint64)
            self.v[op.base][m] = (val & np.uint64(MASK32)).astype(np.uint32)[m]
            self.v[op.base + 1][m] = (val >> np.uint64(32)).astype(np.uint32)[m]

    def vset_regs(self, base, arr, mask):
        """arr: (64, n) uint32 into registers base .. base + n - 1 for the lanes in mask."""
        for i in range(arr.shape[1]):
            self.v[base + i][mask] = arr[mask, i]

    def fsrc(self, op, dtype=np.float32):
        if op.kind == 'flt':
            bits = INLINE_F32[op.value] if dtype == np.float32 else INLINE_F64[op.value]
            x = np.full(64, bits, np.uint32 if dtype == np.float32 else np.uint64).view(dtype)
        elif op.kind == 'lit' and dtype == np.float64:
            # inline integers -16..64 are bit patterns, sign-extended; any other 32-bit literal of a binary64 operand
            # is the value's high word
            v = op.value
            bits = v & MASK64 if -16 <= v <= 64 else (v & MASK32) << 32
            x = np.full(64, bits, np.uint64).view(np.float64)
        else:
            return self.vget(op, 1 if dtype == np.float32 else 2).view(dtype)      # modifiers applied there
        if op.abs:
            x = np.abs(x)
        if op.neg:
            x = -x
        return x


# ------------------------------------------------------------------------------------------------ helpers
def u32(x):
    return np.asarray(x, np.uint64).astype(np.uint32) if np.ndim(x) else np.uint32(int(x) & MASK32)


def i32(x):
    return np.asarray(x, np.uint32).view(np.int32)


def lanes_mask_bits(b):
    """(64,) bool -> 64-bit int."""
    return int(np.packbits(b[::-1].astype(np.uint8)).view('>u8')[0]) if b.size == 64 else 0


def bits_of(v):
    return ((int(v) >> LANES.astype(np.uint64).astype(object)) & 1).astype(bool) if False else \
        ((np.uint64(v) >> LANES.astype(np.uint64)) & np.uint64(1)).astype(bool)


def exact_fma(a, b, c, dtype):
    """a * b + c rounded once (round to nearest even)."""
    a, b, c = np.asarray(a, dtype), np.asarray(b, dtype), np.asarray(c, dtype)
    out = np.empty(64, dtype)
    with np.errstate(all='ignore'):
        if dtype == np.float32:
            # the product of two binary32 values is exact in binary64; s = RN64(p + c) with its exact error e (TwoSum).
            # RN32 of the exact sum differs from RN32(s) only when s is a binary32 midpoint and e != 0
            p = a.astype(np.float64) * b.astype(np.float64)
            c64 = c.astype(np.float64)
            s = p + c64
            bb = s - p
            e = (p - (s - bb)) + (c64 - bb)
            r = s.astype(np.float32)
            up, dn = np.nextafter(r, np.float32(np.inf)), np.nextafter(r, np.float32(-np.inf))
            fix = np.isfinite(s) & (e != 0)
            mid_up = fix & (s == (r.astype(np.float64) + up.astype(np.float64)) / 2)
            mid_dn = fix & (s == (r.astype(np.float64) + dn.astype(np.float64)) / 2)
            r = np.where(mid_up & (e > 0), up, r)
            r = np.where(mid_dn & (e < 0), dn, r)
            out[:] = r
            return out
        # binary64: exact when the product is (then one rounding of p + c); otherwise exact rational arithmetic
        p = a * b
        exact = np.isfinite(p) & (p == 0) | _product_exact(a, b, p)
        out[:] = p + c
    for k in np.nonzero(~exact)[0]:
        x, y, z = float(a[k]), float(b[k]), float(c[k])
        if not (np.isfinite(x) and np.isfinite(y) and np.isfinite(z)):
            out[k] = x * y + z
            continue
        out[k] = round_fraction(Fraction(x) * Fraction(y) + Fraction(z), dtype)
    return out


def _product_exact(a, b, p):
    """a * b == p exactly, by Dekker's splitting (error-free product in binary64)."""
    with np.errstate(all='ignore'):
        def split(x):
            t = x * 134217729.0
            hi = t - (t - x)
            return hi, x - hi
        ah, al = split(a)
        bh, bl = split(b)
        err = ((ah * bh - p) + ah * bl + al * bh) + al * bl
        return np.isfinite(p) & (err == 0) & (np.abs(a) < 1e300) & (np.abs(b) < 1e300)


def round_fraction(f, dtype):
    if f == 0:
        return dtype(0.0)
    d = float(f)                                  # correctly rounded to binary64
    if dtype == np.float64:
        return np.float64(d)
    with np.errstate(over='ignore'):
        c = np.float32(d)
    if not np.isfinite(c):          # past the largest binary32: infinity from 2^128 - 2^103 (its midpoint) on
        big = abs(f) >= Fraction(2 ** 128 - 2 ** 103)
        m = np.float32(np.inf) if big else np.finfo(np.float32).max
        return m if f > 0 else -m
    # correct a double rounding: pick the nearer binary32 neighbour of the exact value, ties to even
    lo = np.nextafter(c, np.float32(-np.inf)) if Fraction(float(c)) > f else c
    hi = np.nextafter(lo, np.float32(np.inf))
    dl, dh = abs(f - Fraction(float(lo))), abs(Fraction(float(hi)) - f)
    if dl < dh:
        return lo
    if dh < dl:
        return hi
    return lo if int(np.float32(lo).view(np.uint32)) % 2 == 0 else hi


# ------------------------------------------------------------------------------------------------ instructions
H = {}


def op(*names):
    def deco(f):
        for n in names:
            H[n] = f
        return f
    return deco


SDWA_OPS = {'v_and_b32': lambda a, b: a & b, 'v_or_b32': lambda a, b: a | b, 'v_xor_b32': lambda a, b: a ^ b,
            'v_lshrrev_b32': lambda a, b: b >> (a & S31), 'v_lshlrev_b32': lambda a, b: b << (a & S31),
            'v_mul_u32_u24': lambda a, b: (a & M24) * (b & M24), 'v_add_u32': lambda a, b: a + b}
SEL = {'DWORD': (0, 32), 'BYTE_0': (0, 8), 'BYTE_1': (8, 8), 'BYTE_2': (16, 8), 'BYTE_3': (24, 8), 'WORD_0': (0, 16),
       'WORD_1': (16, 16)}


def _sdwa(w, i):
    """Sub-dword addressing: each source's selected byte or word (zero-extended), the result's low bits placed at
    dst_sel with the rest of the register padded with 0 or preserved (dst_unused)."""
    f = SDWA_OPS[i.mn[:-5]]
    vals = []
    for k, key in ((1, 'src0_sel'), (2, 'src1_sel')):
        sh, nb = SEL[i.mods.get(key, 'DWORD')]
        if i.ops[k].neg or i.ops[k].abs:
            raise EmuError('sdwa source modifiers are not modelled')
        vals.append((w.vget(i.ops[k]).astype(np.uint64) >> np.uint64(sh)) & np.uint64((1 << nb) - 1))
    r = f(vals[0], vals[1]) & np.uint64(MASK32)
    sh, nb = SEL[i.mods.get('dst_sel', 'DWORD')]
    field = (r & np.uint64((1 << nb) - 1)) << np.uint64(sh)
    unused = i.mods.get('dst_unused', 'UNUSED_PAD')
    if nb < 32 and unused == 'UNUSED_PRESERVE':
        old = w.vget(i.ops[0]).astype(np.uint64)
        keep = np.uint64(MASK32 ^ (((1 << nb) - 1) << sh))
        field = field | (old & keep)
    elif nb < 32 and unused != 'UNUSED_PAD':
        raise EmuError(f'sdwa {unused} is not modelled')
    w.vset(i.ops[0], field)


def _dpp_src_lane(mods):
    """The source lane of each lane for the DPP controls the library's kernels use (rows of 16 lanes)."""
    l = LANES
    if 'quad_perm' in mods:
        perm = [int(x) for x in mods['quad_perm'].strip('[]').split(',')]
        return (l & ~3) + np.array(perm)[l & 3]
    if 'row_mirror' in mods:
        return (l & ~15) + (15 - (l & 15))
    if 'row_half_mirror' in mods:
        return (l & ~7) + (7 - (l & 7))
    raise EmuError(f'DPP control {mods} not modelled')


def _dpp(w, i):
    """src0 read from another lane of the row; a lane whose source lane is disabled reads 0 with bound_ctrl, else it
    is not written."""
    if i.mods.get('row_mask', '0xf') not in ('0xf', '15') or i.mods.get('bank_mask', '0xf') not in ('0xf', '15'):
        raise EmuError('DPP row or bank masks not modelled')
    src = _dpp_src_lane(i.mods)
    act = w.lanes()
    op0 = i.ops[1]
    vals = w.vget(op0)[src]
    src_on = act[src]
    bound = str(i.mods.get('bound_ctrl', '0')) in ('1', 'True')
    vals = np.where(src_on, vals, np.uint32(0))
    write = act & (src_on | bound)
    base = i.mn[:-4]
    if base == 'v_mov_b32':
        w.vset(i.ops[0], vals, mask=write)
    elif base == 'v_add_f32':
        with np.errstate(all='ignore'):
            r = (vals.view(np.float32) + w.fsrc(i.ops[2])).astype(np.float32)
        w.vset(i.ops[0], r.view(np.uint32), mask=write)
    elif base == 'v_max_f32':
        r = np.fmax(vals.view(np.float32), w.fsrc(i.ops[2])).astype(np.float32)
        w.vset(i.ops[0], r.view(np.uint32), mask=write)
    elif base == 'v_add_u32':
        w.vset(i.ops[0], (vals.astype(np.uint64) + w.vget(i.ops[2]).astype(np.uint64)).astype(np.uint32), mask=write)
    else:
        raise EmuError(f'{i.mn} not modelled')


@op('ds_bpermute_b32')
def _(w, i):
    act = w.lanes()
    addr = w.vget(i.ops[1]).astype(np.int64) + int(i.mods.get('offset', 0))
    data = w.vget(i.ops[2])
    src = (addr // 4) % 64
    tmp = np.where(act[src], data[src], np.uint32(0))
    w.vset(i.ops[0], tmp, mask=act)


def _cvt_sdwa(w, i):
    if i.mods.get('src0_sel', 'DWORD') != 'DWORD' or i.mods.get('dst_unused', 'UNUSED_PAD') != 'UNUSED_PAD':
        raise EmuError('sdwa conversion form not modelled')
    x = w.fsrc(i.ops[1]).astype(np.float64)
    r = np.where(np.isnan(x), 0, np.clip(np.trunc(x), -2 ** 31, 2 ** 31 - 1)).astype(np.int64) & MASK32
    sh, nb = SEL[i.mods.get('dst_sel', 'DWORD')]
    w.vset(i.ops[0], ((r & ((1 << nb) - 1)) << sh).astype(np.uint64))


def handler(mn):
    if mn.endswith('_sdwa') and mn[:-5] in SDWA_OPS:
        return _sdwa
    if mn == 'v_cvt_i32_f32_sdwa':
        return _cvt_sdwa
    if mn.endswith('_dpp') and mn[:-4] in ('v_mov_b32', 'v_add_f32', 'v_max_f32', 'v_add_u32'):
        return _dpp
    base = re.sub(r'_e(32|64)$', '', mn)
    if base in H:
        return H[base]
    if mn in H:
        return H[mn]
    raise EmuError(f'instruction {mn} is not modelled')


# --- scalar ALU
def _s2(w, i, f, width=1, scc=None):
    a, b = w.sget(i.ops[1], width), w.sget(i.ops[2], width)
    r = f(a, b)
    mask = MASK32 if width == 1 else MASK64
    w.sset(i.ops[0], r & mask, width)
    w.scc = int((r & mask) != 0) if scc is None else scc(a, b, r)


def sx32(x):
    x &= MASK32
    return x - (1 << 32) if x >> 31 else x


@op('s_mov_b32')
def _(w, i): w.sset(i.ops[0], w.sget(i.ops[1]))


@op('s_mov_b64')
def _(w, i): w.sset(i.ops[0], w.sget(i.ops[1], 2), 2)


@op('s_movk_i32')
def _(w, i): w.sset(i.ops[0], sx16(i.ops[1].value))


def sx16(v):
    v &= 0xFFFF
    return v - 0x10000 if v & 0x8000 else v


@op('s_add_u32')
def _(w, i):
    a, b = w.sget(i.ops[1]), w.sget(i.ops[2])
    w.sset(i.ops[0], a + b)
    w.scc = int(a + b > MASK32)


@op('s_addc_u32')
def _(w, i):
    a, b = w.sget(i.ops[1]), w.sget(i.ops[2])
    r = a + b + w.scc
    w.sset(i.ops[0], r)
    w.scc = int(r > MASK32)


@op('s_sub_u32')
def _(w, i):
    a, b = w.sget(i.ops[1]), w.sget(i.ops[2])
    w.sset(i.ops[0], a - b)
    w.scc = int(b > a)


@op('s_subb_u32')
def _(w, i):
    a, b = w.sget(i.ops[1]), w.sget(i.ops[2])
    w.sset(i.ops[0], a - b - w.scc)
    w.scc = int(b + w.scc > a)


@op('s_add_i32', 's_sub_i32')
def _(w, i):
    a, b = sx32(w.sget(i.ops[1])), sx32(w.sget(i.ops[2]))
    r = a + b if i.mn == 's_add_i32' else a - b
    w.sset(i.ops[0], r)
    w.scc = int(r != sx32(r))


@op('s_addk_i32')
def _(w, i):
    a = sx32(w.sget(i.ops[0]))
    r = a + sx16(i.ops[1].value)
    w.sset(i.ops[0], r)
    w.scc = int(r != sx32(r))


@op('s_mulk_i32')
def _(w, i): w.sset(i.ops[0], sx32(w.sget(i.ops[0])) * sx16(i.ops[1].value))


@op('s_mul_i32')
def _(w, i): w.sset(i.ops[0], w.sget(i.ops[1]) * w.sget(i.ops[2]))


@op('s_mul_hi_u32')
def _(w, i): w.sset(i.ops[0], (w.sget(i.ops[1]) * w.sget(i.ops[2])) >> 32)


@op('s_mul_hi_i32')
def _(w, i): w.sset(i.ops[0], (sx32(w.sget(i.ops[1])) * sx32(w.sget(i.ops[2]))) >> 32)


@op('s_min_i32')
def _(w, i):
    a, b = sx32(w.sget(i.ops[1])), sx32(w.sget(i.ops[2]))
    w.sset(i.ops[0], min(a, b))
    w.scc = int(a < b)


@op('s_abs_i32')
def _(w, i):
    r = abs(sx32(w.sget(i.ops[1]))) & MASK32
    w.sset(i.ops[0], r)
    w.scc = int(r != 0)


for _n, _f in (('and', lambda a, b: a & b), ('or', lambda a, b: a | b), ('xor', lambda a, b: a ^ b),
               ('andn2', lambda a, b: a & ~b), ('nor', lambda a, b: ~(a | b)), ('orn2', lambda a, b: a | ~b)):
    H[f's_{_n}_b32'] = (lambda f: lambda w, i: _s2(w, i, f))(_f)
    H[f's_{_n}_b64'] = (lambda f: lambda w, i: _s2(w, i, f, 2))(_f)


@op('s_lshl_b32')
def _(w, i): _s2(w, i, lambda a, b: a << (b & 31))


@op('s_lshr_b32')
def _(w, i): _s2(w, i, lambda a, b: a >> (b & 31))


@op('s_ashr_i32')
def _(w, i): _s2(w, i, lambda a, b: (sx32(a) >> (b & 31)) & MASK32)


@op('s_lshl_b64')
def _(w, i):
    a, b = w.sget(i.ops[1], 2), w.sget(i.ops[2])
    r = (a << (b & 63)) & MASK64
    w.sset(i.ops[0], r, 2)
    w.scc = int(r != 0)


@op('s_lshr_b64')
def _(w, i):
    a, b = w.sget(i.ops[1], 2), w.sget(i.ops[2])
    r = a >> (b & 63)
    w.sset(i.ops[0], r, 2)
    w.scc = int(r != 0)


@op('s_bfe_i64')
def _(w, i):
    a, b = w.sget(i.ops[1], 2), w.sget(i.ops[2])
    off, width = b & 63, (b >> 16) & 127
    if width == 0:
        r = 0
    else:
        r = (a >> off) & ((1 << width) - 1)
        if r >> (width - 1) & 1:
            r -= 1 << width
    r &= MASK64
    w.sset(i.ops[0], r, 2)
    w.scc = int(r != 0)


@op('s_max_u32')
def _(w, i):
    a, b = w.sget(i.ops[1]), w.sget(i.ops[2])
    w.sset(i.ops[0], max(a, b))
    w.scc = int(a > b)


@op('s_bfe_u32')
def _(w, i):
    a, b = w.sget(i.ops[1]), w.sget(i.ops[2])
    off, width = b & 31, (b >> 16) & 127
    r = (a >> off) & ((1 << width) - 1) if width else 0
    w.sset(i.ops[0], r)
    w.scc = int(r != 0)


@op('s_bitcmp1_b32')
def _(w, i): w.scc = (w.sget(i.ops[0]) >> (w.sget(i.ops[1]) & 31)) & 1


@op('s_not_b32')
def _(w, i):
    r = ~w.sget(i.ops[1]) & MASK32
    w.sset(i.ops[0], r)
    w.scc = int(r != 0)


@op('s_min_u32')
def _(w, i):
    a, b = w.sget(i.ops[1]), w.sget(i.ops[2])
    w.sset(i.ops[0], min(a, b))
    w.scc = int(a < b)


@op('s_max_i32')
def _(w, i):
    a, b = sx32(w.sget(i.ops[1])), sx32(w.sget(i.ops[2]))
    w.sset(i.ops[0], max(a, b))
    w.scc = int(a > b)


@op('s_ff1_i32_b64')
def _(w, i):
    v = w.sget(i.ops[1], 2)
    w.sset(i.ops[0], ((v & -v).bit_length() - 1) & MASK32 if v else MASK32)


@op('s_flbit_i32_b64')
def _(w, i):
    v = w.sget(i.ops[1], 2)
    w.sset(i.ops[0], 64 - v.bit_length() if v else MASK32)


@op('s_bitset1_b32')
def _(w, i): w.sset(i.ops[0], w.sget(i.ops[0]) | (1 << (w.sget(i.ops[1]) & 31)))


@op('s_bcnt1_i32_b64')
def _(w, i):
    r = bin(w.sget(i.ops[1], 2)).count('1')
    w.sset(i.ops[0], r)
    w.scc = int(r != 0)


@op('s_cselect_b32')
def _(w, i): w.sset(i.ops[0], w.sget(i.ops[1]) if w.scc else w.sget(i.ops[2]))


@op('s_cselect_b64')
def _(w, i): w.sset(i.ops[0], w.sget(i.ops[1], 2) if w.scc else w.sget(i.ops[2], 2), 2)


CMP = {'eq': lambda a, b: a == b, 'lg': lambda a, b: a != b, 'ne': lambda a, b: a != b, 'lt': lambda a, b: a < b,
       'le': lambda a, b: a <= b, 'gt': lambda a, b: a > b, 'ge': lambda a, b: a >= b}


def _scmp(w, i):
    m = re.match(r's_cmpk?_(\w+)_([iu])(32|64)$', i.mn)
    c, sign, bits = m.group(1), m.group(2), int(m.group(3))
    a = w.sget(i.ops[0], 1 if bits == 32 else 2)
    if i.mn.startswith('s_cmpk'):
        b = i.ops[1].value & 0xFFFF
        if sign == 'i':
            b = sx16(b)
    else:
        b = w.sget(i.ops[1], 1 if bits == 32 else 2)
    if sign == 'i':
        a, b = sx32(a), sx32(b) if not i.mn.startswith('s_cmpk') else b
    w.scc = int(CMP[c](a, b))


for _c in ('eq', 'lg', 'lt', 'le', 'gt', 'ge'):
    for _t in ('i32', 'u32'):
        H[f's_cmp_{_c}_{_t}'] = _scmp
        H[f's_cmpk_{_c}_{_t}'] = _scmp
H['s_cmp_eq_u64'] = H['s_cmp_lg_u64'] = _scmp


def _saveexec(f):
    def run(w, i):
        src = w.sget(i.ops[1], 2)
        old = w.exec
        w.sset(i.ops[0], old, 2)
        w.exec = f(src, old) & MASK64
        w.scc = int(w.exec != 0)
    return run


H['s_and_saveexec_b64'] = _saveexec(lambda s, e: s & e)
H['s_or_saveexec_b64'] = _saveexec(lambda s, e: s | e)
H['s_andn2_saveexec_b64'] = _saveexec(lambda s, e: s & ~e)


@op('s_nop', 's_setprio', 's_sleep')
def _(w, i): pass


@op('s_set_gpr_idx_on')
def _(w, i):
    """VGPR index mode: the operands named in gpr_idx(...) of the following vector instructions are offset by the
    index (the SGPR's low 8 bits) until s_set_gpr_idx_off."""
    m = re.search(r'gpr_idx\(([^)]*)\)', i.text)
    w.gpr_idx = (w.sget(i.ops[0]) & 0xFF, {x.strip() for x in m.group(1).split(',')})


@op('s_set_gpr_idx_off')
def _(w, i): w.gpr_idx = None


@op('s_waitcnt')
def _(w, i):
    n = None
    if i.ops and i.ops[0].kind == 'lit' and i.ops[0].value == 0:
        n = 0
    elif 'vmcnt' in i.mods:
        n = i.mods['vmcnt']
    if n is not None:
        while len(w.queue) > n:
            w.wg.retire(w, w.queue.pop(0))


@op('s_barrier')
def _(w, i): w.at_barrier = True


@op('s_endpgm')
def _(w, i):
    while w.queue:
        w.wg.retire(w, w.queue.pop(0))
    w.done = True


def _branch(cond):
    def run(w, i):
        if cond(w):
            w.pc = i.target - 1
    return run


H['s_branch'] = _branch(lambda w: True)
H['s_cbranch_scc0'] = _branch(lambda w: w.scc == 0)
H['s_cbranch_scc1'] = _branch(lambda w: w.scc == 1)
H['s_cbranch_vccz'] = _branch(lambda w: (w.s[106] | (w.s[107] << 32)) == 0)
H['s_cbranch_vccnz'] = _branch(lambda w: (w.s[106] | (w.s[107] << 32)) != 0)
H['s_cbranch_execz'] = _branch(lambda w: w.exec == 0)
H['s_cbranch_execnz'] = _branch(lambda w: w.exec != 0)


# --- scalar memory
@op('s_load_dword', 's_load_dwordx2', 's_load_dwordx4', 's_load_dwordx8', 's_load_dwordx16')
def _(w, i):
    n = {'s_load_dword': 1, 's_load_dwordx2': 2, 's_load_dwordx4': 4, 's_load_dwordx8': 8, 's_load_dwordx16': 16}[i.mn]
    base = w.sget(i.ops[1], 2)
    off = w.sget(i.ops[2]) if i.ops[2].kind == 's' else i.ops[2].value
    data = w.wg.mem.read(base + off, 4 * n).view(np.uint32)
    for k in range(n):
        w.s[i.ops[0].base + k] = int(data[k])


# --- vector ALU, 32-bit integer
def _v2(f):
    def run(w, i):
        a, b = w.vget(i.ops[1]).astype(np.uint64), w.vget(i.ops[2]).astype(np.uint64)
        w.vset(i.ops[0], f(a, b) & np.uint64(MASK32))
    return run


def _v3(f):
    def run(w, i):
        a, b, c = (w.vget(i.ops[k]).astype(np.uint64) for k in (1, 2, 3))
        w.vset(i.ops[0], f(a, b, c) & np.uint64(MASK32))
    return run


S31 = np.uint64(31)
M24 = np.uint64(0xFFFFFF)
H['v_add_u32'] = _v2(lambda a, b: a + b)
H['v_sub_u32'] = _v2(lambda a, b: a - b + np.uint64(1 << 32))
H['v_subrev_u32'] = _v2(lambda a, b: b - a + np.uint64(1 << 32))
H['v_and_b32'] = _v2(lambda a, b: a & b)
H['v_or_b32'] = _v2(lambda a, b: a | b)
H['v_xor_b32'] = _v2(lambda a, b: a ^ b)
H['v_lshlrev_b32'] = _v2(lambda a, b: b << (a & S31))
H['v_lshrrev_b32'] = _v2(lambda a, b: b >> (a & S31))
H['v_mul_u32_u24'] = _v2(lambda a, b: (a & M24) * (b & M24))
H['v_mul_lo_u32'] = _v2(lambda a, b: (a * b))
H['v_mul_hi_u32'] = _v2(lambda a, b: (a * b) >> np.uint64(32))
H['v_min_u32'] = _v2(lambda a, b: np.minimum(a, b))
H['v_max_u32'] = _v2(lambda a, b: np.maximum(a, b))
H['v_add3_u32'] = _v3(lambda a, b, c: a + b + c)
H['v_or3_b32'] = _v3(lambda a, b, c: a | b | c)
H['v_xad_u32'] = _v3(lambda a, b, c: (a ^ b) + c)
H['v_and_or_b32'] = _v3(lambda a, b, c: (a & b) | c)
H['v_lshl_or_b32'] = _v3(lambda a, b, c: ((a << (b & S31)) & np.uint64(MASK32)) | c)
H['v_lshl_add_u32'] = _v3(lambda a, b, c: ((a << (b & S31)) & np.uint64(MASK32)) + c)
H['v_mad_u32_u24'] = _v3(lambda a, b, c: (a & M24) * (b & M24) + c)
H['v_alignbit_b32'] = _v3(lambda a, b, c: ((a << np.uint64(32)) | b) >> (c & S31))
H['v_bfe_u32'] = _v3(lambda a, b, c: (a >> (b & S31)) & ((np.uint64(1) << (c & S31)) - np.uint64(1)))


def _v16(f):
    # 16-bit integer ops of the gfx9 family write the low half and zero the high half of the destination
    def run(w, i):
        a, b = (w.vget(i.ops[k]).astype(np.uint64) & np.uint64(0xFFFF) for k in (1, 2))
        w.vset(i.ops[0], f(a, b) & np.uint64(0xFFFF))
    return run


H['v_add_u16'] = _v16(lambda a, b: a + b)
H['v_sub_u16'] = _v16(lambda a, b: a - b + np.uint64(0x10000))
H['v_mul_lo_u16'] = _v16(lambda a, b: a * b)
H['v_lshlrev_b16'] = _v16(lambda a, b: b << (a & np.uint64(15)))
H['v_lshrrev_b16'] = _v16(lambda a, b: b >> (a & np.uint64(15)))


@op('v_not_b32')
def _(w, i): w.vset(i.ops[0], ~w.vget(i.ops[1]))


@op('v_bfrev_b32')
def _(w, i):
    a = w.vget(i.ops[1])
    r = np.zeros(64, np.uint32)
    for b in range(32):
        r |= ((a >> np.uint32(b)) & np.uint32(1)) << np.uint32(31 - b)
    w.vset(i.ops[0], r)


@op('v_bfe_i32')
def _(w, i):
    a = w.vget(i.ops[1]).astype(np.int64)
    off = (w.vget(i.ops[2]) & np.uint32(31)).astype(np.int64)
    wd = (w.vget(i.ops[3]) & np.uint32(31)).astype(np.int64)
    x = (a >> off) & ((np.int64(1) << wd) - 1)
    sgn = (wd > 0) & ((x >> np.maximum(wd - 1, 0)) & 1).astype(bool)
    x = np.where(sgn, x - (np.int64(1) << wd), x)
    w.vset(i.ops[0], (x & MASK32).astype(np.uint32))


@op('v_med3_i32')
def _(w, i):
    a, b, c = (i32(w.vget(i.ops[k])).astype(np.int64) for k in (1, 2, 3))
    w.vset(i.ops[0], np.median(np.stack([a, b, c]), axis=0).astype(np.int64).astype(np.int32).view(np.uint32))


@op('v_ffbh_i32')
def _(w, i):
    # first bit that differs from the sign bit, counted from the MSB; -1 (0xffffffff) for 0 and -1
    a = i32(w.vget(i.ops[1])).astype(np.int64)
    x = np.where(a < 0, ~a, a) & MASK32
    r = np.full(64, MASK32, np.uint64)
    nz = x != 0
    r[nz] = np.array([32 - int(v).bit_length() for v in x[nz]], np.uint64)
    w.vset(i.ops[0], r)


@op('v_ashrrev_i32')
def _(w, i):
    a, b = w.vget(i.ops[1]), i32(w.vget(i.ops[2]))
    w.vset(i.ops[0], (b >> (a & 31).astype(np.int32)).view(np.uint32))


@op('v_min_i32')
def _(w, i): w.vset(i.ops[0], np.minimum(i32(w.vget(i.ops[1])), i32(w.vget(i.ops[2]))).view(np.uint32))


@op('v_max_i32')
def _(w, i): w.vset(i.ops[0], np.maximum(i32(w.vget(i.ops[1])), i32(w.vget(i.ops[2]))).view(np.uint32))


@op('v_mul_hi_i32')
def _(w, i):
    a, b = i32(w.vget(i.ops[1])).astype(np.int64), i32(w.vget(i.ops[2])).astype(np.int64)
    w.vset(i.ops[0], ((a * b) >> 32).astype(np.uint64).astype(np.uint32))


@op('v_mov_b32')
def _(w, i): w.vset(i.ops[0], w.vget(i.ops[1]))


@op('v_mov_b64')
def _(w, i): w.vset(i.ops[0], w.vget(i.ops[1], 2), 2)


@op('v_ffbh_u32')
def _(w, i):
    a = w.vget(i.ops[1]).astype(np.uint64)
    r = np.full(64, MASK32, np.uint64)
    nz = a != 0
    r[nz] = np.uint64(31) - np.floor(np.log2(a[nz].astype(np.float64))).astype(np.uint64)
    # log2 of a 32-bit integer in binary64 is exact enough for its floor, except just below powers of two
    fix = nz & ((np.uint64(1) << (np.uint64(31) - r)) > a)
    r[fix] += np.uint64(1)
    w.vset(i.ops[0], r)


@op('v_perm_b32')
def _(w, i):
    a, b, sel = w.vget(i.ops[1]), w.vget(i.ops[2]), w.vget(i.ops[3])
    src = (a.astype(np.uint64) << np.uint64(32)) | b.astype(np.uint64)
    out = np.zeros(64, np.uint64)
    for k in range(4):
        s = ((sel >> np.uint32(8 * k)) & np.uint32(255)).astype(np.int64)
        byte = np.zeros(64, np.uint64)
        for v in range(8):
            byte = np.where(s == v, (src >> np.uint64(8 * v)) & np.uint64(255), byte)
        byte = np.where(s == 8, np.where((b >> np.uint32(15)) & np.uint32(1), 255, 0).astype(np.uint64), byte)
        byte = np.where(s == 9, np.where((b >> np.uint32(31)) & np.uint32(1), 255, 0).astype(np.uint64), byte)
        byte = np.where(s == 10, np.where((a >> np.uint32(15)) & np.uint32(1), 255, 0).astype(np.uint64), byte)
        byte = np.where(s == 11, np.where((a >> np.uint32(31)) & np.uint32(1), 255, 0).astype(np.uint64), byte)
        byte = np.where(s == 12, np.uint64(0), byte)
        byte = np.where(s >= 13, np.uint64(255), byte)
        out |= byte << np.uint64(8 * k)
    w.vset(i.ops[0], out)


@op('v_bitop3_b32')
def _(w, i):
    a, b, c = (w.vget(i.ops[k]) for k in (1, 2, 3))
    lut = parse_int(str(i.mods['bitop3']))
    out = np.zeros(64, np.uint32)
    for idx in range(8):
        if lut >> idx & 1:
            ta = a if idx & 4 else ~a
            tb = b if idx & 2 else ~b
            tc = c if idx & 1 else ~c
            out |= ta & tb & tc
    w.vset(i.ops[0], out)


@op('v_bitop3_b16')
def _(w, i):
    # the low halves; the high half of the destination is written as zero (16-bit ops of the gfx9 family)
    a, b, c = (w.vget(i.ops[k]) & np.uint32(0xFFFF) for k in (1, 2, 3))
    lut = parse_int(str(i.mods['bitop3']))
    out = np.zeros(64, np.uint32)
    for idx in range(8):
        if lut >> idx & 1:
            out |= (a if idx & 4 else ~a) & (b if idx & 2 else ~b) & (c if idx & 1 else ~c)
    w.vset(i.ops[0], out & np.uint32(0xFFFF))


@op('v_mbcnt_lo_u32_b32', 'v_mbcnt_hi_u32_b32')
def _(w, i):
    src, add = w.sget(i.ops[1]) if i.ops[1].kind != 'v' else None, w.vget(i.ops[2])
    if src is None:
        raise EmuError('v_mbcnt with a vector mask')
    hi = i.mn.startswith('v_mbcnt_hi')
    r = np.zeros(64, np.uint64)
    for l in range(64):
        k = (l - 32) if hi else l
        k = max(0, min(32, k))
        r[l] = bin(src & ((1 << k) - 1)).count('1')
    w.vset(i.ops[0], r + add.astype(np.uint64))


@op('v_readfirstlane_b32')
def _(w, i):
    a = w.vget(i.ops[1])
    m = w.lanes()
    lane = int(np.argmax(m)) if m.any() else 0
    w.sset(i.ops[0], int(a[lane]))


@op('v_readlane_b32')
def _(w, i):
    a = w.vget(i.ops[1])
    w.sset(i.ops[0], int(a[w.sget(i.ops[2]) & 63]))


@op('v_writelane_b32')
def _(w, i):
    lane = w.sget(i.ops[2]) & 63
    m = np.zeros(64, bool)
    m[lane] = True
    w.vset(i.ops[0], np.full(64, w.sget(i.ops[1]), np.uint32), mask=m)


# --- carries and compares
def carry_dst(w, i):
    return i.ops[1] if i.ops[1].kind == 's' else None


def set_mask(w, op_, bits):
    """Per-lane bools into an SGPR pair (VCC or another), inactive lanes 0."""
    val = 0
    act = w.lanes()
    b = bits & act
    for l in np.nonzero(b)[0]:
        val |= 1 << int(l)
    w.sset(op_, val, 2)


def get_mask(w, op_):
    v = w.sget(op_, 2)
    return ((np.uint64(v) >> LANES.astype(np.uint64)) & np.uint64(1)).astype(bool)


@op('v_sub_co_u32', 'v_subrev_co_u32', 'v_add_co_u32')
def _(w, i):
    a, b = w.vget(i.ops[2]).astype(np.int64), w.vget(i.ops[3]).astype(np.int64)
    if i.mn.startswith('v_subrev'):
        a, b = b, a
    if i.mn.startswith('v_add'):
        r, c = a + b, (a + b) > MASK32
    else:
        r, c = a - b, b > a
    w.vset(i.ops[0], (r & MASK32).astype(np.uint32))
    set_mask(w, i.ops[1], c)


@op('v_subb_co_u32', 'v_addc_co_u32', 'v_subbrev_co_u32')
def _(w, i):
    a, b = w.vget(i.ops[2]).astype(np.int64), w.vget(i.ops[3]).astype(np.int64)
    cin = get_mask(w, i.ops[4]).astype(np.int64)
    if i.mn.startswith('v_subbrev'):
        a, b = b, a
    if i.mn.startswith('v_addc'):
        r = a + b + cin
        c = r > MASK32
    else:
        r = a - b - cin
        c = (b + cin) > a
    w.vset(i.ops[0], (r & MASK32).astype(np.uint32))
    set_mask(w, i.ops[1], c)


@op('v_cndmask_b32')
def _(w, i):
    a, b = w.vget(i.ops[1]), w.vget(i.ops[2])
    m = get_mask(w, i.ops[3])
    w.vset(i.ops[0], np.where(m, b, a))


def _vcmp(w, i):
    m = re.match(r'v_cmp_(\w+?)_([iuf])(32|64)', i.mn)
    c, t, bits = m.group(1), m.group(2), int(m.group(3))
    wd = 1 if bits == 32 else 2
    a, b = w.vget(i.ops[1], wd), w.vget(i.ops[2], wd)
    if t == 'i':
        a, b = a.view(np.int32 if wd == 1 else np.int64), b.view(np.int32 if wd == 1 else np.int64)
    elif t == 'f':
        a, b = a.view(np.float32 if wd == 1 else np.float64), b.view(np.float32 if wd == 1 else np.float64)
    set_mask(w, i.ops[0], CMP[c](a, b))


for _c in ('eq', 'ne', 'lt', 'le', 'gt', 'ge', 'lg'):
    for _t in ('i32', 'u32', 'i64', 'u64', 'f32', 'f64'):
        H[f'v_cmp_{_c}_{_t}'] = _vcmp

# float compares: o / u (ordered / unordered) and the negated forms, true when either operand is NaN
FCMP = {'o': lambda a, b: ~(np.isnan(a) | np.isnan(b)), 'u': lambda a, b: np.isnan(a) | np.isnan(b),
        'nge': lambda a, b: ~(a >= b), 'nlg': lambda a, b: ~((a < b) | (a > b)), 'ngt': lambda a, b: ~(a > b),
        'nle': lambda a, b: ~(a <= b), 'neq': lambda a, b: ~(a == b), 'nlt': lambda a, b: ~(a < b)}


def _vfcmp(w, i):
    m = re.match(r'v_cmp_(\w+?)_f(32|64)$', i.mn)
    dt = np.float32 if m.group(2) == '32' else np.float64
    with np.errstate(invalid='ignore'):
        set_mask(w, i.ops[0], FCMP[m.group(1)](w.fsrc(i.ops[1], dt), w.fsrc(i.ops[2], dt)))


for _c in FCMP:
    H[f'v_cmp_{_c}_f32'] = H[f'v_cmp_{_c}_f64'] = _vfcmp


# --- 64-bit integer
@op('v_mad_u64_u32', 'v_mad_i64_i32')
def _(w, i):
    a, b = w.vget(i.ops[2]), w.vget(i.ops[3])
    c = w.vget(i.ops[4], 2)
    if i.mn == 'v_mad_u64_u32':
        prod = a.astype(np.uint64) * b.astype(np.uint64)           # exact: below 2^64
        res = prod + c                                             # modulo 2^64
        carry = res < prod
    else:
        prod = (i32(a).astype(np.int64) * i32(b).astype(np.int64)).view(np.uint64)
        res = prod + c
        carry = np.zeros(64, bool)
    w.vset(i.ops[0], res, 2)
    if i.ops[1].kind == 's':
        set_mask(w, i.ops[1], carry)


@op('v_lshlrev_b64')
def _(w, i):
    s, a = w.vget(i.ops[1]), w.vget(i.ops[2], 2)
    w.vset(i.ops[0], a << (s.astype(np.uint64) & np.uint64(63)), 2)


@op('v_lshrrev_b64')
def _(w, i):
    s, a = w.vget(i.ops[1]), w.vget(i.ops[2], 2)
    w.vset(i.ops[0], a >> (s.astype(np.uint64) & np.uint64(63)), 2)


@op('v_ashrrev_i64')
def _(w, i):
    s, a = w.vget(i.ops[1]), w.vget(i.ops[2], 2).view(np.int64)
    w.vset(i.ops[0], (a >> (s.astype(np.int64) & 63)).view(np.uint64), 2)


@op('v_lshl_add_u64')
def _(w, i):
    a, s, c = w.vget(i.ops[1], 2), w.vget(i.ops[2]), w.vget(i.ops[3], 2)
    w.vset(i.ops[0], (a << (s.astype(np.uint64) & np.uint64(63))) + c, 2)


# --- floating point
def _f2(f, dt=np.float32):
    def run(w, i):
        with np.errstate(all='ignore'):
            r = f(w.fsrc(i.ops[1], dt), w.fsrc(i.ops[2], dt)).astype(dt)
        w.vset(i.ops[0], r.view(np.uint32 if dt == np.float32 else np.uint64), 1 if dt == np.float32 else 2)
    return run


H['v_add_f32'] = _f2(lambda a, b: a + b)
H['v_mul_f32'] = _f2(lambda a, b: a * b)
H['v_sub_f32'] = _f2(lambda a, b: a - b)
H['v_max_f32'] = _f2(np.fmax)
H['v_min_f32'] = _f2(np.fmin)


H['v_add_f64'] = _f2(lambda a, b: a + b, np.float64)
H['v_mul_f64'] = _f2(lambda a, b: a * b, np.float64)
H['v_max_f64'] = _f2(np.fmax, np.float64)
H['v_min_f64'] = _f2(np.fmin, np.float64)
H['v_subrev_f32'] = _f2(lambda a, b: b - a)


@op('v_cvt_f64_f32')
def _(w, i): w.vset(i.ops[0], w.fsrc(i.ops[1]).astype(np.float64).view(np.uint64), 2)


@op('v_rndne_f64')
def _(w, i): w.vset(i.ops[0], np.rint(w.fsrc(i.ops[1], np.float64)).view(np.uint64), 2)


@op('v_rcp_f64')
def _(w, i):
    with np.errstate(all='ignore'):
        w.vset(i.ops[0], (1.0 / w.fsrc(i.ops[1], np.float64)).view(np.uint64), 2)


@op('v_cvt_i32_f64')
def _(w, i):
    x = w.fsrc(i.ops[1], np.float64)
    x = np.where(np.isnan(x), 0, np.clip(np.trunc(x), -2 ** 31, 2 ** 31 - 1))
    w.vset(i.ops[0], x.astype(np.int64).astype(np.int32).view(np.uint32))


@op('v_cvt_u32_f64')
def _(w, i):
    x = w.fsrc(i.ops[1], np.float64)
    x = np.where(np.isnan(x), 0, np.clip(np.trunc(x), 0, MASK32))
    w.vset(i.ops[0], x.astype(np.uint64).astype(np.uint32))


@op('v_fmac_f32', 'v_fmac_f64')
def _(w, i):
    dt = np.float32 if i.mn.endswith('f32') else np.float64
    a, b, c = w.fsrc(i.ops[1], dt), w.fsrc(i.ops[2], dt), w.fsrc(i.ops[0], dt)
    w.vset(i.ops[0], exact_fma(a, b, c, dt).view(np.uint32 if dt == np.float32 else np.uint64),
           1 if dt == np.float32 else 2)


@op('v_fmamk_f32')
def _(w, i):
    a, k, b = w.fsrc(i.ops[1]), w.vget(i.ops[2]).view(np.float32), w.fsrc(i.ops[3])
    w.vset(i.ops[0], exact_fma(a, k, b, np.float32).view(np.uint32))


@op('v_fma_f32', 'v_fma_f64')
def _(w, i):
    dt = np.float32 if i.mn.endswith('f32') else np.float64
    a, b, c = (w.fsrc(i.ops[k], dt) for k in (1, 2, 3))
    w.vset(i.ops[0], exact_fma(a, b, c, dt).view(np.uint32 if dt == np.float32 else np.uint64),
           1 if dt == np.float32 else 2)


@op('v_rcp_f32', 'v_rcp_iflag_f32')
def _(w, i):
    with np.errstate(all='ignore'):
        w.vset(i.ops[0], (np.float32(1.0) / w.fsrc(i.ops[1])).astype(np.float32).view(np.uint32))


@op('v_floor_f32')
def _(w, i): w.vset(i.ops[0], np.floor(w.fsrc(i.ops[1])).astype(np.float32).view(np.uint32))


@op('v_mad_i32_i24')
def _(w, i):
    def s24(x):
        x = (x & 0xFFFFFF).astype(np.int64)
        return np.where(x & 0x800000, x - 0x1000000, x)
    a, b = s24(w.vget(i.ops[1]).astype(np.int64)), s24(w.vget(i.ops[2]).astype(np.int64))
    w.vset(i.ops[0], ((a * b + i32(w.vget(i.ops[3])).astype(np.int64)) & MASK32).astype(np.uint32))


@op('v_trunc_f32')
def _(w, i): w.vset(i.ops[0], np.trunc(w.fsrc(i.ops[1])).astype(np.float32).view(np.uint32))


@op('v_ldexp_f32')
def _(w, i):
    with np.errstate(all='ignore'):
        e = i32(w.vget(i.ops[2])).astype(np.int64).clip(-400, 400).astype(np.int32)
        w.vset(i.ops[0], np.ldexp(w.fsrc(i.ops[1]), e).astype(np.float32).view(np.uint32))


@op('v_cvt_f32_u32')
def _(w, i): w.vset(i.ops[0], w.vget(i.ops[1]).astype(np.float32).view(np.uint32))


@op('v_cvt_f32_ubyte0', 'v_cvt_f32_ubyte1', 'v_cvt_f32_ubyte2', 'v_cvt_f32_ubyte3')
def _(w, i):
    k = int(i.mn[-1])
    w.vset(i.ops[0], ((w.vget(i.ops[1]) >> np.uint32(8 * k)) & np.uint32(255)).astype(np.float32).view(np.uint32))


@op('v_cvt_f32_i32')
def _(w, i): w.vset(i.ops[0], i32(w.vget(i.ops[1])).astype(np.float32).view(np.uint32))


@op('v_cvt_u32_f32')
def _(w, i):
    x = w.fsrc(i.ops[1]).astype(np.float64)
    x = np.where(np.isnan(x), 0, np.clip(np.trunc(x), 0, MASK32))
    w.vset(i.ops[0], x.astype(np.uint64).astype(np.uint32))


@op('v_cvt_i32_f32')
def _(w, i):
    x = w.fsrc(i.ops[1]).astype(np.float64)
    x = np.where(np.isnan(x), 0, np.clip(np.trunc(x), -2 ** 31, 2 ** 31 - 1))
    w.vset(i.ops[0], x.astype(np.int64).astype(np.int32).view(np.uint32))


@op('v_cvt_f64_i32')
def _(w, i): w.vset(i.ops[0], i32(w.vget(i.ops[1])).astype(np.float64).view(np.uint64), 2)


@op('v_cvt_f64_u32')
def _(w, i): w.vset(i.ops[0], w.vget(i.ops[1]).astype(np.float64).view(np.uint64), 2)


@op('v_cvt_f32_f64')
def _(w, i):
    with np.errstate(over='ignore'):        # beyond the binary32 range: infinity, as round to nearest gives
        w.vset(i.ops[0], w.fsrc(i.ops[1], np.float64).astype(np.float32).view(np.uint32))


@op('v_rndne_f32')
def _(w, i): w.vset(i.ops[0], np.rint(w.fsrc(i.ops[1])).astype(np.float32).view(np.uint32))


@op('v_sqrt_f32')
def _(w, i):
    # correctly rounded (the hardware's is within 1 ulp; the compiler's fixup sequence around it makes either exact)
    with np.errstate(invalid='ignore'):
        w.vset(i.ops[0], np.sqrt(w.fsrc(i.ops[1])).astype(np.float32).view(np.uint32))


def f32_class(x):
    """The class bits v_cmp_class tests: 0 sNaN, 1 qNaN, 2 -inf, 3 -normal, 4 -denorm, 5 -0, 6 +0, 7 +denorm,
    8 +normal, 9 +inf."""
    u = x.view(np.uint32)
    neg = (u >> np.uint32(31)).astype(bool)
    exp = (u >> np.uint32(23)) & np.uint32(255)
    man = u & np.uint32(0x7FFFFF)
    cls = np.zeros(x.shape, np.int64)
    nan = (exp == 255) & (man != 0)
    cls = np.where(nan & ((man >> np.uint32(22)) == 0), 0, cls)
    cls = np.where(nan & ((man >> np.uint32(22)) == 1), 1, cls)
    inf = (exp == 255) & (man == 0)
    cls = np.where(inf, np.where(neg, 2, 9), cls)
    norm = (exp > 0) & (exp < 255)
    cls = np.where(norm, np.where(neg, 3, 8), cls)
    den = (exp == 0) & (man != 0)
    cls = np.where(den, np.where(neg, 4, 7), cls)
    zero = (exp == 0) & (man == 0)
    cls = np.where(zero, np.where(neg, 5, 6), cls)
    return cls


@op('v_cmp_class_f32')
def _(w, i):
    x = w.fsrc(i.ops[1])
    mask = w.vget(i.ops[2]).astype(np.int64)
    set_mask(w, i.ops[0], ((mask >> f32_class(x)) & 1).astype(bool))


def _f32exp(x):
    return ((x.view(np.uint32) >> np.uint32(23)) & np.uint32(255)).astype(np.int64)


# The correctly rounded division sequence the compiler emits: v_div_scale (twice: the denominator and the
# numerator), a reciprocal and Newton steps, v_div_fmas, v_div_fixup.  Semantics from the instruction set reference's
# pseudocode; per type: (bias, exponent gap near overflow, scale exponent, tiny-numerator exponent bound, underflow gap,
# top exponent).
_DIV = {np.float32: (127, 96, 64, 23, -150, 255), np.float64: (1023, 768, 128, 53, -1075, 2047)}


def _fexp(x, dt):
    return _f32exp(x) if dt == np.float32 else _f64exp(x)


def _is_denorm(x, dt):
    return (_fexp(x, dt) == 0) & (x != 0)


def _div_scale(w, i, dt):
    """D = S0 (the value to scale: S1 the denominator or S2 the numerator) scaled by 2^+-s so that the reciprocal and
    the Newton steps stay in range; VCC marks the lanes whose quotient comes out scaled (undone by v_div_fmas).
    In priority order: a zero operand gives NaN; a quotient near overflow (exponent gap >= the type's bound) scales
    the denominator up and sets VCC; a denormal denominator scales both up; 1/S1 denormal (in binary64) with a
    denormal quotient scales the denominator up and sets VCC; 1/S1 denormal alone scales both down; a denormal
    quotient scales the numerator up and sets VCC; a tiny numerator scales both up."""
    bias, gap, sc, tiny, _, _ = _DIV[dt]
    s0, s1, s2 = (w.fsrc(i.ops[k], dt) for k in (2, 3, 4))
    e1, e2 = _fexp(s1, dt), _fexp(s2, dt)
    with np.errstate(all='ignore'):
        r64 = np.float64(1.0) / s1.astype(np.float64)
        rcp_den = _is_denorm(r64, np.float64)
        quo_den = _is_denorm((s2 / s1).astype(dt), dt)
        up, down = np.ldexp(s0, sc).astype(dt), np.ldexp(s0, -sc).astype(dt)
    out = s0.copy()
    vcc = np.zeros(64, bool)
    undecided = np.ones(64, bool)

    def case(cond, value=None, set_vcc=False):
        nonlocal out, vcc, undecided
        c = undecided & cond
        if value is not None:
            out = np.where(c, value, out)
        if set_vcc:
            vcc = vcc | c
        undecided = undecided & ~c
    case((s1 == 0) | (s2 == 0), dt(np.nan))
    case(e2 - e1 >= gap, np.where(s0 == s1, up, s0), True)
    case(_is_denorm(s1, dt), up)
    case(rcp_den & quo_den, np.where(s0 == s1, up, s0), True)
    case(rcp_den, down)
    case(quo_den, np.where(s0 == s2, up, s0), True)
    case(e2 <= tiny, up)
    w.vset(i.ops[0], out.astype(dt).view(np.uint32 if dt == np.float32 else np.uint64), 1 if dt == np.float32 else 2)
    set_mask(w, i.ops[1], vcc)


def _div_fmas(w, i, dt):
    """fma(S0, S1, S2), on VCC lanes scaled by 2^+s when S2 (the scaled quotient) has exponent >= the bias, else
    2^-s, with one rounding of the exact scaled value."""
    bias, _, sc, _, _, _ = _DIV[dt]
    a, b, c = (w.fsrc(i.ops[k], dt) for k in (1, 2, 3))
    out = exact_fma(a, b, c, dt)
    vcc = ((np.uint64(w.s[106] | (w.s[107] << 32)) >> LANES.astype(np.uint64)) & np.uint64(1)).astype(bool)
    for l in np.nonzero(vcc & w.lanes())[0]:
        x, y, z = float(a[l]), float(b[l]), float(c[l])
        if not all(np.isfinite(v) for v in (x, y, z)):
            with np.errstate(all='ignore'):
                out[l] = dt(x * y + z) * dt(2.0 ** (sc if _fexp(c[l:l + 1], dt)[0] >= bias else -sc))
            continue
        e = sc if _fexp(c[l:l + 1], dt)[0] >= bias else -sc
        out[l] = round_fraction((Fraction(x) * Fraction(y) + Fraction(z)) * Fraction(2) ** e, dt)
    w.vset(i.ops[0], out.astype(dt).view(np.uint32 if dt == np.float32 else np.uint64), 1 if dt == np.float32 else 2)


def _div_fixup(w, i, dt):
    """The sequence's final step (S0 the quotient, S1 the denominator, S2 the numerator): a NaN operand is returned
    quieted; 0/0 and inf/inf give the default NaN; x/0 and inf/y a signed infinity; x/inf and 0/y a signed zero; an
    exponent gap below the type's underflow bound a signed zero, a denominator with the top exponent a signed
    infinity; otherwise |S0| with the sign of num/den."""
    _, _, _, _, lo, top = _DIV[dt]
    q, den, num = (w.fsrc(i.ops[k], dt) for k in (1, 2, 3))
    ut = np.uint32 if dt == np.float32 else np.uint64
    quiet = ut(1 << 22) if dt == np.float32 else ut(1 << 51)
    sign = np.signbit(den) ^ np.signbit(num)
    signed = lambda v: np.where(sign, dt(-v), dt(v)).astype(dt)
    out = np.where(sign, -np.abs(q), np.abs(q)).astype(dt)
    qnan = np.array([0xFFC00000], np.uint32).view(np.float32)[0] if dt == np.float32 else \
        np.array([0xFFF8000000000000], np.uint64).view(np.float64)[0]
    conds = [
        (np.isnan(num), (num.view(ut) | quiet).view(dt)),
        (np.isnan(den), (den.view(ut) | quiet).view(dt)),
        ((den == 0) & (num == 0), np.full(64, qnan, dt)),
        (np.isinf(den) & np.isinf(num), np.full(64, qnan, dt)),
        ((den == 0) | np.isinf(num), signed(np.inf)),
        (np.isinf(den) | (num == 0), signed(0.0)),
        (_fexp(num, dt) - _fexp(den, dt) < lo, signed(0.0)),
        (_fexp(den, dt) == top, signed(np.inf)),
    ]
    for cond, val in reversed(conds):
        out = np.where(cond, val, out)
    w.vset(i.ops[0], out.astype(dt).view(ut), 1 if dt == np.float32 else 2)


def _f64exp(x):
    return ((x.view(np.uint64) >> np.uint64(52)) & np.uint64(0x7FF)).astype(np.int64)


for _t, _dt in (('f32', np.float32), ('f64', np.float64)):
    H[f'v_div_scale_{_t}'] = (lambda dt: lambda w, i: _div_scale(w, i, dt))(_dt)
    H[f'v_div_fmas_{_t}'] = (lambda dt: lambda w, i: _div_fmas(w, i, dt))(_dt)
    H[f'v_div_fixup_{_t}'] = (lambda dt: lambda w, i: _div_fixup(w, i, dt))(_dt)


# --- matrix core
# layout maps of v_mfma_i32_32x32x32_i8: operand element (row or column r, k) is lane r + 32 (k // 16), byte k % 16;
# result element (i, j) is lane j + 32 ((i // 4) % 2), register 4 (i // 8) + i % 4
_MF_R, _MF_K = np.meshgrid(np.arange(32), np.arange(32), indexing='ij')
_MF_LANE, _MF_BYTE = _MF_R + 32 * (_MF_K // 16), _MF_K % 16
_MF_I, _MF_J = np.meshgrid(np.arange(32), np.arange(32), indexing='ij')
_MF_DLANE, _MF_DREG = _MF_J + 32 * ((_MF_I // 4) % 2), 4 * (_MF_I // 8) + _MF_I % 4


@op('v_mfma_i32_32x32x32_i8')
def _(w, i):
    d, a, b, c = i.ops
    w.check_v(a.base, 4, 'reads')
    w.check_v(b.base, 4, 'reads')
    A = w.v[a.base:a.base + 4].T.copy().view(np.int8).reshape(64, 16)
    B = w.v[b.base:b.base + 4].T.copy().view(np.int8).reshape(64, 16)
    Am = A[_MF_LANE, _MF_BYTE].astype(np.int64)                 # [row][k]
    Bm = B[_MF_LANE, _MF_BYTE].astype(np.int64).T               # [k][col]
    if c.kind == 'lit':
        Cm = np.full((32, 32), c.value, np.int64)
    else:
        w.check_v(c.base, 16, 'reads')
        Creg = w.v[c.base:c.base + 16].T.view(np.int32)
        Cm = Creg[_MF_DLANE, _MF_DREG].astype(np.int64)
    D = ((Am @ Bm + Cm) & MASK32).astype(np.uint32)
    out = np.zeros((64, 16), np.uint32)
    out[_MF_DLANE, _MF_DREG] = D
    w.check_v(d.base, 16, 'writes')
    w.v[d.base:d.base + 16] = out.T


# v_mfma_i32_16x16x64_i8: operand element (row or column r, k) in lane r + 16 (k // 16), byte k % 16; result element
# (i, j) in lane j + 16 (i // 4), register i % 4
_M16_R, _M16_K = np.meshgrid(np.arange(16), np.arange(64), indexing='ij')
_M16_LANE, _M16_BYTE = _M16_R + 16 * (_M16_K // 16), _M16_K % 16
_M16_I, _M16_J = np.meshgrid(np.arange(16), np.arange(16), indexing='ij')
_M16_DLANE, _M16_DREG = _M16_J + 16 * (_M16_I // 4), _M16_I % 4


@op('v_mfma_i32_16x16x64_i8')
def _(w, i):
    d, a, b, c = i.ops
    w.check_v(a.base, 4, 'reads')
    w.check_v(b.base, 4, 'reads')
    A = w.v[a.base:a.base + 4].T.copy().view(np.int8).reshape(64, 16)
    B = w.v[b.base:b.base + 4].T.copy().view(np.int8).reshape(64, 16)
    Am = A[_M16_LANE, _M16_BYTE].astype(np.int64)               # [row][k]
    Bm = B[_M16_LANE, _M16_BYTE].astype(np.int64).T             # [k][col]
    if c.kind == 'lit':
        Cm = np.full((16, 16), c.value, np.int64)
    else:
        w.check_v(c.base, 4, 'reads')
        Cm = w.v[c.base:c.base + 4].T.view(np.int32)[_M16_DLANE, _M16_DREG].astype(np.int64)
    D = ((Am @ Bm + Cm) & MASK32).astype(np.uint32)
    out = np.zeros((64, 4), np.uint32)
    out[_M16_DLANE, _M16_DREG] = D
    w.check_v(d.base, 4, 'writes')
    w.v[d.base:d.base + 4] = out.T


@op('v_dot4c_i32_i8')
def _(w, i):
    a = w.vget(i.ops[1]).view(np.int8).reshape(64, 4).astype(np.int64)
    b = w.vget(i.ops[2]).view(np.int8).reshape(64, 4).astype(np.int64)
    d = i32(w.vget(i.ops[0])).astype(np.int64)
    w.vset(i.ops[0], ((d + (a * b).sum(1)) & MASK32).astype(np.uint32))


# --- LDS
def _ds_addr(w, op_):
    return w.vget(op_).astype(np.int64)


@op('ds_read_b32', 'ds_read_b64', 'ds_read_b128', 'ds_read_u16', 'ds_read_u8', 'ds_read2_b32')
def _(w, i):
    act = w.lanes()
    addr = _ds_addr(w, i.ops[1])
    if i.mn == 'ds_read2_b32':
        offs = [int(i.mods.get('offset0', 0)) * 4, int(i.mods.get('offset1', 0)) * 4]
        out = np.zeros((64, 2), np.uint32)
        for k, o in enumerate(offs):
            out[:, k] = w.wg.lds_read(addr + o, 4, act, w).view(np.uint32).reshape(64)
        w.check_v(i.ops[0].base, 2, 'writes')
        w.vset_regs(i.ops[0].base, out, act)
        return
    size = {'ds_read_b32': 4, 'ds_read_b64': 8, 'ds_read_b128': 16, 'ds_read_u16': 2, 'ds_read_u8': 1}[i.mn]
    data = w.wg.lds_read(addr + int(i.mods.get('offset', 0)), size, act, w)
    if size < 4:
        vals = data.view(np.uint16 if size == 2 else np.uint8).reshape(64).astype(np.uint32)
        w.vset(i.ops[0], vals, mask=act)
        return
    w.check_v(i.ops[0].base, size // 4, 'writes')
    w.vset_regs(i.ops[0].base, data.view(np.uint32).reshape(64, size // 4), act)


@op('ds_read2st64_b32')
def _(w, i):
    act = w.lanes()
    addr = _ds_addr(w, i.ops[1])
    out = np.zeros((64, 2), np.uint32)
    for k, key in enumerate(('offset0', 'offset1')):
        out[:, k] = w.wg.lds_read(addr + int(i.mods.get(key, 0)) * 256, 4, act, w).view(np.uint32).reshape(64)
    w.check_v(i.ops[0].base, 2, 'writes')
    w.vset_regs(i.ops[0].base, out, act)


@op('ds_write2st64_b32', 'ds_write2_b32')
def _(w, i):
    act = w.lanes()
    addr = _ds_addr(w, i.ops[0])
    unit = 256 if 'st64' in i.mn else 4
    for k, key in enumerate(('offset0', 'offset1')):
        data = w.vget(i.ops[1 + k]).view(np.uint8).reshape(64, 4)
        w.wg.lds_write(addr + int(i.mods.get(key, 0)) * unit, data, act, w)


@op('ds_read2st64_b64', 'ds_read2_b64')
def _(w, i):
    act = w.lanes()
    addr = _ds_addr(w, i.ops[1])
    unit = 512 if 'st64' in i.mn else 8
    out = np.zeros((64, 4), np.uint32)
    for k, key in enumerate(('offset0', 'offset1')):
        out[:, 2 * k:2 * k + 2] = w.wg.lds_read(addr + int(i.mods.get(key, 0)) * unit, 8, act, w).view(np.uint32)
    w.check_v(i.ops[0].base, 4, 'writes')
    w.vset_regs(i.ops[0].base, out, act)


@op('ds_write2st64_b64', 'ds_write2_b64')
def _(w, i):
    act = w.lanes()
    addr = _ds_addr(w, i.ops[0])
    unit = 512 if 'st64' in i.mn else 8
    for k, key in enumerate(('offset0', 'offset1')):
        data = w.vget(i.ops[1 + k], 2).view(np.uint8).reshape(64, 8)
        w.wg.lds_write(addr + int(i.mods.get(key, 0)) * unit, data, act, w)


@op('ds_add_u64')
def _(w, i):
    act = w.lanes()
    addr = _ds_addr(w, i.ops[0]) + int(i.mods.get('offset', 0))
    val = w.vget(i.ops[1], 2)
    for l in np.nonzero(act)[0]:               # lanes in order: the adds commute
        a = int(addr[l])
        old_ = w.wg.lds_read(np.full(64, a), 8, np.eye(64, dtype=bool)[0], w)[0].view(np.uint64)[0]
        new_ = np.array([(int(old_) + int(val[l])) & MASK64], np.uint64).view(np.uint8)
        w.wg.lds_write(np.full(64, a), np.tile(new_, (64, 1)), np.eye(64, dtype=bool)[0], w)


@op('ds_write_b8', 'ds_write_b16', 'ds_write_b32', 'ds_write_b64', 'ds_write_b128')
def _(w, i):
    act = w.lanes()
    addr = _ds_addr(w, i.ops[0]) + int(i.mods.get('offset', 0))
    size = {'ds_write_b8': 1, 'ds_write_b16': 2, 'ds_write_b32': 4, 'ds_write_b64': 8, 'ds_write_b128': 16}[i.mn]
    if size <= 4:
        data = w.vget(i.ops[1]).view(np.uint8).reshape(64, 4)[:, :size]
    else:
        data = np.stack([w.vget(Op(f'v{i.ops[1].base + k}')) for k in range(size // 4)], 1).view(np.uint8)
    w.wg.lds_write(addr, data, act, w)


# --- vector memory
def _rsrc(w, op_):
    words = [w.s[op_.base + k] for k in range(4)]
    base = words[0] | ((words[1] & 0xFFFF) << 32)
    stride = (words[1] >> 16) & 0x3FFF
    if stride:
        raise EmuError('strided buffer resources are not modelled')
    return base, words[2]


class Pending:
    __slots__ = ('regs', 'data', 'mask', 'lds')

    def __init__(self, regs=None, data=None, mask=None, lds=None):
        self.regs, self.data, self.mask, self.lds = regs, data, mask, lds


@op('buffer_load_dword', 'buffer_load_dwordx2', 'buffer_load_dwordx4', 'buffer_load_ushort', 'buffer_load_ubyte')
def _(w, i):
    size = {'buffer_load_dword': 4, 'buffer_load_dwordx2': 8, 'buffer_load_dwordx4': 16, 'buffer_load_ushort': 2,
            'buffer_load_ubyte': 1}[i.mn]
    to_lds = 'lds' in i.mods
    if to_lds:
        vaddr_op, rs_op, so_op = i.ops[0], i.ops[1], i.ops[2]
    else:
        vaddr_op, rs_op, so_op = i.ops[1], i.ops[2], i.ops[3]
    if 'idxen' in i.mods:
        raise EmuError('idxen buffer addressing is not modelled')
    base, nrec = _rsrc(w, rs_op)
    act = w.lanes()
    voff = w.vget(vaddr_op).astype(np.int64) if 'offen' in i.mods else np.zeros(64, np.int64)
    ioff = parse_int(str(i.mods.get('offset', 0)))
    soff = w.sget(so_op) if so_op.kind in ('s', 'lit') else 0
    # range check per dword (per element below a dword): in range when per-lane offset + instruction offset + the
    # element's offset < num_records; the scalar offset is added after the check
    off = voff + ioff
    step = 4 if size >= 4 else size
    data = np.zeros((64, size), np.uint8)
    for k in range(0, size, step):
        ok = act & (off + k < nrec)
        if ok.any():
            data[:, k:k + step] = w.wg.mem.gather(base + soff + off + k, step, ok)
    if to_lds:
        m0 = w.s[124] & 0x3FFFF
        dst = m0 + ioff + size * LANES
        w.wg.lds_pending(w, dst, size, act, data)
        w.queue.append(Pending(lds=(dst, size, act, data)))
        return
    nreg = max(1, size // 4)
    if size < 4:
        vals = data[:, :size].copy().view(np.uint16 if size == 2 else np.uint8).reshape(64).astype(np.uint32)
        arr = vals.reshape(64, 1)
    else:
        arr = data.view(np.uint32).reshape(64, nreg)
    w.check_v(i.ops[0].base, 0, '')
    issue_load(w, i.ops[0].base, arr, act)


def issue_load(w, base, arr, act):
    regs = list(range(base, base + arr.shape[1]))
    for r in regs:
        w.pending_v[r] = w.pending_v.get(r, 0) + 1
    w.queue.append(Pending(regs=regs, data=arr, mask=act))


def _gaddr(w, i, vaddr_op, saddr_op):
    act = w.lanes()
    off = parse_int(str(i.mods.get('offset', 0)))
    if saddr_op is None or saddr_op.kind == 'off':
        a = w.vget(vaddr_op, 2).astype(np.int64)
    else:
        a = w.vget(vaddr_op).astype(np.int64) + w.sget(saddr_op, 2)
    return a + off, act


@op('global_load_dword', 'global_load_dwordx2', 'global_load_dwordx4', 'global_load_ushort', 'global_load_ubyte',
    'global_load_sbyte', 'global_load_sshort')
def _(w, i):
    size = {'global_load_dword': 4, 'global_load_dwordx2': 8, 'global_load_dwordx4': 16, 'global_load_ushort': 2,
            'global_load_ubyte': 1, 'global_load_sbyte': 1, 'global_load_sshort': 2}[i.mn]
    addr, act = _gaddr(w, i, i.ops[1], i.ops[2])
    data = np.zeros((64, max(size, 4)), np.uint8)
    data[:, :size] = w.wg.mem.gather(addr, size, act)
    if i.mn in ('global_load_sbyte', 'global_load_sshort'):       # sign-extended into the dword
        neg = (data[:, size - 1] & 0x80) != 0
        data[neg, size:] = 0xFF
    arr = data.view(np.uint32).reshape(64, max(1, size // 4))
    issue_load(w, i.ops[0].base, arr, act)


@op('global_store_dword', 'global_store_dwordx2', 'global_store_dwordx3', 'global_store_dwordx4', 'global_store_short',
    'global_store_byte')
def _(w, i):
    size = {'global_store_dword': 4, 'global_store_dwordx2': 8, 'global_store_dwordx3': 12, 'global_store_dwordx4': 16,
            'global_store_short': 2, 'global_store_byte': 1}[i.mn]
    addr, act = _gaddr(w, i, i.ops[0], i.ops[2])
    nreg = max(1, size // 4)
    w.check_v(i.ops[1].base, nreg, 'reads')
    data = w.v[i.ops[1].base:i.ops[1].base + nreg].T.copy().view(np.uint8)
    w.wg.mem.scatter(addr, data[:, :size], act)
    w.queue.append(Pending())


@op('global_atomic_add')
def _(w, i):
    ret = 'sc0' in i.mods or 'glc' in i.mods
    if ret:
        vdst, vaddr, vdata, saddr = i.ops
    else:
        vaddr, vdata, saddr = i.ops
    addr, act = _gaddr(w, i, vaddr, saddr)
    val = w.vget(vdata)
    old = np.zeros(64, np.uint32)
    for l in np.nonzero(act)[0]:
        a = int(addr[l])
        o = int(w.wg.mem.read(a, 4).view(np.uint32)[0])
        old[l] = o
        w.wg.mem.write(a, np.array([(o + int(val[l])) & MASK32], np.uint32).view(np.uint8))
    if ret:
        issue_load(w, vdst.base, old.reshape(64, 1), act)
    else:
        w.queue.append(Pending())


@op('global_atomic_umax', 'global_atomic_umax_x2')
def _(w, i):
    wide = i.mn.endswith('_x2')
    n = 8 if wide else 4
    ret = 'sc0' in i.mods or 'glc' in i.mods
    if ret:
        vdst, vaddr, vdata, saddr = i.ops
    else:
        vaddr, vdata, saddr = i.ops
    addr, act = _gaddr(w, i, vaddr, saddr)
    val = w.vget(vdata, 2 if wide else 1)
    dt = np.uint64 if wide else np.uint32
    old = np.zeros((64, n // 4), np.uint32)
    for l in np.nonzero(act)[0]:                 # lanes in order: max commutes
        a = int(addr[l])
        o = int(w.wg.mem.read(a, n).view(dt)[0])
        old[l] = np.array([o], dt).view(np.uint32)
        w.wg.mem.write(a, np.array([max(o, int(val[l]))], dt).view(np.uint8))
    if ret:
        issue_load(w, vdst.base, old, act)
    else:
        w.queue.append(Pending())


@op('flat_load_dword', 'flat_load_dwordx2', 'flat_load_dwordx4')
def _(w, i):
    """Generic addresses: the LDS aperture (src_shared_base's high word) reads LDS, anything else device memory."""
    n = int(i.mn[-1]) if i.mn[-2] == 'x' else 1
    act = w.lanes()
    addr = w.vget(i.ops[1], 2).astype(np.int64) + parse_int(str(i.mods.get('offset', 0)))
    lds = ((addr >> 32) == 0x10000) & act
    if (((addr >> 32) == 0x20000) & act).any():
        raise EmuError('flat access to scratch is not modelled')
    data = np.zeros((64, 4 * n), np.uint8)
    if lds.any():
        data[lds] = w.wg.lds_read(addr & MASK32, 4 * n, lds, w)[lds]
    glob = act & ~lds
    if glob.any():
        data[glob] = w.wg.mem.gather(addr, 4 * n, glob)[glob]
    issue_load(w, i.ops[0].base, data.view(np.uint32).reshape(64, n), act)


@op('global_atomic_add_x2', 'global_atomic_swap_x2')
def _(w, i):
    ret = 'sc0' in i.mods or 'glc' in i.mods
    if ret:
        vdst, vaddr, vdata, saddr = i.ops
    else:
        vaddr, vdata, saddr = i.ops
    addr, act = _gaddr(w, i, vaddr, saddr)
    val = w.vget(vdata, 2)
    old = np.zeros((64, 2), np.uint32)
    for l in np.nonzero(act)[0]:
        a = int(addr[l])
        o = int(w.wg.mem.read(a, 8).view(np.uint64)[0])
        old[l] = np.array([o], np.uint64).view(np.uint32)
        n = (o + int(val[l])) & MASK64 if i.mn == 'global_atomic_add_x2' else int(val[l])
        w.wg.mem.write(a, np.array([n], np.uint64).view(np.uint8))
    if ret:
        issue_load(w, vdst.base, old, act)
    else:
        w.queue.append(Pending())


@op('scratch_load_dword', 'scratch_load_dwordx2', 'scratch_load_dwordx3', 'scratch_load_dwordx4')
def _(w, i):
    n = int(i.mn[-1]) if i.mn[-2] == 'x' else 1
    act = w.lanes()
    off = _scratch_off(w, i, i.ops[1], i.ops[2])
    arr = np.zeros((64, n), np.uint32)
    for l in np.nonzero(act)[0]:
        arr[l] = w.priv[l, off[l]:off[l] + 4 * n].view(np.uint32)
    issue_load(w, i.ops[0].base, arr, act)


@op('scratch_store_dword', 'scratch_store_dwordx2', 'scratch_store_dwordx3', 'scratch_store_dwordx4')
def _(w, i):
    n = int(i.mn[-1]) if i.mn[-2] == 'x' else 1
    act = w.lanes()
    off = _scratch_off(w, i, i.ops[0], i.ops[2])
    data = np.stack([w.vget(Op(f'v{i.ops[1].base + k}')) for k in range(n)], 1).view(np.uint8)
    for l in np.nonzero(act)[0]:
        w.priv[l, off[l]:off[l] + 4 * n] = data[l]
    w.queue.append(Pending())


def _scratch_off(w, i, vaddr, saddr):
    off = np.full(64, parse_int(str(i.mods.get('offset', 0))), np.int64)
    if vaddr.kind == 'v':
        off += w.vget(vaddr).astype(np.int64)
    if saddr.kind == 's':
        off += w.sget(saddr)
    if (off < 0).any() or (off + 16 > w.priv.shape[1]).any():
        raise EmuError('scratch access outside the private segment')
    return off


# ------------------------------------------------------------------------------------------------ workgroups
class Workgroup:
    def __init__(self, prog, mem, wg_id, nthreads, wg_id_y=0, dyn_lds=0, wg_id_z=0, kernarg=0):
        self.prog, self.mem = prog, mem
        self.wg_ids = (wg_id, wg_id_y, wg_id_z)
        self.lds_size = prog.lds_bytes + dyn_lds
        self.lds = np.zeros(max(self.lds_size, 4) + 16, np.uint8)
        self.lds_busy = np.zeros(self.lds.size, np.int32)     # bytes that pending copies will write
        self.waves = []
        for wv in range((nthreads + 63) // 64):
            w = Wave(self, wv, prog)
            w.s[0], w.s[1] = kernarg & MASK32, kernarg >> 32
            w.s[2] = wg_id
            k = 3
            if prog.wg_id_y:
                w.s[k] = wg_id_y
                k += 1
            if prog.wg_id_z:
                w.s[k] = wg_id_z
            tid = wv * 64 + LANES
            w.v[0] = tid.astype(np.uint32)
            n = min(64, nthreads - wv * 64)
            w.exec = (1 << n) - 1 if n < 64 else MASK64
            self.waves.append(w)

    def lds_check(self, addr, size, act, w, what):
        a = addr[act].astype(np.int64)
        if a.size == 0:
            return None
        if a.min() < 0 or a.max() + size > self.lds_size:
            raise EmuError(f'LDS {what} of {size} bytes at {int(a.min())}..{int(a.max())} outside the {self.lds_size} '
                           f'allocated')
        idx = a[:, None] + np.arange(size)
        if self.lds_busy[idx].any():
            raise EmuError(f'wave {w.wid} pc {w.pc} ({self.prog.instrs[w.pc].text}): LDS {what} at {int(a.min())} '
                           f'while a copy into it is pending')
        return idx

    def lds_read(self, addr, size, act, w):
        idx = self.lds_check(addr, size, act, w, 'read')
        out = np.zeros((64, size), np.uint8)
        if idx is not None:
            out[act] = self.lds[idx]
        return out

    def lds_write(self, addr, data, act, w):
        idx = self.lds_check(addr, data.shape[1], act, w, 'write')
        if idx is not None:
            self.lds[idx] = data[act]

    def lds_pending(self, w, dst, size, act, data):
        idx = self.lds_check(dst, size, act, w, 'copy')
        if idx is not None:
            np.add.at(self.lds_busy, idx.ravel(), 1)

    def retire(self, w, p):
        if p.lds is not None:
            dst, size, act, data = p.lds
            idx = dst[act].astype(np.int64)[:, None] + np.arange(size)
            np.subtract.at(self.lds_busy, idx.ravel(), 1)
            self.lds[idx] = data[act]
        elif p.regs is not None:
            for k, r in enumerate(p.regs):
                w.pending_v[r] -= 1
                w.v[r][p.mask] = p.data[p.mask, k]

    def exec_one(self, w):
        """One instruction of wave w."""
        ins = self.prog.instrs[w.pc]
        if w.gpr_idx is not None and ins.mn.startswith('v_'):
            ins = indexed(ins, *w.gpr_idx)
        try:
            ins.fn(w, ins)
        except EmuError as e:
            if ' pc ' in str(e):
                raise
            raise EmuError(f'workgroup {self.wg_ids} wave {w.wid} pc {w.pc} ({ins.text}): {e}') from None
        except Exception as e:
            raise EmuError(f'wave {w.wid} pc {w.pc} ({ins.text}): {type(e).__name__}: {e}') from e
        if TRACE is not None:
            TRACE(w, ins)
        w.pc += 1

    def run(self, max_steps=50_000_000):
        steps = 0
        while True:
            live = [w for w in self.waves if not w.done]
            if not live:
                return steps
            progressed = False
            for w in live:
                while not w.done and not w.at_barrier:
                    self.exec_one(w)
                    steps += 1
                    progressed = True
                    if steps > max_steps:
                        raise EmuError('step limit: the kernel does not end')
            live = [w for w in self.waves if not w.done]
            if live and all(w.at_barrier for w in live):
                for w in live:
                    w.at_barrier = False
            elif not progressed:
                raise EmuError('deadlock: waves wait at a barrier that others never reach')

    def step(self, rng, budget):
        """Up to `budget` instructions of this workgroup, its waves taking turns of 1 to 16 instructions in an order
        drawn from rng; returns (instructions run, finished)."""
        steps = 0
        while steps < budget:
            live = [w for w in self.waves if not w.done]
            if not live:
                return steps, True
            runnable = [w for w in live if not w.at_barrier]
            if not runnable:                    # every live wave has reached the barrier: release it
                for w in live:
                    w.at_barrier = False
                continue
            w = runnable[rng.randrange(len(runnable))]
            for _ in range(rng.randint(1, 16)):
                if w.done or w.at_barrier or steps >= budget:
                    break
                self.exec_one(w)
                steps += 1
        return steps, all(w.done for w in self.waves)


def indexed(ins, idx, which):
    """A copy of a vector instruction with the index added to the VGPR operands that index mode names."""
    pos = {'DST': 0, 'SRC0': 1, 'SRC1': 2, 'SRC2': 3}
    new = Instr.__new__(Instr)
    new.mn, new.mods, new.text, new.fn, new.target = ins.mn, ins.mods, ins.text + f' [index {idx}]', ins.fn, ins.target
    new.ops = list(ins.ops)
    for name in which:
        k = pos[name]
        o = new.ops[k]
        if o.kind == 'v':
            c = Op(o.text)
            c.base = o.base + idx
            new.ops[k] = c
    return new


TRACE = None          # debugging hook: called with (wave, instruction) after each instruction


HIDDEN = {'hidden_block_count_x': lambda g, b: g, 'hidden_block_count_y': lambda g, b: 1,
          'hidden_block_count_z': lambda g, b: 1, 'hidden_group_size_x': lambda g, b: b,
          'hidden_group_size_y': lambda g, b: 1, 'hidden_group_size_z': lambda g, b: 1,
          'hidden_remainder_x': lambda g, b: 0, 'hidden_remainder_y': lambda g, b: 0,
          'hidden_remainder_z': lambda g, b: 0, 'hidden_grid_dims': lambda g, b: 1}


def launch(prog, mem, grid, block, kernarg_bytes, dyn_lds=0):
    """Runs every workgroup of the grid (an int, or (x, y) for a 2-D grid) in order, x fastest."""
    if len(kernarg_bytes) > prog.kernarg_size:
        raise EmuError('kernel arguments larger than the kernel expects')
    kbase = mem.alloc(max(prog.kernarg_size, 8) + 64)
    ka = mem.array(kbase, np.uint8, max(prog.kernarg_size, 8) + 64)
    ka[:len(kernarg_bytes)] = np.frombuffer(bytes(kernarg_bytes), np.uint8)
    gx, gy, gz = (grid, 1, 1) if isinstance(grid, int) else (tuple(grid) + (1, 1))[:3]
    if (gy > 1 and not prog.wg_id_y) or (gz > 1 and not prog.wg_id_z):
        raise EmuError('a grid dimension the kernel does not read')
    for off, size, kind in prog.hidden:        # launch dimensions; every other hidden argument (queues, heaps) is 0
        v = HIDDEN[kind](gx, block) if kind in HIDDEN else 0
        if kind == 'hidden_block_count_y':
            v = gy
        if kind == 'hidden_block_count_z':
            v = gz
        if kind == 'hidden_dynamic_lds_size':
            v = dyn_lds
        ka[off:off + size] = np.frombuffer(int(v).to_bytes(size, 'little'), np.uint8)
    steps = 0
    try:
        if INTERLEAVE is None:
            for z in range(gz):
                for y in range(gy):
                    for x in range(gx):
                        steps += Workgroup(prog, mem, x, block, y, dyn_lds, z, kernarg=kbase).run()
        else:
            # every workgroup resident at once, run in turns of random length in a random order, so that the
            # cross-workgroup hand-overs (last arriver of a split tile or K-slice) meet other arrival orders than
            # the grid order; loads take memory as it is when they issue, stores are visible at once
            steps = run_interleaved([Workgroup(prog, mem, x, block, y, dyn_lds, z, kernarg=kbase)
                                     for z in range(gz) for y in range(gy) for x in range(gx)], INTERLEAVE)
    finally:
        mem.release(kbase)
    return steps


def run_interleaved(wgs, seed, max_steps=None):
    """Runs the workgroups all resident at once: a random one (seeded) runs a turn of 1 to 400 instructions, its waves
    taking sub-turns in random order, until every workgroup has ended; returns the instructions run."""
    import random
    rng = random.Random(seed)
    live = list(wgs)
    limit = max_steps or 50_000_000 * max(1, len(live) // 64)
    steps = 0
    while live:
        k = rng.randrange(len(live))
        n, finished = live[k].step(rng, rng.randint(1, 400))
        steps += n
        if finished:
            live.pop(k)
        if steps > limit:
            raise EmuError('step limit: the kernel does not end')
    return steps


# None: workgroups run one after another in grid order.  An integer: they are interleaved (seeded by it), see launch.
# The environment's DET_EMU_INTERLEAVE sets it for a whole test run.
INTERLEAVE = int(os.environ['DET_EMU_INTERLEAVE']) if os.environ.get('DET_EMU_INTERLEAVE') else None
