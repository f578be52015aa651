"""Checker for the vector-memory waits of compiled gfx950 kernels.

Some kernels issue their loads as inline assembly and wait for them with explicit `s_waitcnt vmcnt(n)`; the compiler
does not see those loads, so it cannot protect their destination registers.  The hardware has no interlock either:
an instruction that reads (or overwrites) a VGPR whose load has not returned sees whatever the register held.  This
module compiles a HIP source to assembly with the library's flags and proves, for every kernel in it, that no
instruction touches a VGPR while a load into it may still be outstanding.

Model (gfx9 vector-memory counter): every buffer/global/flat/scratch operation joins one in-order queue;
`s_waitcnt vmcnt(n)` (or a plain `s_waitcnt 0`) leaves at most n of the newest entries.  A load contributes its
destination registers (none for a copy into LDS, or for a store or an atomic without return).  The analysis keeps,
for every VGPR that may be the destination of an outstanding load, the fewest operations issued after that load on
any path; `vmcnt(n)` clears the registers with at least n of them.  States meet at the joins of the kernel's
control-flow graph (basic blocks split at labels and branches) by union with the minimum, and the propagation runs
to a fixed point.  A violation is any instruction whose VGPR operands meet a possibly outstanding destination
(a newer load may overwrite one: loads return in order).
"""
import os
import re
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, 'det_amd', 'csrc')
VMEM = re.compile(r'^(buffer|global|flat|scratch)_')
VREG = re.compile(r'\bv(?:\[(\d+):(\d+)\]|(\d+)\b)')
BRANCH = re.compile(r'^s_(c?branch)\w*$')
CAP = 63            # the counter's capacity: an operation with 63 newer ones has completed


_CACHE = {}


def asm_of(source):
    """compile_asm into a scratch directory, once per source and modification time in this process."""
    import tempfile
    key = (os.path.abspath(source), os.path.getmtime(source))
    if key not in _CACHE:
        d = tempfile.mkdtemp(prefix='det_asm_')
        _CACHE[key] = compile_asm(source, os.path.join(d, os.path.basename(source) + '.s'))
    return _CACHE[key]


def compile_asm(source, out_path):
    """The device assembly of one source file, built with the library's flags (det_amd/build.py).  The source is
    compiled to an object (so that the assembler validates every instruction, inline assembly included) and the
    assembly the object was made from is returned; out_path names a scratch directory's file for it."""
    import glob
    import shutil
    import sys
    sys.path.insert(0, ROOT)
    from det_amd import build
    hipcc = os.path.join(os.environ.get('ROCM_PATH', '/opt/rocm'), 'bin', 'hipcc')
    flags = [f for f in build.HIPFLAGS if f not in ('-shared', '-fPIC')]
    work = os.path.dirname(os.path.abspath(out_path))
    subprocess.check_call([hipcc] + flags + ['-c', '--cuda-device-only', '--save-temps', os.path.abspath(source),
                           '-o', os.path.join(work, 'device.o')], cwd=work, stderr=subprocess.DEVNULL)
    stem = os.path.splitext(os.path.basename(source))[0]
    asm = glob.glob(os.path.join(work, f'{stem}-hip-amdgcn-amd-amdhsa-*.s'))
    assert len(asm) == 1, asm
    shutil.copyfile(asm[0], out_path)
    return open(out_path).read()


def kernels(asm):
    """{symbol: [instruction lines]} for every function in the assembly."""
    out = {}
    name = None
    body = []
    for line in asm.splitlines():
        m = re.match(r'^([A-Za-z_][\w.$]*):', line)
        if m and not line.startswith('.') and not m.group(1).startswith('.L'):
            name, body = m.group(1), []
            continue
        if name is None:
            continue
        if line.startswith('.Lfunc_end'):
            out[name] = body
            name = None
            continue
        body.append(line)
    return out


def vregs(text):
    regs = set()
    for a, b, c in VREG.findall(text):
        if c:
            regs.add(int(c))
        else:
            regs.update(range(int(a), int(b) + 1))
    return regs


def parse(body):
    """Instructions as (mnemonic, operand text) and labels as ('label', name)."""
    items = []
    for line in body:
        s = line.split(';')[0].strip()
        if not s:
            continue
        if re.match(r'^\.?L\w+:$', s):
            items.append(('label', s[:-1]))
            continue
        if s.startswith('.'):
            continue
        parts = s.split(None, 1)
        items.append((parts[0], parts[1] if len(parts) > 1 else ''))
    return items


def vm_effect(mn, ops):
    """(registers read before issue, destination registers or None) of a vector-memory instruction."""
    operands = [o.strip() for o in ops.split(',')]
    allregs = vregs(ops)
    if mn.startswith(('buffer_load', 'global_load', 'flat_load', 'scratch_load')):
        if re.search(r'\blds\b', ops):
            return allregs, None
        dest = vregs(operands[0])
        return vregs(', '.join(operands[1:])), dest
    if 'atomic' in mn and re.search(r'\bsc0\b|\bglc\b', ops):
        dest = vregs(operands[0])
        return vregs(', '.join(operands[1:])), dest
    return allregs, None


def waitcnt_vm(ops):
    """The vmcnt limit of an s_waitcnt, or None when it does not wait on the vector-memory counter."""
    ops = ops.strip()
    if re.fullmatch(r'0|0x0', ops):
        return 0
    m = re.search(r'vmcnt\((\d+)\)', ops)
    return int(m.group(1)) if m else None


def check_kernel(body):
    """Violations [(instruction index, text, registers)] of one kernel."""
    items = parse(body)
    labels = {it[1]: i for i, it in enumerate(items) if it[0] == 'label'}
    starts = {0}
    for i, (mn, ops) in enumerate(items):
        if mn == 'label':
            starts.add(i)
        elif BRANCH.match(mn) or mn == 's_endpgm':
            starts.add(i + 1)
    starts = sorted(s for s in starts if s < len(items))
    block_end = {s: (starts[bi + 1] if bi + 1 < len(starts) else len(items)) for bi, s in enumerate(starts)}
    entry = {0: {}}
    work = [0]
    violations = {}
    while work:
        start = work.pop()
        pend = dict(entry[start])            # register -> fewest operations issued after its pending load
        succ = []
        i = start
        end = block_end[start]
        while i < end:
            mn, ops = items[i]
            if mn == 'label':
                i += 1
                continue
            if mn == 's_waitcnt':
                n = waitcnt_vm(ops)
                if n is not None:
                    pend = {r: y for r, y in pend.items() if y < n}
            elif VMEM.match(mn):
                src, dest = vm_effect(mn, ops)
                bad = src & pend.keys()
                if bad:
                    violations[i] = (mn + ' ' + ops, sorted(bad))
                pend = {r: y + 1 for r, y in pend.items() if y + 1 < CAP}
                for r in dest or ():
                    pend[r] = 0
            else:
                bad = vregs(ops) & pend.keys()
                if bad:
                    violations[i] = (mn + ' ' + ops, sorted(bad))
            if mn == 's_endpgm' or mn.startswith('s_setpc'):
                break
            m = BRANCH.match(mn)
            if m:
                succ.append(labels[ops.split()[0]])
                if m.group(1) == 'cbranch':
                    succ.append(i + 1)
                break
            i += 1
        else:
            succ.append(end)
        for s_ in succ:
            if s_ >= len(items):
                continue
            old = entry.get(s_)
            if old is None:
                entry[s_] = dict(pend)
                work.append(s_)
                continue
            merged = dict(old)
            for r, y in pend.items():
                merged[r] = min(y, merged.get(r, y))
            if merged != old:
                entry[s_] = merged
                work.append(s_)
    return [(i,) + violations[i] for i in sorted(violations)]
