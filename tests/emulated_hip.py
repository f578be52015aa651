"""Test infrastructure: runs the library's own host code (det_amd/libdet_hip.so, unchanged) on a machine without a
GPU, with every kernel launch executed by the instruction-level emulator (tests/gfx950_emu.py).

tests/emu_runtime/hip_on_emulator.cpp stands in for the HIP runtime entry points the library imports.  It is loaded
with RTLD_GLOBAL before the library, so the library's references bind to it, and this module installs three
callbacks into it:
  * launch: the device symbol the library registered for the kernel's host stub, the grid, the block, the argument
    pointers and the dynamic LDS size -> the emulator runs the compiled kernel (assembly from the same sources and
    flags as the library) over the whole grid;
  * alloc / release: "device" buffers are emulator memory, i.e. numpy buffers at their own host addresses, so the
    runtime's copies and fills are plain memcpy / memset and the kernels see them.
Everything on the path from the C ABI to the kernels is thus the shipped code: argument checks, kernel choice, grid
and slice sizes, the partial-result buffers and their reuse, the part routing of the epilogue.

Use from a fresh process only (install() must run before det_amd.ffi loads the library): the tests start one.
"""
import ctypes
import os
import subprocess
import sys
import traceback

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SHIM_SRC = os.path.join(ROOT, 'tests', 'emu_runtime', 'hip_on_emulator.cpp')
SHIM_MAP = os.path.join(ROOT, 'tests', 'emu_runtime', 'versions.map')
CSRC = os.path.join(ROOT, 'det_amd', 'csrc')
LIB = os.path.join(ROOT, 'det_amd', 'libdet_hip.so')

LAUNCH = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_char_p, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint, ctypes.c_uint,
                          ctypes.c_uint, ctypes.c_uint, ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t)
ALLOC = ctypes.CFUNCTYPE(ctypes.c_void_p, ctypes.c_size_t)
RELEASE = ctypes.CFUNCTYPE(ctypes.c_int, ctypes.c_void_p)


def build_shim(out_dir):
    """Compiles the runtime stand-in into out_dir; returns the .so path."""
    out = os.path.join(out_dir, 'libhip_on_emulator.so')
    rocm = os.environ.get('ROCM_PATH', '/opt/rocm')
    subprocess.check_call(['g++', '-std=c++17', '-O1', '-shared', '-fPIC', '-D__HIP_PLATFORM_AMD__',
                           f'-I{rocm}/include', f'-Wl,--version-script={SHIM_MAP}', '-o', out, SHIM_SRC])
    return out


def build_asm(out_dir):
    """The device assembly of every library source (tests/isa_waits.asm_of: the library's flags, cached per process),
    written as out_dir/<stem>/<source>.s."""
    from tests import isa_waits
    for src in sorted(f for f in os.listdir(CSRC) if f.endswith('.hip')):
        d = os.path.join(out_dir, src[:-4])
        os.makedirs(d, exist_ok=True)
        with open(os.path.join(d, src + '.s'), 'w') as fh:
            fh.write(isa_waits.asm_of(os.path.join(CSRC, src)))


def library_is_current():
    """The built library is newer than every source it is made from (else the emulated kernels, compiled from the
    sources, would not be the ones its host code launches)."""
    if not os.path.exists(LIB):
        return False
    t = os.path.getmtime(LIB)
    return all(os.path.getmtime(os.path.join(CSRC, f)) <= t for f in os.listdir(CSRC))


class Emulated:
    """The installed stand-in: its memory, the programs by device symbol, and launch statistics."""

    def __init__(self, shim_path, asm_dir, cus):
        from tests import gfx950_emu as E
        self.E = E
        self.mem = E.Memory()
        self.asm = {}
        for d in sorted(os.listdir(asm_dir)):
            if not os.path.isdir(os.path.join(asm_dir, d)):
                continue
            for f in os.listdir(os.path.join(asm_dir, d)):
                if f.endswith('.hip.s'):
                    self.asm[f] = open(os.path.join(asm_dir, d, f)).read()
        self.programs = {}
        self.launches = []              # (device symbol, grid, block, dynamic LDS bytes)
        self.shim = ctypes.CDLL(shim_path, mode=ctypes.RTLD_GLOBAL)
        self._cb = (LAUNCH(self._launch), ALLOC(self._alloc), RELEASE(self._release))
        self.shim.emu_install(*self._cb, ctypes.c_int(cus))

    def program(self, name):
        if name not in self.programs:
            E = self.E
            hits = [a for a in self.asm.values() if f'\n{name}:' in a]
            if len(hits) != 1:
                raise E.EmuError(f'kernel {name}: found in {len(hits)} sources')
            p = E.Program.__new__(E.Program)
            E.Program.__init__(p, hits[0], name)
            if p.name != name:
                raise E.EmuError(f'kernel {name}: resolved to {p.name}')
            self.programs[name] = p
        return self.programs[name]

    def _launch(self, name, gx, gy, gz, bx, by, bz, args, shared):
        try:
            name = name.decode()
            if by != 1 or bz != 1:
                raise self.E.EmuError(f'{name}: {bx}x{by}x{bz} blocks are not modelled')
            p = self.program(name)
            ka = bytearray(p.kernarg_size)
            for i, (off, size) in enumerate(p.args):
                ka[off:off + size] = ctypes.string_at(args[i], size)
            self.launches.append((name, (gx, gy, gz), bx, int(shared)))
            self.E.launch(p, self.mem, (gx, gy, gz), bx, bytes(ka), dyn_lds=int(shared))
            return 0
        except Exception:
            traceback.print_exc()
            sys.stderr.flush()
            return 1

    def _alloc(self, nbytes):
        return self.mem.alloc(nbytes)

    def _release(self, p):
        self.mem.release(p)
        return 0

    def kernels_run(self):
        return sorted({n for n, *_ in self.launches})


def install(cus=4):
    """Loads the stand-in and installs the emulator behind it, from the paths the parent test passed in the
    environment (DET_EMU_SHIM, DET_EMU_ASM).  Must run before anything loads det_amd/libdet_hip.so."""
    return Emulated(os.environ['DET_EMU_SHIM'], os.environ['DET_EMU_ASM'], cus)


_INSTALLED = None


def pytest_configure(config):
    """As a pytest plugin (`-p tests.emulated_hip`): installs the stand-in before any test module loads the library,
    so that the GPU tests selected on the command line run on the emulator."""
    global _INSTALLED
    if _INSTALLED is None:
        _INSTALLED = install(int(os.environ.get('DET_EMU_CUS', '4')))


def pytest_unconfigure(config):
    """With DET_EMU_LOG set: the device symbols launched in this session, one per line, into that file."""
    path = os.environ.get('DET_EMU_LOG')
    if path and os.environ.get('PYTEST_XDIST_WORKER'):
        path += '.' + os.environ['PYTEST_XDIST_WORKER']     # one file per worker process
    if path and _INSTALLED is not None:
        with open(path, 'w') as fh:
            fh.write('\n'.join(_INSTALLED.kernels_run()) + '\n')
