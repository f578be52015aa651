"""The runtime half of the C ABI on the GPU (det_hip.h; the reference's runtime.cu:83-128 behaviour):
det_malloc zero-fills and is counted by det_allocated_bytes, det_free(NULL) is a no-op, det_free of a pointer
det_malloc did not return aborts with a message, det_memcpy copies in every direction, det_sync returns."""
import ctypes
import subprocess
import sys
import textwrap

import numpy as np
import pytest

from det_amd import ffi

pytestmark = pytest.mark.gpu
ROOT = __import__('os').path.dirname(__import__('os').path.dirname(__import__('os').path.abspath(__file__)))


def test_malloc_zero_fill_and_accounting():
    L = ffi.lib()
    assert L.det_init() == 0
    before = L.det_allocated_bytes()
    a = ffi.Buf(1 << 20, np.uint8)
    assert L.det_allocated_bytes() == before + (1 << 20)
    assert not a.download().any()
    a.write(np.full(1 << 20, 7, np.uint8))
    b = ffi.Buf(1 << 20, np.uint8)
    L.det_memcpy(b.ptr, a.ptr, 1 << 20, None)              # device to device
    assert (b.download() == 7).all()
    a.free()
    b.free()
    assert L.det_allocated_bytes() == before
    L.det_free(None)
    L.det_sync()


def test_free_of_a_foreign_pointer_aborts():
    code = textwrap.dedent(f'''
        import os, sys, ctypes
        sys.path.insert(0, {ROOT!r})
        if os.environ.get('DET_EMU_SHIM'):      # run on the CPU emulator when the parent does
            from tests import emulated_hip
            emulated_hip.install()
        from det_amd import ffi
        L = ffi.lib()
        p = L.det_malloc(64)
        L.det_free(ctypes.c_void_p(p + 16))
        print("returned")
    ''')
    r = subprocess.run([sys.executable, '-c', code], capture_output=True, text=True, timeout=120)
    assert r.returncode != 0 and 'returned' not in r.stdout, r.stdout + r.stderr
    assert 'not returned by det_malloc' in r.stderr, r.stderr
