"""CPU-side checks of the C ABI (include/det_hip.h) and the host logic of libdet_hip.so -- nothing here launches a
kernel: the library loads and exports every declared symbol, the plane sizes of the tiled layout, and the
reference's fail-fast behaviour on invalid arguments (message + abort, kernels/cuda/gemm.cu:1030-1057,
norm.cu:117-139), which the library checks before touching a device."""
import ctypes
import os
import subprocess
import sys
import textwrap

import pytest

from det_amd import ffi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def test_library_exports_every_header_symbol():
    L = ctypes.CDLL(ffi.LIB_PATH)
    names = ffi.header_symbols()
    assert len(names) >= 20
    missing = [n for n in names if not hasattr(L, n)]
    assert not missing, missing


def test_header_compiles_as_c():
    src = '#include "det_hip.h"\nint main(void) { det_qlinear q = {0}; (void)q; return (int)sizeof(det_qlinear) - 40; }\n'
    p = subprocess.run(['gcc', '-x', 'c', '-std=c99', '-fsyntax-only', '-I', os.path.join(ROOT, 'include'),
                        '-I', '/opt/rocm/include', '-D__HIP_PLATFORM_AMD__', '-'], input=src, text=True,
                       capture_output=True)
    assert p.returncode == 0, p.stderr


@pytest.mark.parametrize('N,K,bits', [(1, 128, 6), (64, 128, 8), (65, 256, 4), (9728, 2560, 6), (248320, 2560, 8)])
def test_linear_sizes(N, K, bits):
    wq, c, m = ffi.linear_sizes(N, K, bits)
    T = 2 * ((N + 127) // 128)                         # whole pairs of 64-row tiles
    G = K // 128
    # the decode tiles: T * G * 64 rows' packed groups (the prefill planes of the same size follow them only under
    # DET_PREFILL=streamk, checked by test_prefill_logic.py::test_linear_sizes_with_streamk)
    assert wq == T * G * 64 * 4 * {8: 32, 6: 24, 4: 16}[bits]
    assert c == T * 64 * 4
    assert m == T * G * 64 * 2


def test_scratch_bytes_matches_reference_formula():
    L = ffi.lib()
    for M, K in ((1, 128), (512, 2560), (65, 17408), (0, 2560)):
        assert L.det_gemm_scratch_bytes(M, K) == max(M, 1) * ((K + 127) // 128) * 4


def run_abort(body):
    """Runs `body` (python using ffi) in a subprocess; returns (returncode, stderr)."""
    code = textwrap.dedent(f'''
        import ctypes, sys
        sys.path.insert(0, {ROOT!r})
        from det_amd import ffi
        L = ffi.lib()
        q = ffi.QLinear(None, None, None, 64, 256, 6)
        {body}
        print("returned")
    ''')
    p = subprocess.run([sys.executable, '-c', code], capture_output=True, text=True, timeout=120)
    return p.returncode, p.stderr + p.stdout


@pytest.mark.parametrize('body,msg', [
    ('q.K = 200; L.det_gemm(ctypes.byref(q), None, None, None, 4, ctypes.c_void_p(16), None)', 'bad shape'),
    ('q.N = 0; L.det_gemm(ctypes.byref(q), None, None, None, 4, ctypes.c_void_p(16), None)', 'bad shape'),
    ('L.det_gemm(ctypes.byref(q), None, None, None, 4, None, None)', 'y == NULL'),
    ('q.bits = 5; L.det_gemm(ctypes.byref(q), None, None, None, 4, ctypes.c_void_p(16), None)', 'unsupported bits'),
    ('o = (ctypes.c_int * 5)(0, 1, 2, 3, 4); L.det_gemm_ex(ctypes.byref(q), None, None, None, 4, None, 0, 5, '
     'ctypes.cast(o, ctypes.c_void_p), None, None)', 'at most 4'),
    ('o = (ctypes.c_int * 2)(3, 10); L.det_gemm_ex(ctypes.byref(q), None, None, None, 4, None, 0, 2, '
     'ctypes.cast(o, ctypes.c_void_p), None, None)', 'column 0'),
    ('L.det_quant(ctypes.c_void_p(16), 2, 200, ctypes.c_void_p(16), ctypes.c_void_p(16), ctypes.c_void_p(16), None)',
     'n % 128'),
    ('L.det_rmsnorm_quant(ctypes.c_void_p(16), ctypes.c_void_p(16), 1e-6, 2, 16384, None, ctypes.c_void_p(16), '
     'ctypes.c_void_p(16), ctypes.c_void_p(16), None)', 'unsupported n'),
    ('L.det_quantize_rows(None, 4, 100, 6, None, None)', 'bad K'),
])
def test_invalid_arguments_abort(body, msg):
    rc, out = run_abort(body)
    assert rc != 0 and 'returned' not in out, out
    assert msg in out, out


def test_empty_batch_is_a_noop():
    rc, out = run_abort('L.det_gemm(ctypes.byref(q), None, None, None, 0, None, None)')
    assert rc == 0 and 'returned' in out, out


def test_bench_refuses_more_than_one_gpu():
    p = subprocess.run([sys.executable, os.path.join(ROOT, 'bench.py'), '--gpus', '2'], capture_output=True, text=True,
                       timeout=120)
    assert p.returncode == 2 and 'one GPU' in p.stderr
