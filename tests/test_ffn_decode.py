"""The model runner's one-token FFN path on the GPU through its test hooks: the gate|up GEMV that stores silu_f of
the gate part (det_test_gemv_silu0) and the multiply-only row quantization that follows it (det_test_mul_quant),
against the oracle's GEMM, silu_f (spec/prim.rs:147-149) and silu_mul_quant (cpu.rs:187-211), bit for bit.  Shapes
cover W4, W6 and W8, a fused linear large enough for one K-slice, one small enough that the GEMV splits K across
workgroups, and a part boundary that is not on a 64-row tile edge."""
import ctypes

import numpy as np
import pytest

import oracle
from det_amd import ffi
from tests.helpers import same_f32, same_int

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('bits', [4, 6, 8])
@pytest.mark.parametrize('widths,K', [((640, 640), 2560), ((40, 88), 2560), ((100, 156, 36), 1024)])
def test_gemv_silu0(bits, widths, K):
    print(f'gemv silu0 W{bits} widths={widths} K={K}', flush=True)
    rng = oracle.Rng(31 + bits + K)
    N = sum(widths)
    rows = rng.fake_rows(bits, N, K)
    lin = ffi.Linear(rows, K, bits, widths=widths)
    xq, sx, mx = oracle.quant(rng.acts_x(1, K))
    outs = [ffi.Buf((1, w), np.float32) for w in widths]
    offs = (ctypes.c_int * len(widths))(*np.cumsum([0] + list(widths[:-1])).tolist())
    dsts = (ctypes.c_void_p * len(widths))(*[o.ptr for o in outs])
    xb, sb, mb = ffi.Buf.upload(xq), ffi.Buf.upload(sx), ffi.Buf.upload(mx)     # held until the call returns
    ffi.lib().det_test_gemv_silu0(ctypes.byref(lin.q), xb.ptr, sb.ptr, mb.ptr, len(widths),
                                  ctypes.cast(offs, ctypes.c_void_p), ctypes.cast(dsts, ctypes.c_void_p), None)
    want = oracle.gemm(rows, N, K, bits, xq, sx, mx, widths=list(widths))
    silu = oracle.lib().ora_silu_f
    want[0] = np.array([[silu(float(v)) for v in want[0][0]]], np.float32)
    for p, (o, w) in enumerate(zip(outs, want)):
        d = same_f32(w, o.download())
        assert d is None, f'part {p}: {d}'


@pytest.mark.parametrize('n', [2560, 9728, 17408])
def test_mul_quant_equals_silu_mul_quant(n):
    print(f'mul_quant n={n}', flush=True)
    rng = np.random.default_rng(n)
    g = (rng.standard_normal((1, n)) * 3).astype(np.float32)
    u = rng.standard_normal((1, n)).astype(np.float32)
    g[0, :7] = [0.0, -0.0, 1e-30, -1e-30, 80.0, -80.0, 1e-3]
    silu = oracle.lib().ora_silu_f
    a = np.array([[silu(float(v)) for v in g[0]]], np.float32)
    want = oracle.silu_mul_quant(g, u)
    ab, bb = ffi.Buf.upload(a), ffi.Buf.upload(u)
    xq, sx, mx = ffi.Buf((1, n), np.int8), ffi.Buf(1, np.float32), ffi.Buf((1, n // 128), np.uint16)
    ffi.lib().det_test_mul_quant(ab.ptr, bb.ptr, 1, n, xq.ptr, sx.ptr, mx.ptr, None)
    assert same_int(want[0], xq.download()) is None
    assert same_f32(want[1], sx.download()) is None
    assert same_int(want[2], mx.download()) is None
