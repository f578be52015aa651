"""Activation quantization parity on the GPU: det_quant / det_rmsnorm_quant / det_silu_mul_quant against the
CPU oracle (codes, multipliers and scales bit for bit).  Rows and shapes follow the reference's norms suite
(crates/det/src/conformance.rs:453-537, Rng seed 3), plus the BASELINE activation rows and K values."""
import numpy as np
import pytest

import oracle
from det_amd import ffi
from tests.helpers import same_f32, same_int, norm_rows, baseline_acts

pytestmark = pytest.mark.gpu

NORM_SHAPES = [(1, 2560), (6, 2560), (33, 4096), (9, 9216), (4, 5120), (3, 17408)]


def gpu_quant(kind, x, u=None, w=None, group=True):
    M, n = x.shape
    xb = ffi.Buf.upload(x)
    q, s = ffi.Buf((M, n), np.int8), ffi.Buf(M, np.float32)
    mb = ffi.Buf((M, n // 128), np.uint16) if group else None
    if kind == 'quant':
        ffi.quant(xb, M, n, q, s, mb)
    elif kind == 'rmsnorm_quant':
        ffi.rmsnorm_quant(xb, ffi.Buf.upload(w), np.float32(1e-6), M, n, q, s, mb)
    else:
        ffi.silu_mul_quant(xb, ffi.Buf.upload(u), M, n, q, s, mb)
    return q.download(), s.download(), (mb.download() if group else None)


def check(name, want, got):
    errs = []
    for what, a, b, f in (('codes', want[0], got[0], same_int), ('multipliers', want[2], got[2], same_int),
                          ('scales', want[1], got[1], same_f32)):
        if a is None:
            continue
        d = f(a, b)
        if d:
            errs.append(f'{name} {what}: {d}')
    return errs


def test_conformance_norms():
    rng = oracle.Rng(3)
    errs = []
    for m, n in NORM_SHAPES:
        print(f'norms m={m} n={n}', flush=True)
        x, u, w = norm_rows(rng, m, n)
        if n <= 8192:
            errs += check(f'rmsnorm_quant m={m} n={n}', oracle.rmsnorm_quant(x, w, np.float32(1e-6)),
                          gpu_quant('rmsnorm_quant', x, w=w))
        errs += check(f'quant m={m} n={n}', oracle.quant(x), gpu_quant('quant', x))
        errs += check(f'silu_mul_quant m={m} n={n}', oracle.silu_mul_quant(x, u), gpu_quant('silu_mul_quant', x, u=u))
    assert not errs, '\n'.join(errs)


@pytest.mark.parametrize('K', [2560, 4096, 5120, 6144, 9728, 17408])
def test_baseline_activation_rows(K):
    """BASELINE activations: N(0,1) rows, every 37th x1e-3, one all-zero row; group and per-row modes."""
    x = baseline_acts(K, 75, K, zero_row=40)
    errs = check(f'quant K={K}', oracle.quant(x), gpu_quant('quant', x))
    errs += check(f'quant_act_i8 K={K}', oracle.quant(x, group=False), gpu_quant('quant', x, group=False))
    assert not errs, '\n'.join(errs)


def test_scale_underflow_rows():
    """smax > 0 but smax/65535 underflows to 0: multipliers become 0 (Rust `NaN as u16`), codes saturate or
    become 0 (Rust `NaN as i8`); plus the mixed denormal/zero groups around it."""
    K = 1024
    x = np.zeros((5, K), np.float32)
    x[0, :] = np.float32(1e-41)
    x[1, 128:256] = np.float32(-3e-43)
    x[1, 5] = np.float32(1e-45)
    x[2, ::2] = np.float32(2e-39)
    x[3, 7] = np.float32(1e-38)
    x[4, :] = np.float32(-0.0)
    errs = check('underflow', oracle.quant(x), gpu_quant('quant', x))
    errs += check('underflow per-row', oracle.quant(x, group=False), gpu_quant('quant', x, group=False))
    assert not errs, '\n'.join(errs)
