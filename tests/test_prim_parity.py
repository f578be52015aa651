"""det_test_prim on the GPU against the oracle's primitives, following the reference's primitive suite
(crates/det/src/conformance.rs:180-345): random, denormal, zero and infinite operands; int64 -> fp32 on crafted
round-half-even ties (own routine, op 5, and the compiler's cast, op 12); saturating fp32 -> int32; treesum."""
import numpy as np
import pytest

import oracle
from det_amd import ffi
from tests.helpers import same_f32

pytestmark = pytest.mark.gpu


def prim_inputs():
    rng = oracle.Rng(1)
    n = 1 << 16
    x = np.zeros(n, np.float32)
    for i in range(n):
        if i % 7 == 0:
            x[i] = np.uint32(rng.next() & 0x00FFFFFF).view(np.float32)
        else:
            x[i] = np.float32(rng.unit()) * np.float32(100.0)
    inf = np.float32(np.inf)
    lhs = [1e-40, inf, 0.0, -1e-42, -inf, 1e-39, 0.0, 1.0, np.finfo(np.float32).tiny, -1e-41, 0.0, -0.0, 3e-39, inf]
    rhs = [inf, 1e-40, 1e-40, 0.0, -1e-39, -inf, 0.0, 1e-40, inf, inf, -0.0, 0.0, 2e-39, inf]
    for i, (a, b) in enumerate(zip(lhs, rhs)):
        x[i] = np.float32(a)
        x[n - 1 - i] = np.float32(b)
    x[len(lhs)] = np.finfo(np.float32).tiny
    x[len(lhs) + 1] = -np.finfo(np.float32).tiny / np.float32(2)
    return rng, x


def test_unary_binary_prims():
    rng, x = prim_inputs()
    n = x.size
    L = oracle.lib()
    errs = []
    ref = {0: L.ora_exp_f, 3: L.ora_sigmoid_f, 4: L.ora_silu_f, 6: L.ora_rint}
    for op, f in ref.items():
        want = np.array([f(float(v)) for v in x], np.float32)
        d = same_f32(want, ffi.test_prim(op, x, 1, n))
        if d:
            errs.append(f'op {op}: {d}')
    ax = np.abs(x)
    d = same_f32(np.sqrt(ax), ffi.test_prim(8, ax, 1, n))
    if d:
        errs.append(f'sqrt: {d}')
    pos = (np.abs(x) + np.float32(1e-30)).astype(np.float32)
    d = same_f32(np.array([L.ora_log_f(float(v)) for v in pos], np.float32), ffi.test_prim(1, pos, 1, n))
    if d:
        errs.append(f'log_f: {d}')
    d = same_f32(np.array([L.ora_softplus_f(float(v)) for v in x], np.float32), ffi.test_prim(2, x, 1, n))
    if d:
        errs.append(f'softplus_f: {d}')
    y = x[::-1]
    with np.errstate(all='ignore'):
        binary = {9: x * y, 10: x + y, 14: x / y, 15: x - y,
                  16: np.array([L.ora_fmax(float(a), float(b)) for a, b in zip(x, y)], np.float32)}
    for op, want in binary.items():
        d = same_f32(want.astype(np.float32), ffi.test_prim(op, x, 1, n))
        if d:
            errs.append(f'op {op}: {d}')
    assert not errs, '\n'.join(errs)


def test_i64_to_f32_ties():
    rng, _ = prim_inputs()
    vals = []
    for i in range((1 << 16) // 2):
        if i % 3 == 0:
            vals.append(np.int64(np.uint64(rng.next()).view(np.int64)) >> np.int64(rng.below(40)))
        else:
            vals.append(np.int64(np.uint64(rng.next()).view(np.int64)) >> np.int64(20))
    for s in range(1, 40):
        for _ in range(300):
            m = (rng.next() & 0x7FFFFF) | 0x800000
            half = 1 << (s - 1)
            for tail in (half, half + 1, half - 1, half | 1, 1, (1 << s) - 1):
                v = (m << s) + tail
                vals += [v, -v]
    v = np.array(vals, np.int64)
    bits = v.view(np.uint32).astype(np.uint32).view(np.float32)     # little endian: (lo, hi) pairs
    want = np.array([oracle.lib().ora_i64_to_f32(int(a)) for a in v], np.float32)
    for op in (5, 12):
        got = ffi.test_prim(op, bits, 1, bits.size)[0::2]
        assert same_f32(want, got) is None, f'op {op}'


def test_saturation_and_treesum():
    big = np.array([3e9, -3e9, 2147483648.0, 2147483520.0, -2147483648.0, -2147483904.0, 1e20, -1e20, np.inf, -np.inf,
                    2.5, -2.5, 3.5, 1e38, -1e38, 4294967296.0], np.float32)
    want = np.array([float(np.clip(np.rint(v), -2**31, 2**31 - 1)) if np.isfinite(v) else (2**31 - 1 if v > 0 else -2**31)
                     for v in big.astype(np.float64)], np.float32)
    assert same_f32(want, ffi.test_prim(13, big, 1, big.size)) is None
    rng = oracle.Rng(99)
    rows = rng.units(8 * 5120)
    for i in range(0, rows.size, 97):
        rows[i] = rng.denorm()
    want = np.array([oracle.lib().ora_treesum(r.ctypes.data, r.size) for r in rows.reshape(8, 5120)], np.float32)
    assert same_f32(want, ffi.test_prim(11, rows, 8, 5120)) is None
    for n in (1, 3, 8, 9, 100, 4096, 8192):
        r = rng.units(2 * n)
        want = np.array([oracle.lib().ora_treesum(q.ctypes.data, n) for q in r.reshape(2, n)], np.float32)
        assert same_f32(want, ffi.test_prim(11, r, 2, n)) is None, n
