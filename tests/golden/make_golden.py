"""Writes the golden fixtures of the quantized-linear path (tests/golden/*.npz).

The reference ships no stored vectors for this path (its conformance suite compares backends against its CPU
backend on freshly generated inputs, crates/det/src/conformance.rs).  These fixtures are produced by the C
restatement (oracle/det_oracle.c) and accepted only when the independent numpy restatement written from
docs/SPEC.md (oracle/spec_np.py) agrees bit for bit.  Inputs follow the reference suite's Rng and row classes.

    python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

import oracle  # noqa: E402
from oracle import spec_np  # noqa: E402


def same(a, b):
    a, b = np.asarray(a), np.asarray(b)
    if a.dtype == np.float32:
        return (a.view(np.uint32) == b.view(np.uint32)).all()
    return (a == b).all()


def main():
    out = {}
    # GEMM: every width, conformance-style random codes (incl. W8 -128) and multipliers, mixed-scale activations
    rng = oracle.Rng(2024)
    for bits in (8, 6, 4):
        for n, k, m in ((24, 256, 3), (16, 384, 9)):
            rows = rng.fake_rows(bits, n, k)
            x = rng.acts_x(m, k)
            x[0, :128] = 0.0                       # a zero group
            xq, sx, mx = oracle.quant(x)
            y = oracle.gemm(rows, n, k, bits, xq, sx, mx)
            assert same(y, spec_np.gemm(rows, bits, k, xq, sx, mx)), (bits, n, k, m)
            acc0 = rng.units(m * n).reshape(m, n)
            ya = oracle.gemm(rows, n, k, bits, xq, sx, mx, y=acc0, accumulate=True)
            assert same(ya, (acc0 + spec_np.gemm(rows, bits, k, xq, sx, mx)).astype(np.float32))
            tag = f'gemm_w{bits}_{n}x{k}_m{m}'
            out.update({f'{tag}_rows': rows, f'{tag}_x': x, f'{tag}_y': y, f'{tag}_acc0': acc0, f'{tag}_yacc': ya})
    # activation quantization on the reference's norm row classes (denormal, zero, tiny, mixed)
    from tests.helpers import norm_rows
    qr = oracle.Rng(3)
    x, u, w = norm_rows(qr, 6, 1024)
    for name, group in (('quant_g', True), ('quant_row', False)):
        xq, sx, mx = oracle.quant(x, group=group)
        if group:
            xq2, sx2, mx2 = spec_np.quant_act_i8g(x)
            assert same(mx, mx2)
        else:
            xq2, sx2 = spec_np.quant_act_i8(x)
        assert same(xq, xq2) and same(sx, sx2), name
        out[f'{name}_x'] = x
        out[f'{name}_xq'] = xq
        out[f'{name}_sx'] = sx
        if group:
            out[f'{name}_mx'] = mx
    # weight quantizer: the reference KAT input (quantize.rs:108-140) and seeded Gaussian rows
    i = np.arange(512)
    kat = ((((i * 7919) % 1000).astype(np.float32) / np.float32(500.0) - np.float32(1.0)) * np.float32(0.05)
           * (np.float32(1.0) + (i // 128).astype(np.float32))).astype(np.float32).reshape(1, 512)
    gauss = (np.random.default_rng(7).standard_normal((6, 384), dtype=np.float32) * np.float32(0.02))
    gauss[1, 128:256] = 0.0
    for bits in (4, 6, 8):
        for nm, wts in (('kat', kat), ('gauss', gauss)):
            r = oracle.quantize_rows(wts, bits)
            assert same(r, spec_np.quantize_rows(wts, bits)), (bits, nm)
            out[f'quantize_{nm}_w{bits}_w'] = wts
            out[f'quantize_{nm}_w{bits}_rows'] = r
    path = os.path.join(HERE, 'quantized_linear.npz')
    np.savez_compressed(path, **out)
    print(f'wrote {path}: {len(out)} arrays, {os.path.getsize(path)} bytes')


if __name__ == '__main__':
    main()
