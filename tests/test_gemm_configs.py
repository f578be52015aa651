"""GEMM parity at the BASELINE configs' full layer shapes (configs 3 and 4), on the GPU through the C ABI.

Config 3 is the 4B model's linears under the `6,ffn_gate=4,ffn_up=4,ffn_down=4` preset with GDN a|b at W8
(convert.rs:117); fused projections are routed into their parts as the model does (model.rs:180-197, GemmOut::Parts).
Config 4 is the 27B shapes at W6 and W8.  Every shape runs at M = 1, 16 and 512 (decode, the matrix-core decode and
prefill kernels).  The oracle evaluates a fixed subset of output rows of every part (its first, middle and last
rows), bit for bit; the inputs are the reference suite's fake det rows and activations (conformance.rs:104-160).
"""
import numpy as np
import pytest

import oracle
from det_amd import ffi
from tests.helpers import same_f32

pytestmark = pytest.mark.gpu

# (name, part widths along N, K, bits)
CONFIG3 = [
    ('attn_qkv', (8192, 1024, 1024), 2560, 6),
    ('attn_o', (2560,), 4096, 6),
    ('gdn_qkvz', (8192, 4096), 2560, 6),
    ('gdn_ab', (32, 32), 2560, 8),
    ('gdn_out', (2560,), 4096, 6),
    ('ffn_gate_up', (9728, 9728), 2560, 4),
    ('ffn_down', (2560,), 9728, 4),
]
CONFIG4 = [(f'{name}_w{bits}', (n,), k, bits)
           for bits in (6, 8) for name, n, k in (('ffn_up', 17408, 5120), ('ffn_down', 5120, 17408), ('attn_o', 5120, 6144))]
MS = (1, 16, 512)


def sample_rows(width, edge=48, mid=32):
    """First, middle and last rows of a part of `width` rows (all of them when it is small)."""
    if width <= 2 * edge + mid:
        return np.arange(width)
    c = width // 2 - mid // 2
    return np.concatenate([np.arange(edge), np.arange(c, c + mid), np.arange(width - edge, width)])


def check_shape(seed, name, widths, K, bits):
    rng = oracle.Rng(seed)
    N = sum(widths)
    rows = rng.fake_rows(bits, N, K)
    lin = ffi.Linear(rows, K, bits, widths=widths)
    offs = np.cumsum([0] + list(widths[:-1]))
    fails = []
    for M in MS:
        print(f'{name} W{bits} K={K} N={widths} M={M}', flush=True)
        xq, sx, mx = oracle.quant(rng.acts_x(M, K))
        xb, sb, mb = ffi.Buf.upload(xq), ffi.Buf.upload(sx), ffi.Buf.upload(mx)
        if len(widths) > 1:
            outs = [ffi.Buf((M, w), np.float32) for w in widths]
            ffi.gemm(lin, xb, sb, mb, M, parts=outs)
            got = [o.download() for o in outs]
        else:
            y = ffi.Buf((M, N), np.float32)
            ffi.gemm(lin, xb, sb, mb, M, write=y)
            got = [y.download()]
        for p, (off, w) in enumerate(zip(offs, widths)):
            sel = sample_rows(w)
            want = oracle.gemm(rows[off + sel], len(sel), K, bits, xq, sx, mx)
            d = same_f32(want, got[p][:, sel])
            if d:
                fails.append(f'{name} part {p} M={M}: {d}')
    return fails


@pytest.mark.parametrize('spec', CONFIG3, ids=[s[0] for s in CONFIG3])
def test_config3_layer(spec):
    name, widths, K, bits = spec
    fails = check_shape(4000 + sum(widths) + K, name, widths, K, bits)
    assert not fails, '\n'.join(fails)


@pytest.mark.parametrize('spec', CONFIG4, ids=[s[0] for s in CONFIG4])
def test_config4_shape(spec):
    name, widths, K, bits = spec
    fails = check_shape(5000 + sum(widths) + K + bits, name, widths, K, bits)
    assert not fails, '\n'.join(fails)
