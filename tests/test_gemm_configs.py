"""GEMM parity at every BASELINE GEMM config's full shape, every output checked, on the GPU through the C ABI.

* configs[0]/[1]: the W6 K=2560 -> N=9728 linear at M = 1, 64 and 512, and the W8 output head K=2560 -> N=248320
  at M = 1, 16 and 512;
* the 4B layer's linears under the `6,ffn_gate=4,ffn_up=4,ffn_down=4` preset with GDN a|b at W8
  (convert.rs:117), fused projections routed into their parts as the model does (model.rs:180-197, GemmOut::Parts);
* the 27B shapes at W6 and W8.
Weights are seeded N(0, 0.02) quantized by det_quantize_rows (itself byte-exact to det convert's quantizer,
tests/test_quantizer_parity.py; a row sample is re-checked here against the oracle's quantizer).  Activations are
N(0, 1) rows with every 37th row scaled by 1e-3 and one all-zero row, quantized by the oracle
(quant_act_i8g).  Every output of every part is compared bit for bit with det's x86 GEMM restated in C
(oracle/x86_gemm.c, pinned bit for bit to the scalar oracle by tests/test_x86_baseline.py); the scalar oracle
(cpu.rs:142-185) re-checks a row sample (first, middle and last rows of each part) as a second, independent
reference.  The reference suite's own GEMM cases are in tests/test_gemm_parity.py.
"""
import numpy as np
import pytest

import oracle
from det_amd import ffi
from tests.helpers import same_f32, gaussian_weights, baseline_acts

pytestmark = pytest.mark.gpu

# (name, part widths along N, K, bits, token counts)
CONFIG2 = [
    ('w6_9728x2560', (9728,), 2560, 6, (1, 64, 512)),
    ('w8_head_248320x2560', (248320,), 2560, 8, (1, 16, 512)),
]
MS = (1, 16, 512)
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


def sample_rows(width, edge=16, mid=16):
    """First, middle and last rows of a part of `width` rows (all of them when it is small)."""
    if width <= 2 * edge + mid:
        return np.arange(width)
    c = width // 2 - mid // 2
    return np.concatenate([np.arange(edge), np.arange(c, c + mid), np.arange(width - edge, width)])


def quantized_rows(seed, N, K, bits):
    """Seeded N(0, 0.02) weights through det_quantize_rows; 8 rows re-quantized by the oracle must match."""
    w = gaussian_weights(seed, N, K)
    wd = ffi.Buf.upload(w)
    rows = ffi.quantize_rows(wd, N, K, bits).download()
    wd.free()
    pick = np.unique(np.linspace(0, N - 1, 8).astype(int))
    assert (oracle.quantize_rows(w[pick], bits) == rows[pick]).all(), 'det_quantize_rows differs from the oracle'
    return rows


def check_shape(seed, name, widths, K, bits, Ms):
    N = sum(widths)
    rows = quantized_rows(seed, N, K, bits)
    lin = ffi.Linear(rows, K, bits, widths=widths)
    x86 = oracle.X86Linear(rows, N, K, bits)
    offs = np.cumsum([0] + list(widths[:-1]))
    fails = []
    for M in Ms:
        print(f'{name} W{bits} K={K} N={widths} M={M}', flush=True)
        x = baseline_acts(seed + M, M, K, every37=True, zero_row=M // 2 if M > 2 else None)
        xq, sx, mx = oracle.quant(x)
        xb, sb, mb = ffi.Buf.upload(xq), ffi.Buf.upload(sx), ffi.Buf.upload(mx)
        if len(widths) > 1:
            outs = [ffi.Buf((M, w), np.float32) for w in widths]
            ffi.gemm(lin, xb, sb, mb, M, parts=outs)
            got = np.concatenate([o.download() for o in outs], axis=1)
        else:
            y = ffi.Buf((M, N), np.float32)
            ffi.gemm(lin, xb, sb, mb, M, write=y)
            got = y.download()
        want = x86.gemm(xq, sx, mx)
        d = same_f32(want, got)
        if d:
            fails.append(f'{name} M={M} vs x86 restatement: {d}')
        for off, w in zip(offs, widths):
            sel = off + sample_rows(w)
            d = same_f32(oracle.gemm(rows[sel], len(sel), K, bits, xq, sx, mx), got[:, sel])
            if d:
                fails.append(f'{name} part at {off} M={M} vs scalar oracle: {d}')
    return fails


@pytest.mark.parametrize('spec', CONFIG2, ids=[s[0] for s in CONFIG2])
def test_config2_shapes(spec):
    name, widths, K, bits, Ms = spec
    fails = check_shape(3000 + sum(widths) + K, name, widths, K, bits, Ms)
    assert not fails, '\n'.join(fails)


@pytest.mark.parametrize('spec', CONFIG3, ids=[s[0] for s in CONFIG3])
def test_config3_layer(spec):
    name, widths, K, bits = spec
    fails = check_shape(4000 + sum(widths) + K, name, widths, K, bits, MS)
    assert not fails, '\n'.join(fails)


@pytest.mark.parametrize('spec', CONFIG4, ids=[s[0] for s in CONFIG4])
def test_config4_shape(spec):
    name, widths, K, bits = spec
    fails = check_shape(5000 + sum(widths) + K + bits, name, widths, K, bits, MS)
    assert not fails, '\n'.join(fails)
