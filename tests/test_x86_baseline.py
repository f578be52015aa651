"""The CPU baseline's GEMM (oracle/x86_gemm.c, det's x86 backend algorithm: crates/det/src/x86/gemm.rs) against
the scalar oracle, bit for bit, on both dot-product paths (AVX2 vpmaddubsw and AVX-VNNI vpdpbusd where the CPU has
it): rows and tokens that do not fill a strip pair or a 4-token tile, K across the 1024-k chunks, no activation
group multipliers, and the extreme codes and multipliers."""
import numpy as np
import pytest

import oracle
from tests.helpers import same_f32

PATHS = [0, 1] if oracle.has_vnni() else [0]


@pytest.mark.parametrize('bits', [8, 6, 4])
@pytest.mark.parametrize('vnni', PATHS)
def test_x86_gemm_matches_oracle(bits, vnni):
    rng = oracle.Rng(900 + bits)
    for N, K, M in ((1, 128, 1), (37, 1280, 70), (200, 384, 3), (64, 2560, 129), (17, 3072, 5)):
        rows = rng.fake_rows(bits, N, K)
        xq, sx, mx = oracle.quant(rng.acts_x(M, K))
        X = oracle.X86Linear(rows, N, K, bits)
        assert same_f32(oracle.gemm(rows, N, K, bits, xq, sx, mx), X.gemm(xq, sx, mx, vnni=vnni)) is None, (N, K, M)
        assert same_f32(oracle.gemm(rows, N, K, bits, xq, sx, None), X.gemm(xq, sx, None, vnni=vnni)) is None, (N, K, M)


@pytest.mark.parametrize('bits', [8, 6, 4])
@pytest.mark.parametrize('vnni', PATHS)
def test_x86_gemm_extremes(bits, vnni):
    """Every code at its most negative value, multipliers 65535 and activations at -127: the largest group partials
    and int64 products of the format."""
    N, K, M = 24, 1152, 6
    qmin = {8: -128, 6: -32, 4: -8}[bits]
    codes = np.full((N, K), qmin, np.int8)
    codes[1::2] = {8: 127, 6: 31, 4: 7}[bits]
    packed = np.stack([oracle.pack(codes[n], bits) for n in range(N)])
    G = K // 128
    tail = np.zeros((N, 4 + 2 * G), np.uint8)
    tail[:, :4] = np.frombuffer(np.float32(1e-9).tobytes(), np.uint8)
    tail[:, 4:] = np.frombuffer(np.full(G, 65535, np.uint16).tobytes(), np.uint8)
    rows = np.concatenate([packed, tail], axis=1)
    xq = np.full((M, K), -127, np.int8)
    xq[1] = 127
    sx = np.ones(M, np.float32)
    mx = np.full((M, G), 65535, np.uint16)
    X = oracle.X86Linear(rows, N, K, bits)
    assert same_f32(oracle.gemm(rows, N, K, bits, xq, sx, mx), X.gemm(xq, sx, mx, vnni=vnni)) is None
