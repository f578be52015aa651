"""det_quantize_rows (GPU, binary64) against the oracle's quantize_rows (quantize.rs:33-100), byte for byte,
and the repack round trip of det_linear_repack."""
import numpy as np
import pytest

import oracle
from det_amd import ffi
from tests.helpers import gaussian_weights

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize('bits', [4, 6, 8])
@pytest.mark.parametrize('N,K', [(37, 128), (300, 2560), (64, 17408)])
def test_quantizer_bytes(bits, N, K):
    w = gaussian_weights(N * 7 + K + bits, N, K)
    w[0, :128] = 0.0                    # an all-zero group: scale 1.0
    w[1 % N] *= np.float32(1e-30)       # tiny row
    want = oracle.quantize_rows(w, bits)
    got = ffi.quantize_rows(ffi.Buf.upload(w), N, K, bits).download()
    bad = np.flatnonzero((want != got).any(axis=1))
    assert bad.size == 0, f'{bad.size} rows differ, first {bad[0]}'


def test_quantizer_kat():
    """quantize.rs:108-140 closed-form input through the GPU quantizer equals the oracle's."""
    k = 512
    i = np.arange(k)
    w = ((((i * 7919) % 1000).astype(np.float32) / np.float32(500.0) - np.float32(1.0)) * np.float32(0.05)
         * (np.float32(1.0) + (i // 128).astype(np.float32))).astype(np.float32).reshape(1, k)
    for bits in (4, 6, 8):
        assert (oracle.quantize_rows(w, bits) == ffi.quantize_rows(ffi.Buf.upload(w), 1, k, bits).download()).all()


@pytest.mark.parametrize('bits', [4, 6, 8])
def test_repack_layout(bits):
    """det_linear_repack writes the documented tiled planes: chunk c of tile row r holds bytes [16c, 16c+16) of
    the row's packed group; c and m are gathered per row; rows past N are zero."""
    rng = oracle.Rng(5)
    N, K = 130, 384
    rows = rng.fake_rows(bits, N, K)
    lin = ffi.Linear(rows, K, bits)
    wq, c, m = lin.wq.download(), lin.c.download(), lin.m.download()
    G, GB = K // 128, 4 * {8: 32, 6: 24, 4: 16}[bits]
    T = 2 * ((N + 127) // 128)
    nc = K // 32 * {8: 32, 6: 24, 4: 16}[bits]
    planes = wq.reshape(T, G, GB // 16, 64, 16)
    for n in range(T * 64):
        t, r = divmod(n, 64)
        got = planes[t, :, :, r, :].reshape(-1)
        want = rows[n, :nc] if n < N else np.zeros(nc, np.uint8)
        assert (got == want).all(), n
        assert c.view(np.uint32)[n] == (rows[n, nc:nc + 4].view(np.uint32)[0] if n < N else 0)
        mrow = m.reshape(T, G, 64)[t, :, r]
        assert (mrow == (rows[n, nc + 4:].view('<u2') if n < N else 0)).all()
