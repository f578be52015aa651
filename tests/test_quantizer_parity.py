"""det_quantize_rows (GPU, binary64) against the oracle's quantize_rows (quantize.rs:33-100), byte for byte,
and the repack round trip of det_linear_repack."""
import os

import numpy as np
import pytest

import oracle
from det_amd import ffi
from tests.helpers import gaussian_weights, tie_group

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


@pytest.mark.parametrize('bits', [4, 6])
def test_quantizer_tie_takes_the_first(bits):
    """Groups whose scale search ties between two candidates (quantize.rs:50-52, strict <: the first wins), alone
    and inside a Gaussian row, byte for byte against the oracle."""
    w = gaussian_weights(91 + bits, 3, 384)
    w[0] = 0.0
    w[0, :128] = tie_group(bits)
    w[1, 256:] = tie_group(bits, 2.0 ** -12)
    w[2, 128:256] = tie_group(bits, 2.0 ** -20)
    want = oracle.quantize_rows(w, bits)
    got = ffi.quantize_rows(ffi.Buf.upload(w), 3, 384, bits).download()
    assert (want == got).all()


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
    planes = wq[:T * G * GB * 64].reshape(T, G, GB // 16, 64, 16)
    for n in range(T * 64):
        t, r = divmod(n, 64)
        got = planes[t, :, :, r, :].reshape(-1)
        want = rows[n, :nc] if n < N else np.zeros(nc, np.uint8)
        assert (got == want).all(), n
        assert c.view(np.uint32)[n] == (rows[n, nc:nc + 4].view(np.uint32)[0] if n < N else 0)
        mrow = m.reshape(T, G, 64)[t, :, r]
        assert (mrow == (rows[n, nc + 4:].view('<u2') if n < N else 0)).all()


def pf_unpack(words, bits):
    """The kernel's unpack of one lane's prefill words (det_amd/csrc/prefill.hip pf_unpack), as int8 codes scaled
    by 2^SH, in the lane's k order."""
    w = words.astype(np.uint32)
    out = []
    for s in range(4):
        if bits == 8:
            ops = list(w[4 * s:4 * s + 4])
        elif bits == 6:
            d0, d1, d2 = w[3 * s:3 * s + 3]
            lo = np.uint32(0x03030303)
            sp = np.uint32(((((int(d0 & lo) << 2) | int(d1 & lo)) << 2 | int(d2 & lo)) << 2) & 0xffffffff)
            hi = np.uint32(0xfcfcfcfc)
            ops = [d0 & hi, d1 & hi, d2 & hi, sp]
        else:
            n0, n1 = w[2 * s:2 * s + 2]
            hi = np.uint32(0xf0f0f0f0)
            ops = [n0 & hi, np.uint32((int(n0) << 4) & 0xffffffff) & hi, n1 & hi, np.uint32((int(n1) << 4) & 0xffffffff) & hi]
        out.append(np.array(ops, np.uint32).view(np.int8))
    return np.concatenate(out).astype(np.int64)


@pytest.mark.skipif(os.environ.get('DET_PREFILL') != 'streamk',
                    reason='the prefill planes exist only when DET_PREFILL=streamk selects the kernel that reads them')
@pytest.mark.parametrize('bits', [4, 6, 8])
def test_prefill_planes(bits):
    """det_linear_repack's prefill planes (after the decode tiles): per 32-row block and group, lane l (row l % 32,
    half h = l / 32) holds the codes of k = 32 (i / 16) + 16 h + i % 16, i < 64, and the kernel's unpack of them
    gives 2^SH times the det codes (spec/quant.rs:63-97 via the oracle's unpack); rows past N give zero."""
    rng = oracle.Rng(9)
    N, K = 150, 384
    rows = rng.fake_rows(bits, N, K)
    lin = ffi.Linear(rows, K, bits)
    wq = lin.wq.download()
    G = K // 128
    NP, SH = {8: (4, 0), 6: (3, 2), 4: (2, 4)}[bits]
    nb32 = 4 * ((N + 127) // 128)
    pf = wq[wq.size // 2:].reshape(nb32, G, NP, 64, 16)     # the planes follow the decode tiles (same size)
    nc = K // 32 * {8: 32, 6: 24, 4: 16}[bits]
    codes = np.zeros((nb32 * 32, K), np.int64)
    for n in range(N):
        codes[n] = oracle.unpack_row(rows[n, :nc], bits, K)
    i = np.arange(64)
    for b in range(nb32):
        for g in range(G):
            for l in range(64):
                r, h = l % 32, l // 32
                words = pf[b, g, :, l, :].reshape(-1).view('<u4')
                got = pf_unpack(words, bits)
                want = codes[b * 32 + r, g * 128 + 32 * (i // 16) + 16 * h + i % 16] << SH
                assert (got == want).all(), (b, g, l)
