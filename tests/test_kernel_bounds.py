"""Bounds of the buffer-unit copies the HIP kernels issue through inline assembly (CPU only).

The global->LDS copies in det_amd/csrc/gemm.hip are `buffer_load_dwordx4 ... offen lds` in inline assembly, so the
compiler checks nothing about them.  This test restates their address arithmetic for k_prefill2 (activation and
weight runs, multiplier loads) and k_decode_ms (activation runs) and applies the buffer unit's rules: the per-lane
offset plus the instruction offset is checked against the resource's size (a lane past it reads zero), the scalar
offset is not checked.  Every byte a lane can reach must lie inside its allocation and every LDS byte it writes
inside its array, over many shapes, including partial token blocks.  A change to that arithmetic in gemm.hip must be
made here too.
"""
import itertools

import numpy as np
import pytest

GROUP, TILE_N, P2_BM = 128, 64, 128
NC = {4: 4, 6: 6, 8: 8}               # 1 KB planes per tile-group


def reached(base, voff, inst, soff, nrec, nbytes=16):
    """Byte ranges a copy can touch: (lo, hi) per lane that passes the range check, relative to the allocation."""
    voff = np.asarray(voff, np.int64)
    ok = voff + inst + nbytes <= nrec
    part = (voff + inst < nrec) & ~ok
    assert not part.any(), 'a lane straddles the end of its resource'
    lo = base + soff + voff[ok] + inst
    return lo, lo + nbytes


def check_in(lo, hi, size, what):
    if len(lo):
        assert lo.min() >= 0 and hi.max() <= size, f'{what}: bytes [{lo.min()}, {hi.max()}) of {size}'


def prefill2_copies(N, K, M, bits):
    G = K // GROUP
    T = 2 * ((N + 127) // 128)
    nbn, nbt = (N + TILE_N - 1) // TILE_N, (M + P2_BM - 1) // P2_BM
    nc, wb = NC[bits], NC[bits] * 1024
    lane = np.arange(64)
    xq_size, wq_size, mx_size, ms_size = M * K, T * G * wb, M * G * 2, T * G * TILE_N * 2
    for nb, tb, g, wv in itertools.product(range(nbn), range(nbt), sorted({0, G // 2, G - 1}), range(4)):
        t0 = tb * P2_BM
        # activations: copy i through resource xq + 8iK - 1024i of size (M - 8i)K + 1024i, per-lane offset a_vo or
        # a_vo ^ 64 (odd copies), instruction offset 1024 i, scalar offset g * 128; LDS As + 4096 wv + 1024 i + 16 lane
        a_vo = (t0 + wv * 32 + (lane >> 3)) * K + (((lane & 7) ^ (lane >> 4)) * 16)
        for i in range(4):
            nrec = (M - 8 * i) * K + 1024 * i if M > 8 * i else 0
            voff = a_vo if i % 2 == 0 else a_vo ^ 64
            lo, hi = reached(8 * i * K - 1024 * i, voff, 1024 * i, g * GROUP, nrec)
            check_in(lo, hi, xq_size, f'prefill2 A copy {i} N={N} K={K} M={M} tb={tb} wv={wv} g={g}')
            lds = 4096 * wv + 1024 * i + 16 * lane
            assert lds.max() + 16 <= P2_BM * 128
        # W8 codes: resource wq + nb G WB of size G WB, per-lane offset 16 lane, the wave's planes 2 wv, 2 wv + 1;
        # W4/W6 codes: plain loads of block wv of row lane, two groups ahead (into registers)
        if bits == 8:
            for i in range(2):
                lo, hi = reached(nb * G * wb, 16 * lane, 1024 * i, g * wb + wv * 2048, G * wb)
                check_in(lo, hi, wq_size, f'prefill2 W copy N={N} K={K}')
                assert wv * 2048 + 1024 * i + 16 * 63 + 16 <= wb
        else:
            check_code_loads(bits, nb * G * wb + g * wb + lane * 16, np.full(64, wv), wq_size)
        # multipliers: mx through a resource of size M G 2 at per-lane offset (t0 + tid) G 2, scalar offset 2 g;
        # m through a resource of size (nb + 1) G 128 at (nb G 64 + row) 2, scalar offset 128 g
        tid = 64 * wv + lane
        if wv < 2:
            lo, hi = reached(0, (t0 + tid) * G * 2, 0, 2 * g, mx_size, 2)
            check_in(lo, hi, mx_size, 'prefill2 mx load')
        elif wv == 2:
            lo, hi = reached(0, (nb * G * 64 + (tid - P2_BM)) * 2, 0, 128 * g, (nb + 1) * G * 128, 2)
            check_in(lo, hi, ms_size, 'prefill2 m load')


def check_code_loads(bits, base, blk, wq_size):
    """Per-lane loads of one 32-code block blk of a row whose tile-group slot starts at base (plane c of the group
    at + 1024 c): in bounds, aligned, and exactly bytes BPL blk .. BPL blk + BPL - 1 of the row's group, in the
    word order the unpack takes (W6 odd blocks: the 8-byte load's words first)."""
    bpl = {4: 16, 6: 24, 8: 32}[bits]
    if bits == 4:
        spans = [(blk * 1024, 16)]
    elif bits == 8:
        spans = [(2 * blk * 1024, 16), ((2 * blk + 1) * 1024, 16)]
    else:   # v (words 0-3), w (words 4-5)
        pp = 3 * (blk >> 1)
        spans = [((pp + 2 * (blk & 1)) * 1024, 16), ((pp + 1) * 1024 + 8 * (blk & 1), 8)]
    for rel, n in spans:
        off = base + rel
        assert off.min() >= 0 and (off + n).max() <= wq_size, f'code load W{bits}'
        assert (off % n == 0).all(), 'unaligned code load'
    # row-group byte of each loaded byte: plane c byte j is byte 16 c + j
    grp = [16 * (rel // 1024) + rel % 1024 + np.arange(n)[:, None] for rel, n in spans]
    if bits == 6:
        words = np.where((blk & 1).astype(bool), np.concatenate([grp[1], grp[0]]), np.concatenate(grp))
    else:
        words = np.concatenate(grp)
    assert (words == bpl * blk + np.arange(bpl)[:, None]).all(), 'lane block bytes'


def decode_ms_copies(N, K, M, ts, KS=1):
    """k_decode_ms: token block y (tokens t0 = 32 ts y ..) copies through a resource based at xq + t0 K whose range
    is its own M - t0 rows; K-slice planes and counters are indexed by the block as well."""
    G = K // GROUP
    mt = 32 * ts
    ncp = mt // 16
    T = (N + TILE_N - 1) // TILE_N
    NB = (M + mt - 1) // mt
    lane = np.arange(64)
    for tbk in range(NB):
        t0, Mb = tbk * mt, M - tbk * mt
        assert Mb >= 1
        for hf, g in itertools.product(range(2), sorted({0, G - 1})):
            R = (mt // 2) * hf + 8 * np.arange(ncp)[:, None] + (lane >> 3)[None, :]
            xvo = R * K + (((lane & 7)[None, :] ^ ((R >> 1) & 7)) * 16) - 1024 * (np.arange(ncp)[:, None] & 3)
            for c0 in range(0, ncp, 4):
                n = 4 if ncp - c0 >= 4 else 2
                for j in range(n):
                    lo, hi = reached(t0 * K, xvo[c0 + j], 1024 * j, g * GROUP, Mb * K)
                    check_in(lo, hi, M * K, f'decode_ms copy N={N} K={K} M={M} block={tbk} hf={hf}')
                    lds = (mt // 2) * hf * 128 + c0 * 1024 + 1024 * j + 16 * lane
                    assert lds.max() + 16 <= mt * 128
        # token multipliers mx[t0 + lane][g] for lane < min(M - t0, MT); sx[t0 + min(lane, M - t0 - 1)]
        tl = lane[lane < min(Mb, mt)]
        assert ((t0 + tl) * G + G - 1).max() < M * G and t0 + min(63, Mb - 1) < M
        # K-slice planes part[NB][KS][MT][T * 64] and counters cnt[NB][T]
        npad = T * TILE_N
        for ks in range(KS):
            idx = ((tbk * KS + ks) * mt + np.arange(min(Mb, mt))[:, None]) * npad + np.arange(npad)
            assert idx.max() < NB * KS * mt * T * TILE_N
        assert tbk * T + T - 1 < NB * T


SHAPES = [(640, 2560), (9728, 2560), (2560, 9728), (200, 384), (48, 128), (17408, 5120), (5120, 17408)]


@pytest.mark.parametrize('bits', [4, 6, 8])
@pytest.mark.parametrize('N,K', SHAPES)
def test_prefill2_copies_in_bounds(N, K, bits):
    for M in (65, 100, 128, 300, 512):
        prefill2_copies(N, K, M, bits)


@pytest.mark.parametrize('N,K', SHAPES)
def test_decode_ms_copies_in_bounds(N, K):
    for M, ts in ((17, 1), (20, 1), (32, 1), (33, 2), (50, 2), (64, 2), (33, 1), (50, 1), (64, 1)):
        decode_ms_copies(N, K, M, ts, KS=1 if K < 4096 else 3)


def test_scalar_offset_is_not_checked():
    """The rule the test applies: a copy whose scalar offset walks past the resource's size reads past it, which is
    what a copy of a partial block must never do (the first multiplier-copy variant of the prefill did)."""
    lo, hi = reached(0, np.arange(64) * 16, 0, 4096, 4000)
    assert hi.max() > 4000
