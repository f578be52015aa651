"""CPU checks of the prefill kernel's host-independent logic (det_amd/csrc/prefill.hip), restated here:

* the prefill-plane packing of k_repack_pf and the kernel's unpack (pf_unpack) are inverse: every signed code of
  every width comes back scaled by 2^SH, at the k the MFMA step expects;
* the stream-K split: the workgroup ranges partition the units, pf_owner names the workgroup of every unit, the
  partial-tile slots of split fragments are distinct and inside the 2 P slots the host allocates, the arrival count
  that marks the last fragment equals the tile's fragment count, and the host's no-split test is exact;
* every memory access of k_prefill and k_repack_pf stays inside its allocation (buffer-unit rule: per-lane offset
  plus instruction offset checked against the resource size, scalar offset unchecked), over shapes with partial
  token and row tiles.
A change to that arithmetic in prefill.hip must be made here too.
"""
import itertools

import numpy as np
import pytest

from tests.test_kernel_bounds import reached, check_in
from tests.test_quantizer_parity import pf_unpack

GROUP = 128
NP = {8: 4, 6: 3, 4: 2}
SH = {8: 0, 6: 2, 4: 4}


def pack_lane(c, bits):
    """k_repack_pf: one lane's 64 codes (k order of the lane) -> 4 NP words."""
    q = []
    for s in range(4):
        cs = c[16 * s:16 * s + 16]
        if bits == 8:
            for d in range(4):
                q.append(sum((int(cs[4 * d + j]) & 255) << (8 * j) for j in range(4)))
        elif bits == 6:
            for i in range(3):
                q.append(sum((((int(cs[4 * i + j]) & 63) << 2) | ((int(cs[12 + j]) >> (4 - 2 * i)) & 3)) << (8 * j)
                             for j in range(4)))
        else:
            for i in range(2):
                q.append(sum((((int(cs[8 * i + j]) & 15) << 4) | (int(cs[8 * i + 4 + j]) & 15)) << (8 * j)
                             for j in range(4)))
    return np.array(q, np.uint32)


@pytest.mark.parametrize('bits', [4, 6, 8])
def test_pack_unpack_inverse(bits):
    qmax = (1 << (bits - 1)) - 1
    lo = -qmax - 1
    rng = np.random.default_rng(bits)
    cases = [np.arange(64) % (qmax - lo + 1) + lo, np.full(64, lo), np.full(64, qmax), np.zeros(64, np.int64)]
    cases += [rng.integers(lo, qmax + 1, 64) for _ in range(200)]
    for c in cases:
        got = pf_unpack(pack_lane(c, bits), bits)
        assert (got == np.asarray(c, np.int64) << SH[bits]).all()
        assert np.abs(got).max() <= 128
    # |p| bound of the scaled codes: 128 * 127 * 128 < 2^21 at every width
    assert 128 * 127 * (qmax + 1) << SH[bits] <= 128 * 127 * 128 < 1 << 21


def owner(u, total, P):
    return ((u + 1) * P + total - 1) // total - 1


def ranges(total, P):
    return [(w * total // P, (w + 1) * total // P) for w in range(P)]


def host_P(total, cus):
    P = min(2 * cus, max(1, total // 4))
    if P > 8:
        P &= ~7
    return P


def fragments(tiles, G, P):
    total = tiles * G
    out = []
    for w, (u0, u1) in enumerate(ranges(total, P)):
        u = u0
        while u < u1:
            tile = u // G
            ga = u - tile * G
            gb = min(G, u1 - tile * G)
            out.append((w, tile, ga, gb))
            u = tile * G + gb
    return out


@pytest.mark.parametrize('tiles,G', [(304, 20), (1, 20), (3, 1), (7760, 20), (80, 32), (40, 136), (76, 76), (2, 2),
                                     (5, 48), (160, 80), (8, 8)])
@pytest.mark.parametrize('cus', [256, 80, 4])
def test_stream_k_bookkeeping(tiles, G, cus):
    total = tiles * G
    P = host_P(total, cus)
    fr = fragments(tiles, G, P)
    # the ranges partition the units in order; fragments partition each tile's groups
    seen = np.zeros(total, np.int64)
    for w, tile, ga, gb in fr:
        assert 0 <= ga < gb <= G
        seen[tile * G + ga:tile * G + gb] += 1
        for u in (tile * G + ga, tile * G + gb - 1):
            assert owner(u, total, P) == w
    assert (seen == 1).all()
    split = total % P != 0 or (total // P) % G != 0
    slots = set()
    for w, tile, ga, gb in fr:
        whole = ga == 0 and gb == G
        if not whole:
            assert split, 'a split fragment without the partial buffer'
            wf, wl = owner(tile * G, total, P), owner(tile * G + G - 1, total, P)
            assert wf <= w <= wl
            nfrag = sum(1 for f in fr if f[1] == tile)
            assert nfrag == wl - wf + 1
            first_tile = (w * total // P) // G
            slot = 2 * w + (0 if first_tile == tile else 1)
            assert slot not in slots and 0 <= slot < 2 * P
            slots.add(slot)
    # a workgroup has at most two split fragments (its first and its last)
    for w in range(P):
        mine = [f for f in fr if f[0] == w and not (f[2] == 0 and f[3] == G)]
        assert len(mine) <= 2


def prefill_accesses(N, K, M, bits, cus=256):
    G = K // GROUP
    nbn, nbt = (N + 127) // 128, (M + 127) // 128
    tiles = nbn * nbt
    total = tiles * G
    P = host_P(total, cus)
    np_ = NP[bits]
    T64 = 2 * nbn
    pf_size = T64 * G * 64 * 4 * {8: 32, 6: 24, 4: 16}[bits]      # the prefill planes
    m_size, mx_size, x_size = T64 * G * 64 * 2, M * G * 2, M * K
    lane = np.arange(64)
    for w, tile, ga, gb in fragments(tiles, G, P):
        nb, tb = divmod(tile, nbt)
        t0, n0 = tb * 128, nb * 128
        for g in sorted({ga, (ga + gb) // 2, gb - 1}):
            for wv in range(4):
                # activations: one resource of M K bytes; copy i at avo[i] + 1024 i, scalar offset 128 g
                for i in range(4):
                    row = t0 + wv * 32 + 8 * i + (lane >> 3)
                    avo = row * K - 1024 * i + (((lane & 7) ^ (((i & 1) << 2) | (lane >> 4))) * 16)
                    assert (avo >= 0).all()
                    lo, hi = reached(0, avo, 1024 * i, GROUP * g, x_size)
                    check_in(lo, hi, x_size, f'prefill A copy N={N} K={K} M={M}')
                    # the chunk a lane lands must be chunk (p ^ ((R/2) % 8)) of its token row R
                    R = wv * 32 + 8 * i + (lane >> 3)
                    p = lane & 7
                    assert ((avo + 1024 * i - row * K) // 16 == (p ^ ((R >> 1) & 7))).all()
                    assert 4096 * wv + 1024 * i + 16 * lane.max() + 16 <= 128 * 128
                # codes: block resource of G NP 1 KB at (nb 4 + wv) G NP 1 KB, per-lane 16 lane, offsets 1 KB p
                blk = nb * 4 + wv
                for pl in range(np_):
                    lo, hi = reached(blk * G * np_ * 1024, lane * 16, 1024 * pl, g * np_ * 1024, G * np_ * 1024)
                    check_in(lo, hi, pf_size, 'prefill code load')
                    assert (lo >= blk * G * np_ * 1024).all() and (hi <= (blk + 1) * G * np_ * 1024).all()
                # multipliers: waves 0-1 m of row n0 + sidx, waves 2-3 mx of token t0 + sidx
                sidx = (64 * wv + lane) & 127
                if wv < 2:
                    n = n0 + sidx
                    vo = ((n >> 6) * G * 64 + (n & 63)) * 2 + 128 * g
                    lo, hi = reached(0, vo, 0, 0, nbn * 2 * G * 128, 2)
                    check_in(lo, hi, m_size, 'prefill m load')
                    assert len(lo) == 64
                else:
                    vo = (t0 + sidx) * G * 2 + 2 * g
                    lo, hi = reached(0, vo, 0, 0, mx_size, 2)
                    check_in(lo, hi, mx_size, 'prefill mx load')
                    assert len(lo) == int(((t0 + sidx) < M).sum())


SHAPES = [(640, 2560), (9728, 2560), (2560, 9728), (200, 384), (48, 128), (5120, 17408), (64, 2560)]


@pytest.mark.parametrize('bits', [4, 6, 8])
@pytest.mark.parametrize('N,K', SHAPES)
def test_prefill_accesses_in_bounds(N, K, bits):
    for M in (65, 300, 512):
        prefill_accesses(N, K, M, bits)


def store4_targets(N, nparts, offs, t, n):
    """prefill.hip store4 restated: the (part, flat index) each of columns n .. n + 3 of token t is written to, and
    whether the 16-byte path is taken (base pointers taken as 16-byte aligned, as det_malloc's are)."""
    if nparts <= 1:
        part, lo, width = 0, 0, N
    else:
        part, lo, hi = 0, offs[0], offs[1]
        for j in range(1, 4):
            if j < nparts and n >= offs[j]:
                part, lo, hi = j, offs[j], offs[j + 1]
        width = hi - lo
    vec = n - lo + 4 <= width and (n - lo) % 4 == 0 and width % 4 == 0
    if vec:
        return [(part, t * width + (n - lo) + e) for e in range(4)], True
    out = []
    for e in range(4):                      # the scalar path routes each column on its own (Out::ptr)
        c = n + e
        if c >= N:
            continue
        if nparts <= 1:
            out.append((0, t * N + c))
            continue
        p, l, h = 0, offs[0], offs[1]
        for j in range(1, 4):
            if j < nparts and c >= offs[j]:
                p, l, h = j, offs[j], offs[j + 1]
        out.append((p, t * (h - l) + (c - l)))
    return out, False


@pytest.mark.parametrize('widths', [(256,), (200,), (130, 126), (100, 36, 164), (8192, 1024, 1024), (32, 32),
                                    (3, 5, 7, 9), (1024, 3)])
def test_epilogue_routing(widths):
    """Every column of every token is written exactly once, into the part GemmOut::Parts assigns it
    (backend.rs:138-142: column n in [offs[i], offs[i+1]) goes to dst[i][t][n - offs[i]]), inside that part."""
    N = sum(widths)
    nparts = len(widths)
    offs = list(np.cumsum([0] + list(widths))) + [0] * (5 - nparts - 1)
    M = 3
    hits = {}
    for t in range(M):
        for n0 in range(0, ((N + 127) // 128) * 128, 32):           # wave slabs of 32 rows
            for c4 in range(0, 32, 4):
                n = n0 + c4
                if n >= N:
                    continue
                tg, _ = store4_targets(N, nparts, offs, t, n)
                for tgt in tg:
                    hits[tgt] = hits.get(tgt, 0) + 1
    want = {}
    for t in range(M):
        for c in range(N):
            if nparts <= 1:
                want[(0, t * N + c)] = 1
            else:
                i = max(j for j in range(nparts) if c >= offs[j])
                want[(i, t * widths[i] + c - offs[i])] = 1
    assert hits == want


GB = {8: 128, 6: 96, 4: 64}          # packed bytes of one 128-group
BPL = {8: 32, 6: 24, 4: 16}          # packed bytes of one 32-code block


@pytest.mark.parametrize('bits', [4, 6, 8])
@pytest.mark.parametrize('N,K', SHAPES + [(248320, 2560), (1, 128), (129, 256), (4097, 384)])
def test_repack_writes_in_bounds(N, K, bits):
    """det_linear_repack's two kernels, restated at the extremes of their index ranges: k_repack (decode tiles, c, m)
    and k_repack_pf (prefill planes) write only inside the wq / c / m sizes det_linear_sizes reports, the two wq
    regions are disjoint and together cover wq exactly, and rows are read only for n < N."""
    import os
    from det_amd import ffi
    if not os.path.exists(ffi.LIB_PATH):
        pytest.skip('libdet_hip.so not built')
    wq_dec, c_bytes, m_bytes = ffi.linear_sizes(N, K, bits)
    G = K // GROUP
    T = 2 * ((N + 127) // 128)                              # 64-row tiles, whole pairs
    pf_offset = T * G * GB[bits] * 64                       # prefill.hip pf_offset
    # without DET_PREFILL=streamk (this process) wq holds the decode tiles only; with it, the prefill planes follow
    # and wq is twice as large (test_linear_sizes_with_streamk checks that size in a child process)
    assert wq_dec == pf_offset
    wq_bytes = 2 * pf_offset
    rb = K // 32 * BPL[bits] + 4 + 2 * G
    # k_repack: idx < nchunks = pf_offset / 16; lane r = idx % 64, chunk c, group g, tile
    nchunks = pf_offset // 16                               # (wq_bytes / 16 would overrun m and c)
    NC = GB[bits] // 16
    last = nchunks - 1
    assert 16 * last + 16 == pf_offset <= wq_bytes
    tg_max = (last >> 6) // NC
    assert (tg_max * 64 + 63) * 2 + 2 <= m_bytes                       # ms[tg * 64 + r]
    tile_max = tg_max // G
    assert (tile_max * 64 + 63) * 4 + 4 <= c_bytes                      # cs[n], n = tile * 64 + r
    n_read = min(tile_max * 64 + 63, N - 1)                             # rows read only for n < N
    assert n_read * rb + (G - 1) * GB[bits] + (NC - 1) * 16 + 16 <= N * rb
    assert n_read * rb + K // 32 * BPL[bits] + 6 + 2 * (G - 1) <= N * rb
    # k_repack_pf: items = 4 ceil(N / 128) G 64; block-group bg = idx / 64, lane l; writes dst[p * 64] for p < NP
    items = 4 * ((N + 127) // 128) * G * 64
    bg_max = (items - 1) >> 6
    hi = pf_offset + bg_max * NP[bits] * 1024 + 63 * 16 + (NP[bits] - 1) * 1024 + 16
    assert hi == wq_bytes, (hi, wq_bytes)
    # both kernels together write every byte of wq exactly once: the regions abut and have the sizes written above
    assert nchunks * 16 + items // 64 * NP[bits] * 1024 == wq_bytes


def test_linear_sizes_with_streamk():
    """det_linear_sizes reserves the prefill planes (doubling wq) only when DET_PREFILL=streamk selects the kernel that
    reads them; c and m are the same either way."""
    import os
    import subprocess
    import sys
    from det_amd import ffi
    if not os.path.exists(ffi.LIB_PATH):
        pytest.skip('libdet_hip.so not built')
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    code = ('import sys; sys.path.insert(0, %r); from det_amd import ffi; '
            'print(*ffi.linear_sizes(9728, 2560, 6))' % root)
    got = {}
    for mode in ('', 'streamk'):
        env = dict(os.environ, DET_PREFILL=mode)
        out = subprocess.run([sys.executable, '-c', code], env=env, capture_output=True, text=True, check=True)
        got[mode] = [int(v) for v in out.stdout.split()]
    dec, sk = got[''], got['streamk']
    assert sk[0] == 2 * dec[0] and sk[1:] == dec[1:]
    assert dec[0] == 152 * 20 * 96 * 64                     # 152 tiles of 64 rows (76 pairs), 20 groups, 96 B each
