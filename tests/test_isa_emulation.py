"""The compiled GEMM kernels, run instruction by instruction on the CPU (tests/gfx950_emu.py) and compared bit for bit
with the oracle.

This covers what the lane-level restatement (tests/test_prefill_emulation.py) cannot: the code hipcc actually
generated for gfx950 -- register allocation, the inline-assembly loads and their waits, the buffer-unit copies into
LDS, scalar address arithmetic, spills -- for the load-time repack (k_repack, k_repack_pf) and both prefill kernels.
The emulator keeps every vector-memory load and LDS copy pending until the wave's `s_waitcnt` retires it and fails on
any earlier use, so a missing wait fails here instead of giving wrong results on a GPU.  k_prefill2, which has run
on MI355X and matched the oracle there, is run too: it checks the emulator against the hardware's behaviour.

The host launch logic is restated from det_amd/csrc (launch_prefill, launch_prefill2, det_linear_repack): grid
sizes, K-slices, the persistent grid and the partial-tile buffers, with `cus` chosen small so that the stream-K
kernel splits tiles between workgroups.
"""
import os

import numpy as np
import pytest

import oracle
from tests import gfx950_emu as E
from tests import isa_waits
from tests.helpers import TIE_GROUPS, same_f32, tie_group
from tests.test_prefill_emulation import build_planes

GROUP = 128
BPL = {8: 32, 6: 24, 4: 16}
NP = {8: 4, 6: 3, 4: 2}
HIPCC = os.path.join(os.environ.get('ROCM_PATH', '/opt/rocm'), 'bin', 'hipcc')
pytestmark = pytest.mark.skipif(not os.path.exists(HIPCC), reason='hipcc not available')


@pytest.fixture(scope='module')
def asm():
    return {src: isa_waits.asm_of(os.path.join(isa_waits.CSRC, src)) for src in ('gemm.hip', 'prefill.hip')}


def sizes(N, K, bits):
    T, G = 2 * ((N + 127) // 128), K // GROUP
    gb = 4 * BPL[bits]
    return T, G, 2 * T * G * gb * 64, T * 64 * 4, T * G * 64 * 2


def out_struct(y, nparts=1, offs=(0, 0, 0, 0, 0), dsts=(0, 0, 0, 0), acc=0):
    b = y.to_bytes(8, 'little') + acc.to_bytes(4, 'little') + nparts.to_bytes(4, 'little')
    b += b''.join(int(o).to_bytes(4, 'little', signed=True) for o in offs) + bytes(4)
    b += b''.join(int(d).to_bytes(8, 'little') for d in dsts)
    assert len(b) == 72
    return b


def repack(asm, mem, rows, N, K, bits):
    """det_linear_repack: k_repack over the decode tiles, then k_repack_pf over the prefill planes."""
    T, G, wq_bytes, c_bytes, m_bytes = sizes(N, K, bits)
    rows_d = mem.alloc(rows.nbytes, rows)
    wq, c, m = mem.alloc(wq_bytes), mem.alloc(c_bytes), mem.alloc(m_bytes)
    pf_off = wq_bytes // 2
    nchunks = pf_off // 16
    p = E.Program(asm['gemm.hip'], 'k_repackEPKhiiiPhPfPtm')
    E.launch(p, mem, min((nchunks + 255) // 256, 65536), 256, p.pack_args([rows_d, N, K, bits, wq, c, m, nchunks]))
    items = 4 * ((N + 127) // 128) * G * 64
    p = E.Program(asm['prefill.hip'], 'k_repack_pf')
    E.launch(p, mem, min((items + 255) // 256, 65536), 256, p.pack_args([rows_d, N, K, bits, wq + pf_off, items]))
    return wq, c, m


def check_layout(mem, wq, c, m, rows, N, K, bits):
    T, G, wq_bytes, c_bytes, m_bytes = sizes(N, K, bits)
    nc = K // 32 * BPL[bits]
    gb = 4 * BPL[bits]
    w = mem.array(wq, np.uint8, wq_bytes)
    dec = w[:wq_bytes // 2].reshape(T, G, gb // 16, 64, 16)
    for n in range(T * 64):
        t, r = divmod(n, 64)
        want = rows[n, :nc] if n < N else np.zeros(nc, np.uint8)
        assert (dec[t, :, :, r, :].reshape(-1) == want).all(), f'decode tile row {n}'
    cv = mem.array(c, np.uint32, T * 64)
    mv = mem.array(m, np.uint16, T * G * 64).reshape(T, G, 64)
    for n in range(N):
        assert cv[n] == rows[n, nc:nc + 4].view(np.uint32)[0]
        assert (mv[n // 64, :, n % 64] == rows[n, nc + 4:].view('<u2')).all()
    words = build_planes(rows, N, K, bits)                 # [blk][g][lane][NP * 4]
    pf = w[wq_bytes // 2:].view(np.uint32).reshape(-1, G, NP[bits], 64, 4)
    want = words.reshape(words.shape[0], G, 64, NP[bits], 4).transpose(0, 1, 3, 2, 4)
    assert (pf[:want.shape[0]] == want).all(), 'prefill planes'


def acts(mem, xq, sx, mx):
    return mem.alloc(xq.nbytes, xq), mem.alloc(sx.nbytes, sx), (mem.alloc(mx.nbytes, mx) if mx is not None else 0)


def run_prefill2(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus):
    wq, c, m = lin
    nbn, nbt = (N + 63) // 64, (M + 127) // 128
    G, tiles = K // GROUP, nbn * nbt
    KS = 1
    if 2 * tiles < 3 * cus:
        KS = max(1, min((3 * cus + 2 * tiles - 1) // (2 * tiles), G // 16))
    gs = (G + KS - 1) // KS
    KS = (G + gs - 1) // gs
    part = mem.alloc(KS * nbt * 128 * nbn * 64 * 8) if KS > 1 else 0
    cnt = mem.alloc(max(tiles, 1) * 4) if KS > 1 else 0
    y = mem.alloc(M * N * 4)
    x_d, sx_d, mx_d = acts(mem, xq, sx, mx)
    p = E.Program(asm['prefill.hip'], f'k_prefill2ILi{bits}E')
    E.launch(p, mem, tiles * KS, 256,
             p.pack_args([wq, c, m, N, K, x_d, sx_d, mx_d, M, out_struct(y), nbn, nbt, KS, part, cnt]))
    return mem.array(y, np.float32, M * N).reshape(M, N).copy(), KS


def run_prefill(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus):
    wq, c, m = lin
    G = K // GROUP
    nbn, nbt = (N + 127) // 128, (M + 127) // 128
    tiles = nbn * nbt
    total = tiles * G
    P = min(2 * cus, max(1, total // 4))
    if P > 8:
        P &= ~7
    split = total % P != 0 or (total // P) % G != 0
    part = mem.alloc(2 * P * 128 * 128 * 8 if split else 8)
    cnt = mem.alloc(max(tiles, 1 << 12) * 4)
    y = mem.alloc(M * N * 4)
    x_d, sx_d, mx_d = acts(mem, xq, sx, mx)
    pf = wq + sizes(N, K, bits)[2] // 2
    p = E.Program(asm['prefill.hip'], f'k_prefillILi{bits}E')
    E.launch(p, mem, P, 256, p.pack_args([pf, c, m, N, K, x_d, sx_d, mx_d, M, out_struct(y), nbt, tiles, P, part, cnt]))
    left = mem.array(cnt, np.uint32, tiles)
    assert (left == 0).all(), 'tile counters not reset'
    return mem.array(y, np.float32, M * N).reshape(M, N).copy(), P, split


@pytest.mark.parametrize('bits', [6, 4, 8])
def test_repack_kernels(asm, bits):
    rng = oracle.Rng(3 + bits)
    N, K = 200, 384
    rows = rng.fake_rows(bits, N, K)
    mem = E.Memory()
    lin = repack(asm, mem, rows, N, K, bits)
    check_layout(mem, *lin, rows, N, K, bits)


@pytest.mark.parametrize('bits', [6])
def test_prefill2_matches_oracle(asm, bits):
    """The GPU-verified kernel under the emulator: the emulator's model against known-good code."""
    rng = oracle.Rng(11)
    N, K, M = 72, 384, 70
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(M, K))
    mem = E.Memory()
    lin = repack(asm, mem, rows, N, K, bits)
    got, KS = run_prefill2(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus=1)
    d = same_f32(oracle.gemm(rows, N, K, bits, xq, sx, mx), got)
    assert d is None, d


@pytest.mark.parametrize('bits', [6, 4, 8])
def test_prefill_matches_oracle(asm, bits):
    """k_prefill with tiles split between workgroups (partial tiles, last-arriver combine) and partial token and row
    tiles."""
    rng = oracle.Rng(21 + bits)
    N, K, M = 136, 640, 200                      # 2 x 2 tiles of 5 groups over 5 workgroups of 4 groups each
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(M, K))
    mem = E.Memory()
    lin = repack(asm, mem, rows, N, K, bits)
    got, P, split = run_prefill(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus=3)
    assert split and P == 5
    d = same_f32(oracle.gemm(rows, N, K, bits, xq, sx, mx), got)
    assert d is None, d


@pytest.mark.parametrize('bits,with_mx', [(6, True), (6, False), (8, True), (4, False)])
def test_prefill_bias_batches(asm, bits, with_mx):
    """33 groups split over 2 workgroups: one fragment crosses a full 32-group bias batch, the other ends in a short
    batch; without mx the token multipliers are all 1 (no mx loads)."""
    rng = oracle.Rng(40 + bits)
    N, K, M = 40, 128 * 33, 70
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(M, K))
    mx = mx if with_mx else None
    mem = E.Memory()
    lin = repack(asm, mem, rows, N, K, bits)
    got, P, split = run_prefill(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus=1)
    assert split and P == 2
    d = same_f32(oracle.gemm(rows, N, K, bits, xq, sx, mx), got)
    assert d is None, d


def test_prefill_xcd_remap(asm):
    """A 16-workgroup persistent grid (a multiple of 8: logical ids remapped so that consecutive ones share an
    XCD) over 4 tiles of 20 groups."""
    rng = oracle.Rng(9)
    bits, N, K, M = 6, 256, 2560, 200
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(M, K))
    mem = E.Memory()
    lin = repack(asm, mem, rows, N, K, bits)
    got, P, split = run_prefill(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus=8)
    assert P == 16 and split                     # 5 units each: every tile split between 4 workgroups
    d = same_f32(oracle.gemm(rows, N, K, bits, xq, sx, mx), got)
    assert d is None, d


def run_prefill_out(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus, out):
    """run_prefill with a caller-built output (Parts / Accumulate)."""
    wq, c, m = lin
    G = K // GROUP
    nbn, nbt = (N + 127) // 128, (M + 127) // 128
    tiles = nbn * nbt
    total = tiles * G
    P = min(2 * cus, max(1, total // 4))
    if P > 8:
        P &= ~7
    part = mem.alloc(2 * P * 128 * 128 * 8)
    cnt = mem.alloc(max(tiles, 1 << 12) * 4)
    x_d, sx_d, mx_d = acts(mem, xq, sx, mx)
    pf = wq + sizes(N, K, bits)[2] // 2
    p = E.Program(asm['prefill.hip'], f'k_prefillILi{bits}E')
    E.launch(p, mem, P, 256, p.pack_args([pf, c, m, N, K, x_d, sx_d, mx_d, M, out, nbt, tiles, P, part, cnt]))


def test_prefill_parts_and_accumulate(asm):
    """Three ragged parts (widths 37, 64, 35: unaligned boundaries take the per-column stores), then the same GEMM
    accumulated onto a prefilled output."""
    rng = oracle.Rng(12)
    bits, N, K, M = 6, 136, 640, 130
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(M, K))
    want = oracle.gemm(rows, N, K, bits, xq, sx, mx)
    mem = E.Memory()
    lin = repack(asm, mem, rows, N, K, bits)
    widths = (37, 64, 35)
    offs = (0, 37, 101, 136, 0)
    dsts = [mem.alloc(M * w_ * 4) for w_ in widths]
    run_prefill_out(asm, mem, lin, N, K, bits, xq, sx, mx, M, 3,
                    out_struct(0, nparts=3, offs=offs, dsts=dsts + [0]))
    for i, w_ in enumerate(widths):
        got = mem.array(dsts[i], np.float32, M * w_).reshape(M, w_)
        d = same_f32(want[:, offs[i]:offs[i] + w_], got)
        assert d is None, (i, d)
    base = np.random.default_rng(3).standard_normal((M, N)).astype(np.float32)
    y = mem.alloc(M * N * 4, base)
    run_prefill_out(asm, mem, lin, N, K, bits, xq, sx, mx, M, 3, out_struct(y, acc=1))
    d = same_f32((base + want).astype(np.float32), mem.array(y, np.float32, M * N).reshape(M, N))
    assert d is None, d


@pytest.mark.parametrize('bits,cus', [(8, 1), (4, 1), (6, 8)])
def test_prefill2_widths_and_k_slices(asm, bits, cus):
    """k_prefill2 at W8 and W4, and at W6 with K-slices (one tile, 32 groups, cus = 8: two slices combined by the
    last to arrive)."""
    rng = oracle.Rng(30 + bits)
    N, K, M = (72, 384, 70) if cus == 1 else (64, 4096, 70)
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(M, K))
    mem = E.Memory()
    lin = repack(asm, mem, rows, N, K, bits)
    got, KS = run_prefill2(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus=cus)
    assert KS == (1 if cus == 1 else 2)
    d = same_f32(oracle.gemm(rows, N, K, bits, xq, sx, mx), got)
    assert d is None, d


# ------------------------------------------------------------------ decode kernels (launch_decode, launch_decode_ms)
def run_decode(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus):
    wq, c, m = lin
    MP = 1 if M <= 1 else 4 if M <= 4 else 8 if M <= 8 else 16
    G, T = K // GROUP, (N + 63) // 64
    waves = 8 * cus
    KS = 1
    if 2 * T < cus:
        KS = max(1, min((cus + T - 1) // T, (G + 3) // 4))
    gs = (G + KS - 1) // KS
    S = (waves + T * KS - 1) // (T * KS)
    S = max(1, min(S, min(gs, min(8 if MP >= 4 else 16, 128 // MP))))
    part = mem.alloc(MP * T * 64 * 8) if KS > 1 else 0
    cnt = mem.alloc(T * 4) if KS > 1 else 0
    y = mem.alloc(M * N * 4)
    x_d, sx_d, mx_d = acts(mem, xq, sx, mx)
    p = E.Program(asm['gemm.hip'], f'k_decodeILi{bits}ELi{MP}ELb0E')
    E.launch(p, mem, T * KS, 64 * S,
             p.pack_args([wq, c, m, N, K, x_d, sx_d, mx_d, M, out_struct(y), KS, part, cnt]),
             dyn_lds=S * MP * 64 * 8 if S > 1 else 0)
    if KS > 1:
        assert (mem.array(part, np.int64, MP * T * 64) == 0).all() and (mem.array(cnt, np.uint32, T) == 0).all(), \
            'K-split buffers not left at zero'
    return mem.array(y, np.float32, M * N).reshape(M, N).copy(), MP, KS, S


def dms_slices(units, G, cus):
    KS = 1 if units >= cus else max(1, min((cus + units - 1) // units, G // 16))
    KS = max(KS, (G + 95) // 96)
    gs = (G + KS - 1) // KS
    return (G + gs - 1) // gs


def run_decode_ms(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus):
    wq, c, m = lin
    G, T = K // GROUP, (N + 63) // 64
    split = M > 32 and 2 * T * dms_slices(2 * T, G, cus) > T * dms_slices(T, G, cus)
    TS = 1 if (M <= 32 or split) else 2
    MT = 32 * TS
    NB = (M + MT - 1) // MT
    units = T * NB
    KS = dms_slices(units, G, cus)
    gs = (G + KS - 1) // KS
    P = min(4 if units * KS <= cus else 2, gs)
    part = mem.alloc(NB * KS * MT * T * 64 * 8) if KS > 1 else 0
    cnt = mem.alloc(max(units, 1 << 14) * 4) if KS > 1 else 0
    NS = (gs + 31) & ~31
    lds = max(2 * P * MT * 128, MT * 64 * 8) + 3 * (64 + MT) * NS
    y = mem.alloc(M * N * 4)
    x_d, sx_d, mx_d = acts(mem, xq, sx, mx)
    p = E.Program(asm['gemm.hip'], f'k_decode_msILi{bits}ELi{TS}E')
    E.launch(p, mem, (T * KS, NB), 128 * P,
             p.pack_args([wq, c, m, N, K, x_d, sx_d, mx_d, M, out_struct(y), KS, part, cnt]), dyn_lds=lds)
    return mem.array(y, np.float32, M * N).reshape(M, N).copy(), TS, KS, P


@pytest.mark.parametrize('bits,M,cus', [(6, 1, 4), (6, 1, 16), (8, 4, 4), (4, 8, 16), (6, 16, 4)])
def test_decode_matches_oracle(asm, bits, M, cus):
    """k_decode (M <= 16) through every token count form, with and without the K-split (cus = 16: the tiles fill
    less than half the CUs, so K-slices meet through int64 atomics and the last to arrive finishes)."""
    rng = oracle.Rng(50 + bits + M)
    N, K = 72, 1024
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(M, K))
    mem = E.Memory()
    lin = repack(asm, mem, rows, N, K, bits)
    got, MP, KS, S = run_decode(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus)
    assert (KS > 1) == (cus == 16)
    d = same_f32(oracle.gemm(rows, N, K, bits, xq, sx, mx), got)
    assert d is None, (MP, KS, S, d)


@pytest.mark.parametrize('bits,M,cus', [(6, 40, 4), (6, 64, 16), (8, 20, 4)])
def test_decode_ms_matches_oracle(asm, bits, M, cus):
    rng = oracle.Rng(60 + bits + M)
    N, K = 72, 2048
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(M, K))
    mem = E.Memory()
    lin = repack(asm, mem, rows, N, K, bits)
    got, TS, KS, P = run_decode_ms(asm, mem, lin, N, K, bits, xq, sx, mx, M, cus)
    d = same_f32(oracle.gemm(rows, N, K, bits, xq, sx, mx), got)
    assert d is None, (TS, KS, P, d)


# ------------------------------------------------------------------ cross-workgroup hand-overs, interleaved
# The kernels above that split work between workgroups (k_prefill's split tiles, k_prefill2's K-slices, k_decode's
# K-split atomics, k_decode_ms's K-slice planes) hand partial sums to whichever workgroup arrives last.  Run one after
# another, the last in grid order always finishes; here every workgroup is resident at once and they run in seeded
# random turns (gfx950_emu.run_interleaved), so other workgroups finish, partials are read while their neighbours are
# still mid-flight and the counters see every arrival order.
@pytest.fixture
def interleaved(request):
    old = E.INTERLEAVE
    E.INTERLEAVE = request.param
    yield request.param
    E.INTERLEAVE = old


@pytest.mark.parametrize('case,interleaved', [('prefill_split', 7), ('prefill_split', 8), ('prefill_xcd', 7),
                                              ('prefill2_ks', 8), ('decode_ks', 7), ('decode_ms_ks', 8)],
                         indirect=['interleaved'])
def test_hand_overs_interleaved(asm, interleaved, case):
    if case == 'prefill_split':
        test_prefill_matches_oracle(asm, 6)
    elif case == 'prefill_xcd':
        test_prefill_xcd_remap(asm)
    elif case == 'prefill2_ks':
        test_prefill2_widths_and_k_slices(asm, 6, 8)
    elif case == 'decode_ks':
        test_decode_matches_oracle(asm, 6, 1, 16)
    else:                                      # 64 tokens, 32 groups at 16 CUs: two K-slice planes per tile
        rng = oracle.Rng(77)
        bits, N, K, M = 6, 72, 4096, 64
        rows = rng.fake_rows(bits, N, K)
        xq, sx, mx = oracle.quant(rng.acts_x(M, K))
        mem = E.Memory()
        lin = repack(asm, mem, rows, N, K, bits)
        got, TS, KS, P = run_decode_ms(asm, mem, lin, N, K, bits, xq, sx, mx, M, 16)
        assert KS == 2
        d = same_f32(oracle.gemm(rows, N, K, bits, xq, sx, mx), got)
        assert d is None, (TS, KS, P, d)


# ------------------------------------------------------------------ activation quantization and the FFN decode path
def run_qrow(asm, mem, mode, a, b=None, eps=0.0, w_y=False):
    """launch_qrow: k_qrow<MODE, EPT> over M rows of n (group mode, 16-byte aligned buffers)."""
    M, n = a.shape
    ept = 8 if n <= 8192 else 16 if n <= 16384 else 32
    threads = ((n // ept + 63) // 64) * 64
    a_d = mem.alloc(a.nbytes, a)
    b_d = mem.alloc(b.nbytes, b) if b is not None else 0
    y = mem.alloc(M * n * 4) if w_y else 0
    xq, sx, mx = mem.alloc(M * n), mem.alloc(M * 4), mem.alloc(M * (n // 128) * 2)
    p = E.Program(asm['quant.hip'], f'k_qrowILi{mode}ELi{ept}E')
    E.launch(p, mem, M, threads, p.pack_args([a_d, b_d, np.float32(eps).view(np.uint32), n, y, xq, sx, mx]))
    out = (mem.array(xq, np.int8, M * n).reshape(M, n).copy(), mem.array(sx, np.float32, M).copy(),
           mem.array(mx, np.uint16, M * (n // 128)).reshape(M, n // 128).copy())
    return out, (mem.array(y, np.float32, M * n).reshape(M, n).copy() if w_y else None)


@pytest.fixture(scope='module')
def qasm():
    return {src: isa_waits.asm_of(os.path.join(isa_waits.CSRC, src)) for src in ('quant.hip', 'gemm.hip', 'prefill.hip')}


def rows_for_quant(seed, M, n):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, n)) * rng.choice([1e-3, 1.0, 30.0], (M, 1))).astype(np.float32)
    x[:, ::97] *= 50                                            # outliers in some groups
    return x


@pytest.mark.parametrize('n', [1024, 2560, 9728])
def test_qrow_quant(qasm, n):
    x = rows_for_quant(n, 5, n)
    mem = E.Memory()
    (xq, sx, mx), _ = run_qrow(qasm, mem, 0, x)
    wq_, wsx, wmx = oracle.quant(x)
    assert (xq == wq_).all() and (sx.view(np.uint32) == wsx.view(np.uint32)).all() and (mx == wmx).all()


def test_qrow_rmsnorm_and_silu_mul(qasm):
    n = 2560
    x = rows_for_quant(1, 4, n)
    wgt = (np.random.default_rng(2).standard_normal(n) * 0.1 + 1).astype(np.float32)
    mem = E.Memory()
    (xq, sx, mx), _ = run_qrow(qasm, mem, 1, x, wgt, eps=1e-6, w_y=True)
    wq_, wsx, wmx = oracle.rmsnorm_quant(x, wgt, np.float32(1e-6))
    assert (xq == wq_).all() and (sx.view(np.uint32) == wsx.view(np.uint32)).all() and (mx == wmx).all()
    g, u = rows_for_quant(3, 4, n), rows_for_quant(4, 4, n)
    (xq, sx, mx), _ = run_qrow(qasm, mem, 2, g, u, w_y=True)
    wq_, wsx, wmx = oracle.silu_mul_quant(g, u)
    assert (xq == wq_).all() and (sx.view(np.uint32) == wsx.view(np.uint32)).all() and (mx == wmx).all()


def test_ffn_decode_path(qasm):
    """The model runner's one-token FFN step: the gate|up GEMV with silu on the gate half (k_decode<6, 1, SILU0>,
    output in two parts), then h = silu(g) * u quantized (k_qrow<MUL>) -- equal to det_silu_mul_quant of the
    oracle's GEMV outputs."""
    rng = oracle.Rng(70)
    ff, K, bits = 256, 1024, 6
    N = 2 * ff
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(1, K))
    want = oracle.gemm(rows, N, K, bits, xq, sx, mx)
    wq_, wsx, wmx = oracle.silu_mul_quant(want[:, :ff], want[:, ff:])
    mem = E.Memory()
    wq, c, m = repack(qasm, mem, rows, N, K, bits)
    T, G = (N + 63) // 64, K // GROUP
    cus = 4
    KS = max(1, min((cus + T - 1) // T, (G + 3) // 4)) if 2 * T < cus else 1
    gs = (G + KS - 1) // KS
    S = max(1, min((8 * cus + T * KS - 1) // (T * KS), min(gs, 16)))
    gate, up = mem.alloc(ff * 4), mem.alloc(ff * 4)
    x_d, sx_d, mx_d = acts(mem, xq, sx, mx)
    p = E.Program(qasm['gemm.hip'], f'k_decodeILi{bits}ELi1ELb1E')
    E.launch(p, mem, T * KS, 64 * S,
             p.pack_args([wq, c, m, N, K, x_d, sx_d, mx_d, 1, out_struct(0, 2, (0, ff, N, 0, 0), (gate, up, 0, 0)),
                          KS, 0, 0]), dyn_lds=S * 64 * 8 if S > 1 else 0)
    g_ = mem.array(gate, np.float32, ff).reshape(1, ff).copy()
    u_ = mem.array(up, np.float32, ff).reshape(1, ff).copy()
    silu = oracle.lib().ora_silu_f
    want_g = np.array([[silu(float(v)) for v in want[0, :ff]]], np.float32)
    assert (g_.view(np.uint32) == want_g.view(np.uint32)).all()
    assert (u_.view(np.uint32) == want[:, ff:].view(np.uint32)).all()
    (hq, hs, hm), _ = run_qrow(qasm, mem, 3, g_, u_)
    assert (hq == wq_).all() and (hs.view(np.uint32) == wsx.view(np.uint32)).all() and (hm == wmx).all()


# ------------------------------------------------------------------ det convert's weight quantizer
@pytest.mark.parametrize('bits', [4, 6, 8])
def test_quantize_rows(qasm, bits):
    """k_quantize (binary64 scale search, indexed-register code packing) against the oracle's quantize_rows, byte for
    byte, on Gaussian rows with a zero group, a scaled group, a single outlier and (W4, W6) a group whose scale search
    ties."""
    rng = np.random.default_rng(80 + bits)
    N, K = 6, 512
    w = (rng.standard_normal((N, K)) * 0.02).astype(np.float32)
    w[1, 128:256] = 0
    w[2, :128] *= 1e-3
    w[3, 300] = 1.5
    if bits in TIE_GROUPS:
        w[4, 128:256] = tie_group(bits, 2.0 ** -12)     # two candidates of equal least error: the first must win
    mem = E.Memory()
    w_d = mem.alloc(w.nbytes, w)
    rb = K // 32 * BPL[bits] + 4 + 2 * (K // GROUP)
    out = mem.alloc(N * rb)
    p = E.Program(qasm['gemm.hip'], 'k_quantizeEPKfiiPh')
    E.launch(p, mem, N, 64, p.pack_args([w_d, K, bits, out]))
    got = mem.array(out, np.uint8, N * rb).reshape(N, rb)
    assert (got == oracle.quantize_rows(w, bits)).all()


# ------------------------------------------------------------------ token mixers
@pytest.fixture(scope='module')
def masm():
    return {'mixer.hip': isa_waits.asm_of(os.path.join(isa_waits.CSRC, 'mixer.hip'))}


def test_argmax(masm):
    """k_argmax_part + k_argmax_fin: the first of tied maxima, NaN skipped (a NaN first element gives 0), -0 == +0,
    over several 2048-value slices; the row accumulators are left at zero."""
    rng = np.random.default_rng(5)
    V = 5000
    x = rng.standard_normal((5, V)).astype(np.float32)
    x[0, [17, 4000]] = 9.0                                   # tie across slices: the first wins
    x[1, :] = np.nan
    x[1, 3000] = 1.0
    x[2, :] = -0.0
    x[2, 7] = 0.0                                            # all zeros: index 0
    x[3, 0] = np.nan                                         # a NaN first element reads as 0
    x[4, 2047], x[4, 2048] = 5.0, 5.0                        # tie at the slice boundary
    want = [int(oracle.lib().ora_argmax(P_(row), V)) for row in x]
    mem = E.Memory()
    l_d = mem.alloc(x.nbytes, x)
    acc = mem.alloc(256 * 8)
    out = mem.alloc(5 * 4)
    p = E.Program(masm['mixer.hip'], 'k_argmax_part')
    E.launch(p, mem, ((V + 2047) // 2048, 5), 256, p.pack_args([l_d, V, acc]))
    p = E.Program(masm['mixer.hip'], 'k_argmax_fin')
    E.launch(p, mem, 1, 256, p.pack_args([l_d, 5, V, acc, out]))
    assert mem.array(out, np.int32, 5).tolist() == want
    assert (mem.array(acc, np.uint64, 5) == 0).all()


def P_(a):
    import ctypes
    return np.ascontiguousarray(a).ctypes.data_as(ctypes.c_void_p)


def rope_tables(cap, half, theta=10000000.0):
    pos = np.arange(cap, dtype=np.float64)[:, None]
    inv = 1.0 / theta ** (np.arange(half, dtype=np.float64) / max(half, 1))
    return np.cos(pos * inv).astype(np.float32), np.sin(pos * inv).astype(np.float32)


def f32bits(x):
    return int(np.float32(x).view(np.uint32))


def attn_scratch(mem, M, n_h, hd):
    """attn_layout: qq, sq, mxo, den, num, cnt (256-byte aligned) in one zeroed block; the struct passed by value."""
    al = lambda b: (b + 255) & ~255
    r = M * n_h
    sizes = [al(r * hd), al(r * 4), al(r * 4), al(r * 8), al(r * hd * 8), al(r * 4)]
    base = mem.alloc(sum(sizes))
    ptrs, off = [], 0
    for sz in sizes:
        ptrs.append(base + off)
        off += sz
    return b''.join(int(p).to_bytes(8, 'little') for p in ptrs) + int(off).to_bytes(8, 'little')


def emulate_attention(asm, mem, dev, M, pos0, n_h, n_kv, hd, rot, eps, qg_d, k_d, v_d, o_d):
    """det_attention's launches (mixer.hip), for the paths these shapes take."""
    S = attn_scratch(mem, M, n_h, hd)
    nrows, half = M * (n_kv + n_h), rot // 2
    ept = {256: 4, 128: 2, 64: 1}.get(hd, 0)
    assert ept and half % ept == 0
    p = E.Program(asm, f'k_attn_prep_wILi{ept}E')
    E.launch(p, mem, (nrows + 3) // 4, 256, p.pack_args([
        dev['kn'], dev['vi'], dev['kq'], dev['sk'], dev['vq'], k_d, v_d, dev['qn'], qg_d, dev['cos'], dev['sin'], half,
        f32bits(eps), pos0, n_kv, n_h, M * n_kv, nrows, S]))
    nkeys = pos0 + M
    if M <= 4:
        grid = ((nkeys + 31) // 32, M * n_h)
        p = E.Program(asm, 'k_attn_maxILi32E')
        E.launch(p, mem, grid, 256, p.pack_args([dev['kq'], dev['sk'], pos0, n_h, n_kv, hd, S]))
        p = E.Program(asm, 'k_attn_accILi32ELb1E')
        E.launch(p, mem, grid, 256, p.pack_args([dev['kq'], dev['sk'], dev['vq'], pos0, n_h, n_kv, hd, S, dev['vs'],
                                                 qg_d, o_d]))
    else:
        assert hd in (64, 128, 256)
        rep = n_h // n_kv
        grid = (hd // 32, (M + 15) // 16, n_kv * ((rep + 3) // 4))
        p = E.Program(asm, f'k_attn_mmaILi{hd}E')
        E.launch(p, mem, grid, 256, p.pack_args([dev['kq'], dev['sk'], dev['vq'], pos0, M, n_h, n_kv, S, dev['vs'],
                                                 qg_d, o_d]))


def test_attention_prefill_then_decode(masm):
    """Head dim 256 with 64 rotary dims and 4 q heads per kv head, as in the 4B model: a 20-token batch on the matrix
    cores, then two single-token steps over 32-key chunks; outputs and the KV cache rows against the oracle."""
    import ctypes
    n_h, n_kv, hd, rot, cap = 8, 2, 256, 64, 32
    rng = np.random.default_rng(1)
    f32 = np.float32
    q_norm = (1 + 0.2 * rng.standard_normal(hd)).astype(f32)
    k_norm = (1 + 0.2 * rng.standard_normal(hd)).astype(f32)
    v_scale = np.array([1 / 1024, 1 / 256][:n_kv], f32)
    v_inv = (f32(1) / v_scale).astype(f32)
    cos, sin = rope_tables(cap, rot // 2)
    mem = E.Memory()
    dev = {n: mem.alloc(a.nbytes, a) for n, a in (('qn', q_norm), ('kn', k_norm), ('vs', v_scale), ('vi', v_inv),
                                                  ('cos', cos), ('sin', sin))}
    dev['kq'], dev['sk'], dev['vq'] = mem.alloc(cap * n_kv * hd), mem.alloc(cap * n_kv * 4), mem.alloc(cap * n_kv * hd * 2)
    kq, sk, vq = np.zeros((cap, n_kv, hd), np.int8), np.zeros((cap, n_kv), f32), np.zeros((cap, n_kv, hd), np.int16)
    L = oracle.lib()
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    pos = 0
    for M in (20, 1, 1):
        qg = rng.standard_normal((M, n_h, 2 * hd)).astype(f32)
        k = rng.standard_normal((M, n_kv, hd)).astype(f32)
        v = (rng.standard_normal((M, n_kv, hd)) * 0.05).astype(f32)
        qg_d, k_d, v_d = (mem.alloc(a.nbytes, a) for a in (qg, k, v))
        o_d = mem.alloc(M * n_h * hd * 4)
        emulate_attention(masm['mixer.hip'], mem, dev, M, pos, n_h, n_kv, hd, rot, 1e-6, qg_d, k_d, v_d, o_d)
        o = np.zeros((M, n_h, hd), f32)
        L.ora_attention(ptr(q_norm), ptr(k_norm), ptr(v_scale), ptr(v_inv), ptr(kq), ptr(sk), ptr(vq), ptr(qg), ptr(k),
                        ptr(v), ptr(cos), ptr(sin), rot, f32(1e-6), M, pos, n_h, n_kv, hd, ptr(o))
        got = mem.array(o_d, np.float32, M * n_h * hd).reshape(M, n_h, hd)
        assert (got.view(np.uint32) == o.view(np.uint32)).all(), f'o at M={M} pos0={pos}'
        pos += M
        assert (mem.array(dev['kq'], np.int8, cap * n_kv * hd).reshape(cap, n_kv, hd)[:pos] == kq[:pos]).all()
        assert (mem.array(dev['sk'], np.uint32, cap * n_kv).reshape(cap, n_kv)[:pos] == sk[:pos].view(np.uint32)).all()
        assert (mem.array(dev['vq'], np.int16, cap * n_kv * hd).reshape(cap, n_kv, hd)[:pos] == vq[:pos]).all()


def emulate_gdn(asm, mem, dev, M, n_k, n_v, dk, dv, eps, qkv_d, z_d, a_d, b_d, on_d):
    """gdn_run's launches (mixer.hip) without the fused a|b projection."""
    cd = 2 * n_k * dk + n_v * dv
    nfl = M * cd + 2 * M * n_k * dk + 2 * M * n_v + M * n_v * dv + n_v
    scratch = mem.alloc(nfl * 4)
    y = scratch
    qb = y + M * cd * 4
    kb = qb + M * n_k * dk * 4
    bd = kb + M * n_k * dk * 4
    ob = bd + 2 * M * n_v * 4
    cnt = ob + M * n_v * dv * 4 if M == 1 else 0
    p2 = 1
    while p2 < dk:
        p2 <<= 1
    if M == 1:
        p = E.Program(asm, 'k_gdn_in1')
        E.launch(p, mem, n_k, 256, p.pack_args([
            dev['conv'], dev['cs'], qkv_d, dev['A'], dev['dt'], a_d, b_d, f32bits(eps), n_k, n_v, dk, dv, cd, y, qb, kb,
            bd, cnt, bytes(40), 0, 0, 0]), dyn_lds=(2 * dk + p2 + p2 // 2) * 4)
    else:
        p = E.Program(asm, 'k_gdn_convEPKfS1_S1_iPf')
        E.launch(p, mem, (M, (cd + 255) // 256), 256, p.pack_args([dev['conv'], dev['cs'], qkv_d, cd, y]))
        p = E.Program(asm, 'k_gdn_conv_state')
        E.launch(p, mem, (cd + 255) // 256, 256, p.pack_args([dev['cs'], qkv_d, M, cd]))
        rows = M * n_k
        p = E.Program(asm, f'k_gdn_prep_wILi{1 if dk <= 64 else 2}E')
        E.launch(p, mem, (rows + 3) // 4, 256, p.pack_args([y, dev['A'], dev['dt'], a_d, b_d, f32bits(eps), rows, n_k, n_v,
                                                            dk, cd, qb, kb, bd]))
    R = dk if dk < 16 else 16
    CW = 256 // R
    rl = 2 * (2 * 32 * dk + 32 * CW + 2 * 32) * 4
    tmpl = {4: (1, 4), 8: (1, 8), 16: (1, 16), 32: (2, 16), 64: (4, 16), 128: (8, 16)}[dk]
    p = E.Program(asm, f'k_gdn_recILi{tmpl[0]}ELi{tmpl[1]}E')
    E.launch(p, mem, (n_v, (dv + CW - 1) // CW), 256, p.pack_args([
        dev['S'], qb, kb, y, bd, M, n_k, n_v, dv, cd, ob, dev['norm'], z_d, f32bits(eps), on_d, cnt]), dyn_lds=rl)
    if M == 1:
        return
    rows = M * n_v
    ept = 1 if dv <= 64 else 2 if dv <= 128 else 4
    p = E.Program(asm, f'k_gdn_out_wILi{ept}E')
    E.launch(p, mem, (rows + 3) // 4, 256, p.pack_args([ob, dev['norm'], z_d, f32bits(eps), rows, dv, on_d]))


def test_gdn_prefill_decode_prefill(masm):
    """dk = 128 (the 4B model's key dim, the same recurrence template) with 2 k heads over 4 v heads: a 6-token batch,
    one decode token (conv, window update and prep in one launch; the gated norm run by the recurrence's last block),
    then a 3-token batch; outputs, the conv window and the recurrent state against the oracle after each."""
    import ctypes
    n_k, n_v, dk, dv = 2, 4, 128, 32
    rng = np.random.default_rng(4)
    f32 = np.float32
    cd = 2 * n_k * dk + n_v * dv
    conv_w = (rng.standard_normal((cd, 4)) * 0.5).astype(f32)
    A = (np.abs(rng.standard_normal(n_v)) + 0.1).astype(f32)
    dt = (rng.standard_normal(n_v) * 0.5).astype(f32)
    norm = (1 + 0.1 * rng.standard_normal(dv)).astype(f32)
    mem = E.Memory()
    dev = {n: mem.alloc(a.nbytes, a) for n, a in (('conv', conv_w), ('A', A), ('dt', dt), ('norm', norm))}
    dev['cs'], dev['S'] = mem.alloc(3 * cd * 4), mem.alloc(n_v * dk * dv * 4)
    cs, S = np.zeros((3, cd), f32), np.zeros((n_v, dk, dv), f32)
    L = oracle.lib()
    ptr = lambda a: a.ctypes.data_as(ctypes.c_void_p)
    for M in (6, 1, 3):
        qkv = rng.standard_normal((M, cd)).astype(f32)
        z = rng.standard_normal((M, n_v, dv)).astype(f32)
        a = rng.standard_normal((M, n_v)).astype(f32)
        b = rng.standard_normal((M, n_v)).astype(f32)
        qkv_d, z_d, a_d, b_d = (mem.alloc(x.nbytes, x) for x in (qkv, z, a, b))
        on_d = mem.alloc(M * n_v * dv * 4)
        emulate_gdn(masm['mixer.hip'], mem, dev, M, n_k, n_v, dk, dv, 1e-6, qkv_d, z_d, a_d, b_d, on_d)
        on = np.zeros((M, n_v, dv), f32)
        L.ora_gdn(ptr(conv_w), ptr(A), ptr(dt), ptr(norm), ptr(cs), ptr(S), ptr(qkv), ptr(z), ptr(a), ptr(b), f32(1e-6),
                  M, n_k, n_v, dk, dv, ptr(on))
        assert (mem.array(on_d, np.uint32, M * n_v * dv) == on.view(np.uint32).reshape(-1)).all(), f'on at M={M}'
        assert (mem.array(dev['cs'], np.uint32, 3 * cd) == cs.view(np.uint32).reshape(-1)).all(), f'conv at M={M}'
        assert (mem.array(dev['S'], np.uint32, n_v * dk * dv) == S.view(np.uint32).reshape(-1)).all(), f'S at M={M}'
