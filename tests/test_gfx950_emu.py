"""The instruction-level emulator (tests/gfx950_emu.py) on hand-written instruction sequences: the pending-load and
pending-copy rules it enforces, and instruction semantics against values worked out by hand from the instruction set
reference.  (Its MFMA, buffer-copy and address models are pinned by a real kernel: the emulated k_prefill2, which has
matched the oracle on an MI355X, matches it under the emulator too -- tests/test_isa_emulation.py.)"""
import numpy as np
import pytest

from tests import gfx950_emu as E


def run(lines, lds=0, mem=None, threads=64):
    mem = mem or E.Memory()
    wg = E.Workgroup(E.Program.from_lines(lines, lds_bytes=lds), mem, 0, threads)
    wg.run()
    return wg.waves[0], wg, mem


def addr_lines(base, vlo=2):
    return [f'v_mov_b32 v{vlo}, {base & 0xFFFFFFFF:#x}', f'v_mov_b32 v{vlo + 1}, {base >> 32:#x}']


def test_read_of_pending_load_fails():
    mem = E.Memory()
    base = mem.alloc(4, np.array([7], np.uint32))
    with pytest.raises(E.EmuError, match='pending'):
        run(addr_lines(base) + ['global_load_dword v4, v[2:3], off', 'v_mov_b32 v5, v4', 's_endpgm'], mem=mem)


def test_waited_load_lands():
    mem = E.Memory()
    base = mem.alloc(4, np.array([7], np.uint32))
    w, _, _ = run(addr_lines(base) + ['global_load_dword v4, v[2:3], off', 'global_load_dword v6, v[2:3], off',
                                      's_waitcnt vmcnt(1)', 'v_mov_b32 v5, v4', 's_waitcnt vmcnt(0)', 's_endpgm'],
                  mem=mem)
    assert (w.v[5] == 7).all() and (w.v[6] == 7).all()


def test_too_weak_wait_fails():
    mem = E.Memory()
    base = mem.alloc(4, np.array([7], np.uint32))
    with pytest.raises(E.EmuError, match='pending'):
        run(addr_lines(base) + ['global_load_dword v4, v[2:3], off', 'global_load_dword v6, v[2:3], off',
                                's_waitcnt vmcnt(2)', 'v_mov_b32 v5, v4', 's_endpgm'], mem=mem)


def rsrc_lines(base, nrec, s=8):
    return [f's_mov_b32 s{s}, {base & 0xFFFFFFFF:#x}', f's_mov_b32 s{s + 1}, {base >> 32:#x}',
            f's_mov_b32 s{s + 2}, {nrec:#x}', f's_mov_b32 s{s + 3}, 0x20000']


def test_lds_copy_pending_until_waited():
    mem = E.Memory()
    base = mem.alloc(256, np.arange(64, dtype=np.uint32) + 100)
    copy = rsrc_lines(base, 256) + ['s_mov_b32 m0, 0', 'v_lshlrev_b32 v1, 2, v0',
                                    'buffer_load_dword v1, s[8:11], 0 offen lds']
    with pytest.raises(E.EmuError, match='copy into it is pending'):
        run(copy + ['ds_read_b32 v2, v1', 's_endpgm'], lds=256, mem=mem)
    w, wg, _ = run(copy + ['s_waitcnt vmcnt(0)', 'ds_read_b32 v2, v1', 's_waitcnt lgkmcnt(0)', 's_endpgm'], lds=256,
                   mem=mem)
    assert (w.v[2] == np.arange(64) + 100).all()


def test_buffer_range_check_excludes_scalar_offset():
    """Per-lane offset + instruction offset is checked against num_records; the scalar offset is not."""
    mem = E.Memory()
    base = mem.alloc(512, np.arange(128, dtype=np.uint32))
    w, _, _ = run(rsrc_lines(base, 16) + ['s_movk_i32 s12, 0x100', 'v_lshlrev_b32 v1, 2, v0',
                                         'buffer_load_dword v2, v1, s[8:11], s12 offen', 's_waitcnt vmcnt(0)',
                                         's_endpgm'], mem=mem)
    assert list(w.v[2][:5]) == [64, 65, 66, 67, 0]         # lanes 0-3 in range (offsets 0-12), read at +256


def test_semantics_by_hand():
    w, _, _ = run([
        'v_mov_b32 v1, 0x11223344', 'v_mov_b32 v2, 0x55667788', 'v_mov_b32 v3, 0xc0c0500',
        'v_perm_b32 v4, v1, v2, v3',                                   # bytes 0, 5, zero, zero of {v1:v2}
        'v_bitop3_b32 v5, v1, v2, v3 bitop3:0x80',                    # v1 & v2 & v3
        'v_bitop3_b32 v6, v1, v2, v3 bitop3:0xfe',                    # v1 | v2 | v3
        'v_and_b32_sdwa v7, v1, v2 dst_sel:BYTE_3 dst_unused:UNUSED_PAD src0_sel:DWORD src1_sel:DWORD',
        'v_mov_b32 v8, -1', 'v_mov_b32 v9, -1', 'v_mov_b32 v10, -1', 'v_mov_b32 v11, -1',
        'v_mad_u64_u32 v[12:13], s[20:21], v8, v9, v[10:11]',         # (2^32-1)^2 + 2^64-1 carries out
        'v_mov_b32 v14, 0x3f800000', 'v_mov_b32 v15, 0x40400000',
        'v_fmac_f32_e32 v14, 0.5, v15',                                # 1 + 0.5 * 3, one register written
        'v_mov_b32 v16, 0', 'v_mov_b32 v17, 0x3ff00000', 'v_mov_b32 v18, 0', 'v_mov_b32 v19, 0x40080000',
        'v_fmac_f64_e32 v[16:17], 0x41f00000, v[18:19]',               # 1 + 2^32 * 3: the literal is the high word
        'v_ffbh_u32 v20, v1', 'v_ffbh_u32 v21, 0',
        'v_mov_b32 v22, 0x80000000', 'v_ffbh_u32 v22, v22',
        's_endpgm'])
    assert w.v[4][0] == 0x00003388
    assert w.v[5][0] == 0x11223344 & 0x55667788 & 0x0C0C0500
    assert w.v[6][0] == 0x11223344 | 0x55667788 | 0x0C0C0500
    assert w.v[7][0] == ((0x11223344 & 0x55667788) & 0xFF) << 24
    r = (2 ** 32 - 1) ** 2 + 2 ** 64 - 1
    assert int(w.v[12][0]) | int(w.v[13][0]) << 32 == r % 2 ** 64 and w.s[20] & 1 == 1
    assert w.v[14].view(np.float32)[0] == 2.5 and w.v[15][0] == 0x40400000
    assert np.array([w.v[16][0], w.v[17][0]], np.uint32).view(np.float64)[0] == 1 + 3 * 2.0 ** 32
    assert w.v[20][0] == 3 and w.v[21][0] == 0xFFFFFFFF and w.v[22][0] == 0


def test_mfma_identity():
    """A = the identity (A[i][k] = 1 for k = i) in the documented operand layout, so D = B + C: checks the A, B and
    C/D layouts against one another."""
    rng = np.random.default_rng(1)
    Bm = rng.integers(-128, 128, (32, 32))              # B[k][j]
    Cm = rng.integers(-1000, 1000, (32, 32))
    mem = E.Memory()
    wg = E.Workgroup(E.Program.from_lines(['v_mfma_i32_32x32x32_i8 v[32:47], v[0:3], v[4:7], v[16:31]',
                                           's_endpgm']), mem, 0, 64)
    w = wg.waves[0]
    A = np.zeros((64, 16), np.int8)
    B = np.zeros((64, 16), np.int8)
    for l in range(64):
        for kk in range(16):
            k = 16 * (l // 32) + kk
            A[l, kk] = 1 if l % 32 == k else 0
            B[l, kk] = Bm[k, l % 32]
    w.v[0:4] = A.view(np.uint32).reshape(64, 4).T
    w.v[4:8] = B.view(np.uint32).reshape(64, 4).T
    C = np.zeros((64, 16), np.int32)
    for i in range(32):
        C[np.arange(32) + 32 * ((i // 4) % 2), 4 * (i // 8) + i % 4] = Cm[i]
    w.v[16:32] = C.view(np.uint32).T
    wg.run()
    D = w.v[32:48].T.view(np.int32)
    for i in range(32):
        assert (D[np.arange(32) + 32 * ((i // 4) % 2), 4 * (i // 8) + i % 4] == Bm[i] + Cm[i]).all()


def test_fma_rounds_once():
    """The emulator's fused multiply-add against exact rational arithmetic: random operands over wide exponent ranges,
    and products that are exactly a binary32 midpoint (p = (2^12 + 1)(2^12 + 3) = 2^24 + 2^14 + 3, odd, between two
    binary32 neighbours 2 apart) with a tiny addend of either sign, where a binary64 sum alone would round to the
    midpoint and then to even."""
    from fractions import Fraction
    rng = np.random.default_rng(7)
    for trial in range(40):
        a = (rng.standard_normal(64) * 2.0 ** rng.integers(-30, 30, 64)).astype(np.float32)
        b = (rng.standard_normal(64) * 2.0 ** rng.integers(-30, 30, 64)).astype(np.float32)
        c = (rng.standard_normal(64) * 2.0 ** rng.integers(-60, 60, 64)).astype(np.float32)
        if trial == 0:
            a[:8], b[:8] = np.float32(4097.0), np.float32(4099.0)
            c[:8] = np.float32(2.0 ** -30) * np.array([1, -1, 1, -1, 3, -3, 0.5, -0.5], np.float32)
        got = E.exact_fma(a, b, c, np.float32)
        want = np.array([E.round_fraction(Fraction(float(x)) * Fraction(float(y)) + Fraction(float(z)), np.float32)
                         for x, y, z in zip(a, b, c)], np.float32)
        assert (got.view(np.uint32) == want.view(np.uint32)).all(), trial
    # 4097 * 4101 = 2^24 + 24581: a midpoint whose even neighbour is the lower one; a tiny positive addend rounds up
    got = E.exact_fma(np.full(64, 4097.0, np.float32), np.full(64, 4101.0, np.float32),
                      np.full(64, 2.0 ** -30, np.float32), np.float32)
    assert got[0] == np.float32(2 ** 24 + 24582)
    got = E.exact_fma(np.full(64, 4097.0, np.float32), np.full(64, 4101.0, np.float32),
                      np.zeros(64, np.float32), np.float32)
    assert got[0] == np.float32(2 ** 24 + 24580)                 # the tie itself goes to even: down


def arrival_order(seed):
    """Eight one-lane workgroups each take a ticket from a shared counter (atomic add returning the old value) after a
    few instructions of other work, and store it at their own slot: the tickets give the arrival order."""
    mem = E.Memory()
    cnt = mem.alloc(4, np.zeros(1, np.uint32))
    out = mem.alloc(32, np.zeros(8, np.uint32))
    lines = addr_lines(cnt) + ['v_mov_b32 v4, 1'] + ['v_add_u32 v9, v9, v4'] * 20 + [
        'global_atomic_add v5, v[2:3], v4, off sc0', 's_waitcnt vmcnt(0)',
        f'v_mov_b32 v7, {out & 0xFFFFFFFF:#x}', f'v_mov_b32 v8, {out >> 32:#x}',
        'v_lshlrev_b32 v6, 2, s2', 'v_add_co_u32 v7, vcc, v7, v6', 'v_addc_co_u32 v8, vcc, v8, 0, vcc',
        'global_store_dword v[7:8], v5, off', 's_waitcnt vmcnt(0)', 's_endpgm']
    prog = E.Program.from_lines(lines)
    wgs = []
    for g in range(8):
        wg = E.Workgroup(prog, mem, g, 1)
        wg.waves[0].s[2] = g
        wgs.append(wg)
    if seed is None:
        for wg in wgs:
            wg.run()
    else:
        E.run_interleaved(wgs, seed)
    return [int(v) for v in mem.array(out, np.uint32, 8)]


def test_interleaved_workgroups_arrive_in_other_orders():
    """Run one after another, workgroup g arrives g-th; interleaved, the arrival orders differ from the grid order and
    from each other, while every workgroup still arrives exactly once (the hand-over tests rely on both)."""
    assert arrival_order(None) == list(range(8))
    orders = {tuple(arrival_order(seed)) for seed in range(6)}
    assert all(sorted(o) == list(range(8)) for o in orders)
    assert len(orders - {tuple(range(8))}) >= 4
