"""Lane-level CPU emulation of the stream-K prefill kernel (det_amd/csrc/prefill.hip k_prefill), TEST INFRASTRUCTURE.

The emulation follows the kernel's data movement step by step: the activation copies into the swizzled LDS stage
(per lane and copy, as the buffer unit lands them), the lane's prefill words and their unpack, the B-operand LDS
offsets, v_mfma_i32_32x32x32_i8 with the operand and result layouts the GPU-verified kernels of gemm.hip rely on
(A/B: lane l holds row/column l % 32 and k bytes 16 (l / 32) .. + 15 of the 32-k step; the result element (i, j) sits
in lane j + 32 ((i / 4) % 2), register 4 (i / 8) + i % 4), the biased int64 scaling, the digit-product bias removal
every 32 groups, the stream-K fragments with their partial tiles, and the epilogue's transpose.  The result must
equal the oracle bit for bit: an index mapping that disagrees with the matrix semantics fails here on the CPU.
"""
import numpy as np
import pytest

import oracle
from tests.test_prefill_logic import pack_lane, fragments, owner, host_P
from tests.test_quantizer_parity import pf_unpack
from tests.helpers import same_f32

GROUP = 128
NP = {8: 4, 6: 3, 4: 2}
SH = {8: 0, 6: 2, 4: 4}
BIAS = 1 << 21
M64 = (1 << 64) - 1


def swz(r, c):
    return r * 128 + ((c ^ ((r >> 1) & 7)) << 4)


def mfma(a_lanes, b_lanes, c_regs):
    """v_mfma_i32_32x32x32_i8: a_lanes, b_lanes [64][16] int8, c_regs [64][16] int64 -> d_regs [64][16]."""
    lane = np.arange(64)
    A = np.zeros((32, 32), np.int64)
    B = np.zeros((32, 32), np.int64)
    for l in range(64):
        A[l % 32, 16 * (l // 32):16 * (l // 32) + 16] = a_lanes[l]
        B[16 * (l // 32):16 * (l // 32) + 16, l % 32] = b_lanes[l]
    D = A @ B
    out = c_regs.astype(np.int64).copy()
    for r in range(16):
        i = 8 * (r // 4) + 4 * (lane // 32) + r % 4
        out[:, r] += D[i, lane % 32]
    # int32 wrap of the hardware accumulator
    return ((out + (1 << 31)) % (1 << 32)) - (1 << 31)


def build_planes(rows, N, K, bits):
    """k_repack_pf restated: prefill words [blk][g][lane][NP * 4] (uint32)."""
    G = K // GROUP
    nb32 = 4 * ((N + 127) // 128)
    nc = K // 32 * {8: 32, 6: 24, 4: 16}[bits]
    codes = np.zeros((nb32 * 32, K), np.int64)
    for n in range(N):
        codes[n] = oracle.unpack_row(rows[n, :nc], bits, K)
    i = np.arange(64)
    words = np.zeros((nb32, G, 64, NP[bits] * 4), np.uint32)
    for b in range(nb32):
        for g in range(G):
            for l in range(64):
                r, h = l % 32, l // 32
                words[b, g, l] = pack_lane(codes[b * 32 + r, g * 128 + 32 * (i // 16) + 16 * h + i % 16], bits)
    return words


def emulate(rows, N, K, bits, xq, sx, mx, cus, P=None):
    M = xq.shape[0]
    G = K // GROUP
    nc = K // 32 * {8: 32, 6: 24, 4: 16}[bits]
    mrow = np.zeros((4 * ((N + 127) // 128) * 32, G), np.int64)     # m per row (zero past N), as the m plane
    crow = np.zeros(mrow.shape[0], np.float32)
    for n in range(N):
        mrow[n] = rows[n, nc + 4:].view('<u2')
        crow[n] = rows[n, nc:nc + 4].view('<f4')[0]
    words = build_planes(rows, N, K, bits)
    nbn, nbt = (N + 127) // 128, (M + 127) // 128
    tiles = nbn * nbt
    total = tiles * G
    P = host_P(total, cus) if P is None else P
    lane = np.arange(64)
    l32, h = lane % 32, lane // 32
    y = np.zeros((M, N), np.float32)
    partial = {}
    count = {}
    frs = fragments(tiles, G, P)
    # fragments finish in the order their workgroups reach them; any order gives the same sums: run them in list
    # order, the last of a tile's fragments finishing it
    for w, tile, ga, gb in frs:
        nb, tb = divmod(tile, nbt)
        t0, n0 = tb * 128, nb * 128
        U = np.zeros((4, 4, 64, 16), np.uint64)          # [wave][t-block][lane][register]
        dig = np.zeros((3, 256, 32), np.int64)           # [digit][entry: rows 0-127, tokens 128-255][slot]
        for i, g in enumerate(range(ga, gb)):
            slot = i % 32
            if slot == 0 and gb - g < 32:
                dig[:] = 0
            # LDS stage: copy ci of wave wv lands tokens 32 wv + 8 ci + lane / 8 at 4096 wv + 1024 ci + 16 lane
            As = np.zeros(128 * 128, np.int64)
            for wv in range(4):
                for ci in range(4):
                    row = t0 + wv * 32 + 8 * ci + (lane >> 3)
                    chunk = (lane & 7) ^ (((ci & 1) << 2) | (lane >> 4))
                    for l in range(64):
                        dst = 4096 * wv + 1024 * ci + 16 * l
                        if row[l] < M:
                            As[dst:dst + 16] = xq[row[l], g * 128 + 16 * chunk[l]:g * 128 + 16 * chunk[l] + 16]
            mv = np.array([mrow[n0 + s, g] for s in range(128)], np.int64)
            xv = np.array([(int(mx[t0 + s, g]) if t0 + s < M else 0) if mx is not None else 1 for s in range(128)],
                          np.int64)
            sv = np.concatenate([mv, xv])                    # sv_s[par]: thread tid stages entry tid
            for e in range(256):
                for d in range(3):
                    dig[d, e, slot] = (sv[e] >> (7 * d)) & 127 if d < 2 else sv[e] >> 14
            boff = [np.array([swz(int(l32[l]), 2 * s + int(h[l])) for l in range(64)]) for s in range(4)]
            for wv in range(4):
                a = np.stack([pf_unpack(words[nb * 4 + wv, g, l], bits) for l in range(64)])   # [64][64] k order
                xm = [sv[128 + 32 * j + l32] for j in range(4)]
                for p in range(2):
                    d0 = np.full((64, 16), BIAS, np.int64)
                    d1 = np.full((64, 16), BIAS, np.int64)
                    for s in range(4):
                        b0 = np.stack([As[boff[s][l] + 64 * p * 128:boff[s][l] + 64 * p * 128 + 16] for l in range(64)])
                        b1 = np.stack([As[boff[s][l] + (64 * p + 32) * 128:boff[s][l] + (64 * p + 32) * 128 + 16]
                                       for l in range(64)])
                        d0 = mfma(a[:, 16 * s:16 * s + 16], b0, d0)
                        d1 = mfma(a[:, 16 * s:16 * s + 16], b1, d1)
                    for q4 in range(4):
                        for e in range(4):
                            r = 4 * q4 + e
                            mvv = sv[wv * 32 + 8 * q4 + 4 * h + e]
                            for jj, dd in ((2 * p, d0), (2 * p + 1, d1)):
                                assert (dd[:, r] >= 0).all(), 'biased partial negative'
                                prod = (dd[:, r].astype(np.uint64) * (mvv * xm[jj]).astype(np.uint64))
                                U[wv, jj, :, r] = U[wv, jj, :, r] + prod
            if slot == 31 or g + 1 == gb:
                for wv in range(4):
                    Ad = [np.stack([dig[d, wv * 32 + l32[l], 16 * h[l]:16 * h[l] + 16] for l in range(64)])
                          for d in range(3)]
                    for j in range(4):
                        Bd = [np.stack([dig[d, 128 + 32 * j + l32[l], 16 * h[l]:16 * h[l] + 16] for l in range(64)])
                              for d in range(3)]
                        z = np.zeros((64, 16), np.int64)
                        S = np.zeros((64, 16), object)
                        for da in range(3):
                            for db in range(3):
                                S = S + mfma(Ad[da], Bd[db], z).astype(object) * (1 << (7 * (da + db)))
                        for r in range(16):
                            for l in range(64):
                                U[wv, j, l, r] = np.uint64((int(U[wv, j, l, r]) - (int(S[l, r]) << 21)) & M64)
        whole = ga == 0 and gb == G
        if not whole:
            partial[(tile, w)] = U.copy()
            count[tile] = count.get(tile, 0) + 1
            wf, wl = owner(tile * G, total, P), owner(tile * G + G - 1, total, P)
            if count[tile] < wl - wf + 1:
                continue
            U = np.zeros_like(U)
            for v in range(wf, wl + 1):
                U = U + partial[(tile, v)]
        for wv in range(4):
            for j in range(4):
                for l in range(64):
                    t = t0 + 32 * j + l32[l]
                    for r in range(16):
                        n = n0 + wv * 32 + 8 * (r // 4) + 4 * h[l] + r % 4
                        if t < M and n < N:
                            acc = int(U[wv, j, l, r].astype(np.int64)) >> SH[bits]
                            y[t, n] = (np.float32(acc) * crow[n]) * sx[t]
    return y


@pytest.mark.parametrize('bits', [8, 6, 4])
def test_prefill_emulation_matches_oracle(bits):
    rng = oracle.Rng(77 + bits)
    N, K, M = 200, 1280, 130                     # partial row tile, partial token tile
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(M, K))
    want = oracle.gemm(rows, N, K, bits, xq, sx, mx)
    got = emulate(rows, N, K, bits, xq, sx, mx, cus=3)   # P = 6 over 40 units: tiles split across workgroups
    d = same_f32(want, got)
    assert d is None, d


def test_prefill_emulation_full_batch():
    """40 groups in one fragment: a full 32-group bias batch, then a short one (slots cleared)."""
    rng = oracle.Rng(5)
    N, K, M, bits = 40, 5120, 70, 6
    rows = rng.fake_rows(bits, N, K)
    xq, sx, mx = oracle.quant(rng.acts_x(M, K))
    want = oracle.gemm(rows, N, K, bits, xq, sx, mx)
    d = same_f32(want, emulate(rows, N, K, bits, xq, sx, mx, cus=0, P=1))
    assert d is None, d
    # and without mx (all ones)
    want = oracle.gemm(rows, N, K, bits, xq, sx, None)
    d = same_f32(want, emulate(rows, N, K, bits, xq, sx, None, cus=0, P=3))
    assert d is None, d
