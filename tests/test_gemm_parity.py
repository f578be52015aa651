"""GEMM parity on the GPU: det_gemm_ex (HIP, through the C ABI) against the CPU oracle, bit for bit.

Mirrors the reference's GEMM conformance suite (crates/det/src/conformance.rs:348-449: every width, odd shapes,
every batch-size path, Write and Accumulate, fused parts) with its own Rng and seed, then adds the edge cases the
suite lacks (zero, denormal and tiny rows, int64->fp32 rounding ties, extreme multipliers, W8 code -128) and the
BASELINE shapes.
"""
import numpy as np
import pytest

import oracle
from det_amd import ffi
from tests.helpers import same_f32, gaussian_weights, baseline_acts, make_group, det_rows_from

pytestmark = pytest.mark.gpu

SHAPES = [(96, 256), (200, 384), (640, 2560), (2560, 1024), (48, 128)]


def run_gemm(lin, xq, sx, mx, M, accumulate_into=None):
    xb, sb = ffi.Buf.upload(xq), ffi.Buf.upload(sx)
    mb = None if mx is None else ffi.Buf.upload(mx)
    if accumulate_into is not None:
        y = ffi.Buf.upload(accumulate_into)
        ffi.gemm(lin, xb, sb, mb, M, accumulate=y)
    else:
        y = ffi.Buf((M, lin.N), np.float32)
        ffi.gemm(lin, xb, sb, mb, M, write=y)
    return y.download()


def test_conformance_gemm():
    """conformance.rs:348-385: W8/W6/W4 x 5 shapes x M in {1,3,8,9,16,17,32,45,64[,65,100,300]}."""
    rng = oracle.Rng(11)
    fails = []
    for bits in (8, 6, 4):
        for n, k in SHAPES:
            rows = rng.fake_rows(bits, n, k)
            lin = ffi.Linear(rows, k, bits)
            ms = [1, 3, 8, 9, 16, 17, 32, 45, 64] + ([65, 100, 300] if (n, k) == (640, 2560) else [])
            for m in ms:
                print(f'gemm W{bits} n={n} k={k} m={m}', flush=True)
                x = rng.acts_x(m, k)
                xq, sx, mx = oracle.quant(x)
                yc = oracle.gemm(rows, n, k, bits, xq, sx, mx)
                d = same_f32(yc, run_gemm(lin, xq, sx, mx, m))
                if d:
                    fails.append(f'gemm W{bits} n={n} k={k} m={m}: {d}')
                acc = rng.units(m * n).reshape(m, n)
                ac = oracle.gemm(rows, n, k, bits, xq, sx, mx, y=acc, accumulate=True)
                d = same_f32(ac, run_gemm(lin, xq, sx, mx, m, accumulate_into=acc))
                if d:
                    fails.append(f'gemm accumulate W{bits} n={n} k={k} m={m}: {d}')
    assert not fails, '\n'.join(fails)


def test_conformance_fused_parts():
    """conformance.rs:387-448: two W6 tensors (100 + 60 rows, K=512) fused along N, routed into two parts."""
    rng = oracle.Rng(11)
    # advance the Rng exactly as the reference suite does before its fused-parts block
    for bits in (8, 6, 4):
        for n, k in SHAPES:
            rng.fake_rows(bits, n, k)
            ms = [1, 3, 8, 9, 16, 17, 32, 45, 64] + ([65, 100, 300] if (n, k) == (640, 2560) else [])
            for m in ms:
                rng.acts_x(m, k)
                rng.units(m * n)
    k = 512
    r1 = rng.fake_rows(6, 100, k)
    r2 = rng.fake_rows(6, 60, k)
    rows = np.concatenate([r1, r2])
    lin = ffi.Linear(rows, k, 6, widths=[100, 60])
    for m in (1, 7, 20, 90):
        xq, sx, mx = oracle.quant(rng.acts_x(m, k))
        ac, bc = oracle.gemm(rows, 160, k, 6, xq, sx, mx, widths=[100, 60])
        ag, bg = ffi.Buf((m, 100), np.float32), ffi.Buf((m, 60), np.float32)
        ffi.gemm(lin, ffi.Buf.upload(xq), ffi.Buf.upload(sx), ffi.Buf.upload(mx), m, parts=[ag, bg])
        assert same_f32(ac, ag.download()) is None, f'part a m={m}'
        assert same_f32(bc, bg.download()) is None, f'part b m={m}'


@pytest.mark.parametrize('bits', [8, 6, 4])
def test_four_parts_and_accumulate_edges(bits):
    """Four fused parts of ragged widths (the GemmOut::Parts maximum), across tile boundaries."""
    rng = oracle.Rng(101 + bits)
    widths = [1, 63, 130, 70]
    k = 384
    rows = np.concatenate([rng.fake_rows(bits, w, k) for w in widths])
    lin = ffi.Linear(rows, k, bits, widths=widths)
    for m in (1, 5, 9, 40, 130):
        xq, sx, mx = oracle.quant(rng.acts_x(m, k))
        want = oracle.gemm(rows, sum(widths), k, bits, xq, sx, mx, widths=widths)
        outs = [ffi.Buf((m, w), np.float32) for w in widths]
        ffi.gemm(lin, ffi.Buf.upload(xq), ffi.Buf.upload(sx), ffi.Buf.upload(mx), m, parts=outs)
        for i, (w_, o) in enumerate(zip(want, outs)):
            assert same_f32(w_, o.download()) is None, f'part {i} m={m}'


@pytest.mark.parametrize('bits', [8, 6, 4])
def test_edge_rows(bits):
    """Activation rows that are all zero, all denormal, 1e-3 scaled, tiny (sx underflow), mixed; mx == NULL."""
    rng = oracle.Rng(7 + bits)
    n, k = 300, 1024
    rows = rng.fake_rows(bits, n, k)
    lin = ffi.Linear(rows, k, bits)
    for m in (1, 6, 12, 70):
        x = rng.acts_x(m, k)
        x[0] = 0.0
        if m > 1:
            x[1] = np.array([rng.denorm() for _ in range(k)], np.float32)
        if m > 2:
            x[2] *= np.float32(1e-3)
        if m > 3:
            x[3] = np.float32(1e-41)        # every group tiny: smax/65535 underflows to 0, multipliers become 0
            x[3, :128] = 0.0
        if m > 4:
            x[4, ::3] = -0.0
        for group in (True, False):
            xq, sx, mx = oracle.quant(x, group=group)
            want = oracle.gemm(rows, n, k, bits, xq, sx, mx)
            assert same_f32(want, run_gemm(lin, xq, sx, mx, m)) is None, f'm={m} group={group}'


def test_int64_to_fp32_ties():
    """Accumulators built to be exact round-half-even ties (and neighbours) of the int64 -> fp32 conversion,
    with c = sx = 1 so y = f32(acc).  Groups: s = m*mx in {65535^2, 4096*256, 1}."""
    prng = np.random.default_rng(5)
    K, G = 384, 3
    mx = np.array([[65535, 256, 1]], np.uint16)
    xg = [127] * 127 + [1]
    xq = np.array([xg * G], np.int8)
    targets = []
    for _ in range(512):
        e = int(prng.integers(25, 52))
        a = int(prng.integers(1 << 23, 1 << 24))
        base = a << (e - 23)
        half = 1 << (e - 24)
        t = base + half + int(prng.choice([0, 0, 1, -1]))
        targets.append(t * int(prng.choice([1, -1])))
    codes, ms = [], []
    s1, s2 = 65535 * 65535, 4096 * 256
    for t in targets:
        sg = 1 if t >= 0 else -1
        r = abs(t)
        p1 = r // s1
        r -= p1 * s1
        p2 = r // s2
        p3 = r - p2 * s2
        assert max(p1, p2, p3) <= 127 * 127 * 127
        codes.append(np.concatenate([make_group(sg * p, xg, 127) for p in (p1, p2, p3)]))
        ms.append([65535, 4096, 1])
    codes = np.array(codes, np.int8)
    N = len(targets)
    rows = det_rows_from(codes, np.ones(N, np.float32), np.array(ms), 8)
    sx = np.ones(1, np.float32)
    want = oracle.gemm(rows, N, K, 8, xq, sx, mx)
    lin = ffi.Linear(rows, K, 8)
    got = run_gemm(lin, xq, sx, mx, 1)
    assert same_f32(want, got) is None
    # the same columns through the matrix-core paths (decode M = 9, tiled M = 20): repeat the token
    for M in (9, 20):
        xqm = np.repeat(xq, M, axis=0)
        mxm = np.repeat(mx, M, axis=0)
        sxm = np.ones(M, np.float32)
        wantm = oracle.gemm(rows, N, K, 8, xqm, sxm, mxm)
        assert same_f32(wantm, run_gemm(lin, xqm, sxm, mxm, M)) is None, f'M={M}'


@pytest.mark.parametrize('bits,code', [(8, 127), (8, -127), (8, -128), (6, 31), (6, -32), (4, 7), (4, -8)])
def test_extreme_accumulators(bits, code):
    """Every code at its extreme, every activation +-127, m = mx = 65535, K = 17408: |acc| near 2^61."""
    K, N = 17408, 72
    G = K // 128
    codes = np.full((N, K), code, np.int8)
    rows = det_rows_from(codes, np.full(N, 1e-30, np.float32), np.full((N, G), 65535), bits)
    lin = ffi.Linear(rows, K, bits)
    for M in (1, 3, 16, 65):
        xq = np.full((M, K), 127, np.int8)
        xq[1::2] = -127
        mx = np.full((M, G), 65535, np.uint16)
        sx = np.full(M, 3e-7, np.float32)
        want = oracle.gemm(rows, N, K, bits, xq, sx, mx)
        assert same_f32(want, run_gemm(lin, xq, sx, mx, M)) is None, f'M={M}'


@pytest.mark.parametrize('M', [1, 64, 512])
def test_baseline_w6_9728x2560(M):
    """W6, K=2560, N=9728, quantized Gaussian weights, activations per spec."""
    K, N = 2560, 9728
    w = gaussian_weights(1, N, K)
    rows = oracle.quantize_rows(w, 6)
    lin = ffi.Linear(rows, K, 6)
    x = baseline_acts(2 + M, M, K, zero_row=M // 2 if M > 1 else None)
    xq, sx, mx = oracle.quant(x)
    want = oracle.gemm(rows, N, K, 6, xq, sx, mx)
    assert same_f32(want, run_gemm(lin, xq, sx, mx, M)) is None


@pytest.mark.parametrize('bits', [8, 6, 4])
def test_decode_every_m(bits):
    """Every small batch M = 1..65 (each decode variant: dot-product M = 1, matrix-core M = 2..16, two to four token
    sets M = 17..64, tiled M = 65), on a
    shape whose tiles are few (split over K, int64 atomics across workgroups) and one whose tiles fill the device;
    group and per-row activation scales; repeated calls, so the split's accumulators must come back to zero."""
    rng = oracle.Rng(300 + bits)
    for n, k in ((200, 3072), (9000, 512)):
        rows = rng.fake_rows(bits, n, k)
        lin = ffi.Linear(rows, k, bits)
        for m in range(1, 66):
            x = rng.acts_x(m, k)
            for group in (True, False):
                print(f'decode W{bits} n={n} k={k} m={m} group={group}', flush=True)
                xq, sx, mx = oracle.quant(x, group=group)
                want = oracle.gemm(rows, n, k, bits, xq, sx, mx)
                assert same_f32(want, run_gemm(lin, xq, sx, mx, m)) is None, f'n={n} m={m} group={group}'


@pytest.mark.parametrize('bits', [6, 4])
def test_decode_ms_long_k(bits):
    """Token-set decode (16 < M <= 64) with more groups per wave than one 32-group digit step: n = 9000 rows fill the
    device without a K-split, k = 17920 (140 groups) gives each wave 35 rounds, so the bias correction runs twice."""
    rng = oracle.Rng(500 + bits)
    n, k = 9000, 17920
    rows = rng.fake_rows(bits, n, k)
    lin = ffi.Linear(rows, k, bits)
    for m in (20, 50):
        print(f'decode_ms W{bits} n={n} k={k} m={m}', flush=True)
        xq, sx, mx = oracle.quant(rng.acts_x(m, k))
        want = oracle.gemm(rows, n, k, bits, xq, sx, mx)
        assert same_f32(want, run_gemm(lin, xq, sx, mx, m)) is None, f'm={m}'
