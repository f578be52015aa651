"""Pins the CPU oracle (oracle/det_oracle.c) to facts that do not come from retyping its formulas:

* the reference's known-answer test for the weight quantizer (crates/det/src/quantize.rs:108-140): pack/unpack
  round trip and the dequantization error bound, on its closed-form input;
* the packing layout of docs/SPEC.md:30-36, checked bit by bit on hand-built codes, plus an exhaustive
  pack -> unpack identity over every code value;
* exact integers: the GEMM accumulator against Python integers, and int64 -> fp32 round-half-even against an
  exact rational rounding routine written here, on crafted ties;
* closed forms and invariants of the activation quantization (zero rows, the max group's multiplier, the
  reconstruction bound, power-of-two scale invariance, the Rust NaN casts when sx underflows);
* the reference suite's xorshift64 generator against a pure-Python one;
* agreement with the independent numpy restatement (oracle/spec_np.py) and with the golden fixtures.
"""
import os
from fractions import Fraction

import numpy as np
import pytest

import oracle
from oracle import spec_np
from tests.helpers import TIE_GROUPS, tie_group

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), 'golden', 'quantized_linear.npz')


def f32_bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def rne_f32(v: int) -> np.float32:
    """Exact round-half-even of an integer to binary32 (independent of any float conversion)."""
    if v == 0:
        return np.float32(0.0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.bit_length() - 1
    if e <= 23:
        return np.float32(sign * a)
    sh = e - 23
    kept, rem = a >> sh, a & ((1 << sh) - 1)
    half = 1 << (sh - 1)
    if rem > half or (rem == half and kept & 1):
        kept += 1
    return np.float32(sign * float(Fraction(kept << sh)))


# ---------------------------------------------------------------- weight quantizer KAT (quantize.rs:108-140)
def kat_input():
    i = np.arange(512)
    return ((((i * 7919) % 1000).astype(np.float32) / np.float32(500.0) - np.float32(1.0)) * np.float32(0.05)
            * (np.float32(1.0) + (i // 128).astype(np.float32))).astype(np.float32)


@pytest.mark.parametrize('bits', [4, 6, 8])
def test_quantizer_kat(bits):
    w = kat_input()
    k = w.size
    row = oracle.quantize_rows(w.reshape(1, k), bits)[0]
    nc = k // 32 * {8: 32, 6: 24, 4: 16}[bits]
    codes = oracle.unpack_row(row[:nc], bits, k)
    assert (oracle.pack(codes, bits) == row[:nc]).all(), 'pack/unpack roundtrip'
    c = row[nc:nc + 4].view('<f4')[0]
    m = row[nc + 4:].view('<u2')
    qmax = (1 << (bits - 1)) - 1
    assert np.abs(codes.astype(int)).max() <= qmax
    back = (c * m[np.arange(k) // 128].astype(np.float32)).astype(np.float32) * codes.astype(np.float32)
    for g in range(k // 128):
        amax = np.abs(w[g * 128:(g + 1) * 128]).max()
        err = np.abs(back[g * 128:(g + 1) * 128] - w[g * 128:(g + 1) * 128])
        assert (err <= amax / np.float32(qmax)).all(), f'W{bits} group {g}'
    assert m.max() == 65535 and m.min() >= 1          # c = max_g s_g / 65535: the largest group gets 65535


def test_quantizer_zero_group_and_numpy():
    rng = np.random.default_rng(3)
    w = (rng.standard_normal((5, 512)) * 0.02).astype(np.float32)
    w[2, 128:256] = 0.0
    w[4] = 0.0
    for bits in (4, 6, 8):
        rows = oracle.quantize_rows(w, bits)
        assert (rows == spec_np.quantize_rows(w, bits)).all()
        nc = 512 // 32 * {8: 32, 6: 24, 4: 16}[bits]
        assert (oracle.unpack_row(rows[2, :nc], bits, 512)[128:256] == 0).all()
        # an all-zero row: every group scale is 1.0, c = f32(1/65535), m = 65535, codes 0
        assert rows[4, nc:nc + 4].view('<f4')[0] == np.float32(1.0 / 65535.0)
        assert (rows[4, nc + 4:].view('<u2') == 65535).all()


# ---------------------------------------------------------------- packing layout (SPEC.md:30-36)
def test_pack_layout_by_hand():
    codes = np.zeros(32, np.int8)
    # W6: u = wq + 32; low nibbles: byte i = lo(u[i]) | lo(u[i+16]) << 4; high pairs: byte i = hi[i] | hi[i+8]<<2 | ...
    codes[:] = -32                      # u = 0 everywhere
    codes[17] = 5                       # u = 37 = 0b10_0101: lo 5 into byte 1's high nibble, hi 2 into byte 16+1 bits 4-5
    codes[3] = 31                       # u = 63: lo 15 into byte 3's low nibble, hi 3 into byte 16+3 bits 0-1
    p = oracle.pack(codes, 6)
    want = np.zeros(24, np.uint8)
    want[1] = 5 << 4
    want[16 + 1] = 2 << 4
    want[3] = 15
    want[16 + 3] = 3
    assert (p == want).all(), p
    # W4: u = wq + 8; byte i = u[i] | u[i+16] << 4
    c4 = np.full(32, -8, np.int8)
    c4[20] = 7                          # u = 15 into byte 4's high nibble
    c4[0] = 0                           # u = 8 into byte 0's low nibble
    p4 = oracle.pack(c4, 4)
    want4 = np.zeros(16, np.uint8)
    want4[4] = 15 << 4
    want4[0] = 8
    assert (p4 == want4).all()
    # W8: the code byte itself
    c8 = np.arange(-16, 16, dtype=np.int8)
    assert (oracle.pack(c8, 8) == c8.view(np.uint8)).all()


@pytest.mark.parametrize('bits', [4, 6, 8])
def test_pack_unpack_exhaustive(bits):
    lo, hi = (-8, 7) if bits == 4 else (-32, 31) if bits == 6 else (-128, 127)
    vals = np.arange(lo, hi + 1)
    k = ((vals.size + 31) // 32) * 32 * 2
    codes = np.resize(vals, k).astype(np.int8)
    codes[k // 2:] = np.random.default_rng(bits).permutation(codes[k // 2:])
    packed = oracle.pack(codes, bits)
    assert (oracle.unpack_row(packed, bits, k) == codes).all()
    assert (spec_np.unpack_codes(packed, bits, k) == codes).all()
    assert (spec_np.pack_codes(codes, bits) == packed).all()


# ---------------------------------------------------------------- exact integers
def test_gemm_acc_brute_force():
    rng = np.random.default_rng(11)
    for bits in (4, 6, 8):
        lo, hi = {4: (-8, 7), 6: (-32, 31), 8: (-128, 127)}[bits]
        k, n, mt = 256, 5, 3
        codes = rng.integers(lo, hi + 1, (n, k)).astype(np.int8)
        m = rng.integers(1, 65536, (n, k // 128)).astype(np.uint16)
        xq = rng.integers(-127, 128, (mt, k)).astype(np.int8)
        mx = rng.integers(0, 65536, (mt, k // 128)).astype(np.uint16)
        c = np.float32(rng.uniform(1e-8, 1e-6))
        sx = rng.uniform(1e-6, 1e-3, mt).astype(np.float32)
        for t in range(mt):
            for r in range(n):
                acc = 0
                for g in range(k // 128):
                    part = sum(int(codes[r, i]) * int(xq[t, i]) for i in range(g * 128, (g + 1) * 128))
                    acc += int(m[r, g]) * int(mx[t, g]) * part
                got = oracle.lib().ora_gemm_acc(codes[r].ctypes.data, m[r].ctypes.data, xq[t].ctypes.data,
                                                mx[t].ctypes.data, k)
                assert got == acc
                y = oracle.lib().ora_gemm_row(codes[r].ctypes.data, float(c), m[r].ctypes.data, xq[t].ctypes.data,
                                              float(sx[t]), mx[t].ctypes.data, k)
                want = np.float32(np.float32(rne_f32(acc) * c) * sx[t])
                assert f32_bits(y) == f32_bits(want)


def test_i64_to_f32_ties():
    rng = np.random.default_rng(5)
    vals = [0, 1, -1, (1 << 24) + 1, (1 << 24) + 3, -(1 << 63), (1 << 63) - 1]
    for s in range(1, 40):
        for _ in range(20):
            m = int(rng.integers(1 << 23, 1 << 24))
            half = 1 << (s - 1)
            for tail in (half, half + 1, half - 1, 1, (1 << s) - 1):
                vals += [(m << s) + tail, -((m << s) + tail)]
    for v in vals:
        assert f32_bits(oracle.lib().ora_i64_to_f32(v)) == f32_bits(rne_f32(v)), v


# ---------------------------------------------------------------- activation quantization
def test_quant_zero_row_and_max_group():
    x = np.zeros((2, 512), np.float32)
    x[1] = np.random.default_rng(1).standard_normal(512).astype(np.float32)
    xq, sx, mx = oracle.quant(x)
    assert sx[0] == 1.0 and (mx[0] == 1).all() and (xq[0] == 0).all()     # sx = 1 when smax == 0
    amax = np.abs(x[1].reshape(4, 128)).max(axis=1)
    gmax = int(amax.argmax())
    assert mx[1, gmax] == 65535                                             # the largest group
    assert np.abs(xq[1, gmax * 128:(gmax + 1) * 128]).max() == 127
    # reconstruction within half a step (plus fp32 slack) in every group
    eff = (sx[1] * mx[1].astype(np.float32)).astype(np.float64)
    rec = xq[1].astype(np.float64) * np.repeat(eff, 128)
    assert (np.abs(rec - x[1]) <= np.repeat(eff, 128) * 0.5 * (1 + 1e-5)).all()


def test_quant_power_of_two_invariance():
    x = np.random.default_rng(2).standard_normal((3, 384)).astype(np.float32)
    xq, sx, mx = oracle.quant(x)
    for e in (-20, -3, 5, 30):
        y = (x * np.float32(2.0 ** e)).astype(np.float32)
        yq, sy, my = oracle.quant(y)
        assert (yq == xq).all() and (my == mx).all()
        assert (sy == (sx * np.float32(2.0 ** e)).astype(np.float32)).all()


def test_quant_underflow_rust_casts():
    """smax > 0 but smax / 65535 underflows to 0 (spec/quant.rs:31-45): s_g / 0 is inf -> m = 65535, 0/0 is NaN ->
    `as u16` gives 0; the codes of a group whose effective scale is 0 are x * inf: +-127 or NaN -> 0."""
    x = np.zeros((1, 256), np.float32)
    x[0, 5] = np.float32(1e-45)          # smallest denormal: s_0 = 1e-45/127 rounds to 0 -> smax = 0 after all
    xq, sx, mx = oracle.quant(x)
    assert sx[0] == 1.0                   # s_g underflowed to 0, so smax == 0
    x[0, 5] = np.float32(3e-39)           # s_0 = 2.4e-41 (denormal), smax / 65535 underflows to 0
    xq, sx, mx = oracle.quant(x)
    assert sx[0] == 0.0
    assert mx[0, 0] == 65535 and mx[0, 1] == 0
    assert xq[0, 5] == 127 and (np.delete(xq[0], 5) == 0).all()


def test_quant_matches_numpy_on_norm_rows():
    from tests.helpers import norm_rows
    x, u, w = norm_rows(oracle.Rng(3), 12, 1024)
    for group in (True, False):
        a = oracle.quant(x, group=group)
        b = spec_np.quant_act_i8g(x) if group else spec_np.quant_act_i8(x)
        assert (a[0] == b[0]).all() and (f32_bits(a[1]) == f32_bits(b[1])).all()
        if group:
            assert (a[2] == b[2]).all()


# ---------------------------------------------------------------- conformance RNG (conformance.rs:35-59)
def test_rng_matches_python_xorshift():
    s = 11
    r = oracle.Rng(11)
    mask = (1 << 64) - 1
    for _ in range(1000):
        s ^= (s << 13) & mask
        s ^= s >> 7
        s ^= (s << 17) & mask
        assert r.next() == s
    r2 = oracle.Rng(99)
    v = r2.next()
    r3 = oracle.Rng(99)
    assert r3.byte() == v >> 56
    assert np.float32(oracle.Rng(99).unit()) == np.float32((v >> 11) / float(1 << 53) * 2.0 - 1.0)


# ---------------------------------------------------------------- golden fixtures
def test_golden_fixtures():
    z = np.load(GOLDEN)
    names = sorted({k.rsplit('_', 1)[0] for k in z.files if k.startswith('gemm_')})
    assert names
    for tag in names:
        bits = int(tag.split('_')[1][1:])
        n, k = (int(v) for v in tag.split('_')[2].split('x'))
        rows, x = z[f'{tag}_rows'], z[f'{tag}_x']
        xq, sx, mx = oracle.quant(x)
        assert (f32_bits(oracle.gemm(rows, n, k, bits, xq, sx, mx)) == f32_bits(z[f'{tag}_y'])).all(), tag
        ya = oracle.gemm(rows, n, k, bits, xq, sx, mx, y=z[f'{tag}_acc0'], accumulate=True)
        assert (f32_bits(ya) == f32_bits(z[f'{tag}_yacc'])).all(), tag
    xq, sx, mx = oracle.quant(z['quant_g_x'])
    assert (xq == z['quant_g_xq']).all() and (mx == z['quant_g_mx']).all()
    assert (f32_bits(sx) == f32_bits(z['quant_g_sx'])).all()
    xq, sx, _ = oracle.quant(z['quant_row_x'], group=False)
    assert (xq == z['quant_row_xq']).all() and (f32_bits(sx) == f32_bits(z['quant_row_sx'])).all()
    for key in z.files:
        if key.startswith('quantize_') and key.endswith('_rows'):
            bits = int(key.split('_')[2][1:])
            assert (oracle.quantize_rows(z[key[:-5] + '_w'], bits) == z[key]).all(), key


# ---------------------------------------------------------------- fp32 primitives of the fused producers
def ulp_err(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    ulp = np.spacing(np.abs(want).astype(np.float32)).astype(np.float64)
    return np.abs(got - want) / np.maximum(ulp, np.finfo(np.float32).smallest_subnormal)


def test_transcendentals_against_math():
    """exp_f / log_f / sigmoid_f / silu_f / softplus_f (spec/prim.rs:78-149) stay within a few ulp of the exact
    functions (a wrong constant, sign or step would not), hit their closed forms, and follow their clamps."""
    L = oracle.lib()
    xs = np.linspace(-86.0, 88.0, 20001).astype(np.float32)
    e = np.array([L.ora_exp_f(float(v)) for v in xs], np.float32)
    assert ulp_err(e, np.exp(xs.astype(np.float64))).max() <= 2.0
    assert L.ora_exp_f(0.0) == 1.0 and L.ora_exp_f(-87.5) == 0.0
    assert L.ora_exp_f(1000.0) == L.ora_exp_f(88.0)                     # clamped at 88
    ps = np.exp(np.linspace(-80, 80, 20001)).astype(np.float32)
    lg = np.array([L.ora_log_f(float(v)) for v in ps], np.float32)
    err = np.abs(lg.astype(np.float64) - np.log(ps.astype(np.float64)))
    assert (err <= 4 * np.spacing(np.maximum(np.abs(np.log(ps)), 1e-3).astype(np.float32))).all()
    assert L.ora_log_f(1.0) == 0.0
    zs = np.linspace(-30, 30, 6001).astype(np.float32)
    sg = np.array([L.ora_sigmoid_f(float(v)) for v in zs], np.float32)
    assert ulp_err(sg, 1.0 / (1.0 + np.exp(-zs.astype(np.float64)))).max() <= 4.0
    si = np.array([L.ora_silu_f(float(v)) for v in zs], np.float32)
    assert ulp_err(si, zs.astype(np.float64) / (1.0 + np.exp(-zs.astype(np.float64)))).max() <= 6.0
    sp = np.array([L.ora_softplus_f(float(v)) for v in zs], np.float32)
    # log_f(1 + exp_f(x)) for -15 <= x <= 20 rounds 1 + e^x first: a few ulp of (1 + e^x) absolute
    true_sp = np.log1p(np.exp(zs.astype(np.float64)))
    bound = 4 * np.spacing((1.0 + np.exp(zs.astype(np.float64))).astype(np.float32)).astype(np.float64)
    assert (np.abs(sp.astype(np.float64) - true_sp) <= np.maximum(bound, 6 * np.spacing(true_sp.astype(np.float32)))).all()
    low = np.linspace(-40, -15.01, 500).astype(np.float32)                # x < -15: exp_f(x) itself
    assert all(L.ora_softplus_f(float(v)) == L.ora_exp_f(float(v)) for v in low)
    assert L.ora_softplus_f(25.0) == 25.0                                 # x > 20 returns x


def test_treesum_order():
    """treesum is the balanced pairwise tree over the row padded to a power of two (spec/prim.rs:154-170)."""
    L = oracle.lib()
    v = np.array([1e8, 1.0, 1.0, 1.0, -1e8, 3.0], np.float32)   # padded to 8: ((1e8+1)+(1+1)) + ((-1e8+3)+(0+0))
    f = np.float32
    want = (f(f(1e8) + f(1)) + f(f(1) + f(1))) + (f(f(-1e8) + f(3)) + f(0))
    assert np.float32(L.ora_treesum(v.ctypes.data, v.size)) == want
    ints = np.arange(1, 1001, dtype=np.float32)                   # exact integer sums are order-free
    assert L.ora_treesum(ints.ctypes.data, ints.size) == 500500.0


# ---------------------------------------------------------------- the quantizer's scale search (quantize.rs:33-55)
# A one-group row (K = 128) keeps its chosen scale s in the row: m = 65535 and c = f32(s / 65535), so s is read
# back to within 2^-23 relative, and the step follows from s / base = 0.80 + 0.02 step (steps 2 % apart).
def chosen_step(w, bits):
    qmax = (1 << (bits - 1)) - 1
    row = oracle.quantize_rows(np.asarray(w, np.float32).reshape(1, 128), bits)[0]
    nc = 4 * {8: 32, 6: 24, 4: 16}[bits]
    c = float(row[nc:nc + 4].view('<f4')[0])
    assert row[nc + 4:].view('<u2')[0] == 65535
    base = float(np.abs(np.asarray(w, np.float64)).max()) / qmax
    r = (c * 65535.0 / base - 0.80) / 0.02
    step = int(round(r))
    assert abs(r - step) < 1e-3, r
    return step


def exact_sse(w, bits, step):
    """The squared error of candidate `step` in exact rational arithmetic (no float rounding anywhere)."""
    qmax = (1 << (bits - 1)) - 1
    wv = [Fraction(float(v)) for v in np.asarray(w, np.float32)]
    base = max(abs(v) for v in wv) / qmax
    s = base * (Fraction(4, 5) + Fraction(step, 50))
    err = Fraction(0)
    for v in wv:
        x = v / s
        q = round(x)                       # Python rounds halves to even, as round_ties_even
        q = max(-qmax, min(qmax, q))
        err += (q * s - v) ** 2
    return err


def brute_step(w, bits):
    """The first candidate of least exact error, and the margin to the runner-up (relative)."""
    errs = [exact_sse(w, bits, k) for k in range(11)]
    best = min(range(11), key=lambda k: (errs[k], k))
    others = [e for k, e in enumerate(errs) if k != best]
    return best, float((min(others) - errs[best]) / max(min(others), Fraction(1, 10 ** 30)))


def test_scale_search_step10_exact_grid():
    """Every value an integer multiple of base (a power of two): step 10 has zero error and every other step clamps
    amax, so step 10 is the unique best; a loop that stops at step 9 fails."""
    for bits in (4, 6, 8):
        qmax = (1 << (bits - 1)) - 1
        b = 2.0 ** -9
        j = (np.arange(128) * 37) % (2 * qmax + 1) - qmax
        j[5] = qmax
        w = (j * b).astype(np.float32)
        assert brute_step(w, bits)[0] == 10
        assert chosen_step(w, bits) == 10


def test_scale_search_every_step():
    """For each candidate k: amax = qmax * base and the other values on the grid of s_k (multiples j s_k that stay
    unclamped), drawn with a preference for multiples far from the other candidates' grids.  Step k then has the
    amax term as its only error; the first seeded draw whose exact brute-force winner is k by a clear margin is kept,
    and the oracle must pick k for it.  With one clamped amax the small steps can only win at W4 (the amax error
    (qmax (0.2 - 0.02 k) base)^2 outgrows what 127 grid values can cost the other steps): W4 isolates all 11 steps,
    W6 steps 5-10, W8 steps 9-10.  That fixes the first candidate (0.80), the increment (0.02) and the count (11): a
    wrong start, increment or range picks another scale."""
    rng = np.random.default_rng(1)
    reach = {4: range(0, 11), 6: range(5, 11), 8: range(9, 11)}
    for bits in (4, 6, 8):
        qmax = (1 << (bits - 1)) - 1
        for k in reach[bits]:
            base = 2.0 ** -8
            s = base * (0.80 + 0.02 * k)
            lim = min(qmax, int(qmax * base / s))      # multiples that stay unclamped at s_k
            cand = np.arange(1, lim + 1)
            v = cand * (0.80 + 0.02 * k)
            far = sum((np.abs(v / sm - np.round(v / sm)) * sm) ** 2
                      for sm in (0.80 + 0.02 * m for m in range(11) if m != k))
            for _ in range(300):
                p = np.exp(far * rng.uniform(1, 40))
                j = rng.choice(cand, 128, p=p / p.sum()) * rng.choice([-1, 1], 128)
                w = (j * s).astype(np.float32)
                w[7] = np.float32(qmax * base)
                best, margin = brute_step(w, bits)
                if best == k and margin > 0.01:
                    break
            else:
                raise AssertionError(f'no isolating group for W{bits} step {k}')
            assert chosen_step(w, bits) == k, (bits, k)


def test_scale_search_random_groups_against_exact_brute_force():
    """Gaussian groups: whenever the exact brute force has a winner by a margin well above f64 rounding, the oracle
    picks it."""
    rng = np.random.default_rng(4)
    checked = 0
    for bits in (4, 6, 8):
        for _ in range(40):
            w = (rng.standard_normal(128) * 0.02).astype(np.float32)
            best, margin = brute_step(w, bits)
            if margin < 1e-9:
                continue
            assert chosen_step(w, bits) == best
            checked += 1
    assert checked > 100


def f64_sse(w, bits, step):
    """The squared error of candidate `step` as quantize.rs:40-49 computes it: binary64, summed in element order."""
    qmax = (1 << (bits - 1)) - 1
    wd = [float(v) for v in np.asarray(w, np.float32)]
    base = max(abs(v) for v in wd) / qmax
    s = base * (0.80 + 0.02 * step)
    err = 0.0
    for v in wd:
        q = max(-qmax, min(qmax, round(v / s)))
        err += (q * s - v) * (q * s - v)
    return err


@pytest.mark.parametrize('bits', [4, 6])
@pytest.mark.parametrize('scale', [1.0, 2.0 ** -12])
def test_scale_search_tie_takes_the_first(bits, scale):
    """Two candidates with identical least error, exactly and in binary64: the strict < keeps the earlier one
    (quantize.rs:50-52).  A <= comparison, or a search that runs from step 10 down, picks the later step and fails."""
    (first, second), _ = TIE_GROUPS[bits]
    w = tie_group(bits, scale)
    exact = [exact_sse(w, bits, k) for k in range(11)]
    assert exact[first] == exact[second] == min(exact)
    assert sorted(exact).count(min(exact)) == 2
    f64 = [f64_sse(w, bits, k) for k in range(11)]
    assert f64[first] == f64[second] == min(f64)
    assert chosen_step(w, bits) == first
    # the two choices store different c (one group per row: c = f32(s / 65535), m = 65535), so a byte comparison of
    # rows also tells them apart
    qmax = (1 << (bits - 1)) - 1
    base = float(np.abs(w).max()) / qmax
    c_first, c_second = (np.float32(base * (0.80 + 0.02 * k) / 65535.0) for k in (first, second))
    assert c_first != c_second
    row = oracle.quantize_rows(w.reshape(1, 128), bits)[0]
    assert row[128 * bits // 8:][:4].view('<f4')[0] == c_first


def test_scale_search_zero_group():
    """An all-zero group takes scale 1.0 (quantize.rs:35-37): c = f32(1 / 65535), m = 65535, codes 0."""
    for bits in (4, 6, 8):
        row = oracle.quantize_rows(np.zeros((1, 128), np.float32), bits)[0]
        nc = 4 * {8: 32, 6: 24, 4: 16}[bits]
        assert row[nc:nc + 4].view('<f4')[0] == np.float32(1.0 / 65535.0)
        assert row[nc + 4:].view('<u2')[0] == 65535
        assert (oracle.unpack_row(row[:nc], bits, 128) == 0).all()


def test_quant_act_multiplies_by_the_reciprocal():
    """quant_act_i8g (spec/quant.rs:21-49) scales by inv = 1 / (sx * mx), a multiply, not a division: values where
    rint(x * f32(1 / eff)) and rint(x / eff) differ follow the multiply.  The row has one group whose max sets
    sx = amax / 127 / 65535 and mx = 65535."""
    rng = np.random.default_rng(8)
    found = 0
    for _ in range(2000):
        amax = np.float32(rng.uniform(0.5, 2.0))
        sg = np.float32(amax / np.float32(127.0))
        sx = np.float32(sg / np.float32(65535.0))
        eff = np.float32(sx * np.float32(65535.0))
        inv = np.float32(np.float32(1.0) / eff)
        # candidates just around the rounding midpoints j + 1/2
        x = np.float32((rng.integers(0, 127) + 0.5) * float(eff))
        for cand in (x, np.nextafter(x, np.float32(0)), np.nextafter(x, np.float32(10))):
            a = np.rint(np.float32(cand * inv))
            b = np.rint(np.float32(cand / eff))
            if a != b and abs(cand) < amax:
                row = np.zeros((1, 128), np.float32)
                row[0, 0] = amax
                row[0, 1] = cand
                xq, sxo, mxo = oracle.quant(row)
                assert sxo[0] == sx and mxo[0, 0] == 65535
                assert xq[0, 1] == int(a), (cand, a, b)
                found += 1
    assert found >= 3, found
