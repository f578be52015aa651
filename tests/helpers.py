"""Input builders shared by the parity tests (TEST INFRASTRUCTURE).

The conformance inputs follow the reference suite (crates/det/src/conformance.rs:104-160,348-449) with its
xorshift64 Rng; the BASELINE-config inputs are seeded numpy Gaussians quantized by det's quantizer rules.
"""
import numpy as np

import oracle
from oracle import spec_np


def same_f32(a, b):
    """conformance.rs:63-78 `same`: bit-exact, any two NaNs match.  Returns None or a description."""
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    assert a.shape == b.shape, (a.shape, b.shape)
    bad = (a.view(np.uint32) != b.view(np.uint32)) & ~(np.isnan(a) & np.isnan(b))
    if not bad.any():
        return None
    i = int(np.flatnonzero(bad)[0])
    return f'{int(bad.sum())} of {a.size} differ, first at {i}: cpu {a[i]!r} ({a.view(np.uint32)[i]:#010x}) ' \
           f'gpu {b[i]!r} ({b.view(np.uint32)[i]:#010x})'


def same_int(a, b):
    a = np.asarray(a).reshape(-1)
    b = np.asarray(b).reshape(-1)
    assert a.shape == b.shape
    bad = a != b
    if not bad.any():
        return None
    i = int(np.flatnonzero(bad)[0])
    return f'{int(bad.sum())} of {a.size} differ, first at {i}: cpu {a[i]} gpu {b[i]}'


def gaussian_weights(seed, N, K, std=0.02):
    return (np.random.default_rng(seed).standard_normal((N, K), dtype=np.float32) * np.float32(std)).astype(np.float32)


def baseline_acts(seed, M, K, every37=True, zero_row=None):
    """fp32 N(0,1) rows; every 37th row scaled by 1e-3; optionally one all-zero row."""
    x = np.random.default_rng(seed).standard_normal((M, K), dtype=np.float32)
    if every37:
        x[::37] *= np.float32(1e-3)
    if zero_row is not None and zero_row < M:
        x[zero_row] = 0.0
    return x


def norm_rows(rng, m, n):
    """conformance.rs:464-501 row classes for the quantization suites (x and u)."""
    x = np.zeros(m * n, np.float32)
    for i in range(m * n):
        row, col = divmod(i, n)
        r6 = row % 6
        if r6 == 0:
            v = rng.denorm()
        elif r6 == 1:
            v = rng.denorm() if col % 2 == 0 else np.float32(0.0)
        elif r6 == 2:
            c8 = col % 8
            v = (np.float32(rng.unit()) * np.float32(1e-20) if c8 == 0 else
                 np.float32(rng.unit()) * np.float32(1e-23) if c8 == 1 else
                 rng.denorm() if c8 == 2 else
                 np.float32(rng.unit()) if c8 == 3 else
                 np.float32(0.0) if c8 == 4 else
                 np.float32(rng.unit()) * np.float32(1e-30) if c8 == 5 else
                 np.float32(-0.0) if c8 == 6 else
                 np.float32(rng.unit()) * np.float32(1e3))
        elif r6 == 3:
            v = np.float32(rng.unit()) * (np.float32(1e-19) if col % 5 == 0 else np.float32(1e-38))
        else:
            p = np.float32(1.0)
            for _ in range((i // 128) % 4):
                p = np.float32(p * np.float32(10.0))
            v = np.float32(rng.unit()) * (np.float32(1.0) / p)
        x[i] = v
    u = np.zeros(m * n, np.float32)
    for i in range(m * n):
        c3 = (i % n) % 3
        u[i] = (np.float32(rng.unit()) * np.float32(1e-20) if c3 == 0 else rng.denorm() if c3 == 1
                else np.float32(rng.unit()) * np.float32(3.0))
    w = np.array([np.float32(1.0) + np.float32(rng.unit()) for _ in range(n)], np.float32)
    return x.reshape(m, n), u.reshape(m, n), w


def make_group(p, xq_group, wmax):
    """Codes wq[128] with sum(wq * xq_group) == p (xq_group = [127]*r + small weights), |wq| <= wmax."""
    small = [i for i, v in enumerate(xq_group) if v != 127]
    big = [i for i, v in enumerate(xq_group) if v == 127]
    wq = np.zeros(128, np.int64)
    # residue through the small entries (greedy from the largest weight), rest through the 127s
    best = None
    sv = [int(xq_group[i]) for i in small]
    import itertools
    rng_vals = range(-wmax, wmax + 1)
    for combo in itertools.product(rng_vals, repeat=len(small)) if len(small) <= 2 else []:
        r = p - sum(a * b for a, b in zip(combo, sv))
        if r % 127 == 0 and abs(r // 127) <= wmax * len(big):
            best = combo
            break
    assert best is not None, p
    for i, v in zip(small, best):
        wq[i] = v
    a = (p - sum(a * b for a, b in zip(best, sv))) // 127
    for i in big:
        step = max(-wmax, min(wmax, a))
        wq[i] = step
        a -= step
    assert a == 0
    assert int((wq * np.asarray(xq_group, np.int64)).sum()) == p
    return wq.astype(np.int8)


def det_rows_from(codes, c, m, bits):
    """Assemble det rows [codes][c][m] (spec/tensor.rs:49-55) from signed codes [N][K], c [N], m [N][G]."""
    N, K = codes.shape
    packed = spec_np.pack_codes(np.asarray(codes, np.int8), bits)
    return np.concatenate([packed, np.asarray(c, np.float32).reshape(N, 1).view(np.uint8),
                           np.asarray(m, '<u2').view(np.uint8)], axis=1)
