"""Second, independent restatement of det's quantized-linear numerics in numpy (TEST INFRASTRUCTURE ONLY).

Written from the format and GEMM text of docs/SPEC.md (sections 2-3, lines 27-64) and the search rule of
crates/det/src/quantize.rs:33-85, vectorised over whole rows with numpy instead of the scalar loops of
det_oracle.c, so that a slip in one restatement shows up as a disagreement with the other.  Only tests/
and tests/golden/make_golden.py import it.
"""
import numpy as np

GROUP = 128
F32 = np.float32


def bytes_per_32(bits):
    return {8: 32, 6: 24, 4: 16}[bits]


def row_bytes(bits, k):
    return k // 32 * bytes_per_32(bits) + 4 + 2 * (k // GROUP)


def unpack_codes(packed, bits, k):
    """SPEC.md:30-36 packing per 32 weights -> signed codes, packed is uint8 [..., k/32*bpl]."""
    p = packed.reshape(packed.shape[:-1] + (k // 32, bytes_per_32(bits)))
    if bits == 8:
        q = p.view(np.int8).astype(np.int16)
    elif bits == 4:
        u = np.concatenate([p & 0xF, p >> 4], axis=-1).astype(np.int16)  # byte i = u[i] | u[i+16] << 4
        q = u - 8
    else:
        lo = np.concatenate([p[..., :16] & 0xF, p[..., :16] >> 4], axis=-1).astype(np.int16)
        hb = p[..., 16:24]
        # byte i = hi[i] | hi[i+8]<<2 | hi[i+16]<<4 | hi[i+24]<<6
        hi = np.concatenate([(hb >> (2 * j)) & 3 for j in range(4)], axis=-1).astype(np.int16)
        q = (lo | (hi << 4)) - 32
    return q.reshape(packed.shape[:-1] + (k,)).astype(np.int8)


def pack_codes(q, bits):
    """Inverse of unpack_codes (SPEC.md:30-36), q int8 [..., k]."""
    k = q.shape[-1]
    b = q.reshape(q.shape[:-1] + (k // 32, 32)).astype(np.int16)
    if bits == 8:
        out = b.astype(np.int8).view(np.uint8)
    elif bits == 4:
        u = (b + 8).astype(np.uint8)
        out = u[..., :16] | (u[..., 16:] << 4)
    else:
        u = (b + 32).astype(np.uint8)
        lo = (u[..., :16] & 0xF) | ((u[..., 16:] & 0xF) << 4)
        h = u >> 4
        hi = h[..., 0:8] | (h[..., 8:16] << 2) | (h[..., 16:24] << 4) | (h[..., 24:32] << 6)
        out = np.concatenate([lo, hi], axis=-1)
    return out.astype(np.uint8).reshape(q.shape[:-1] + (k // 32 * bytes_per_32(bits),))


def split_rows(rows, bits, k):
    """det rows [N][row_bytes] -> (codes int8 [N][k], c f32 [N], m u16 [N][G])  (SPEC.md:36, 168-177)."""
    nc = k // 32 * bytes_per_32(bits)
    codes = unpack_codes(rows[:, :nc], bits, k)
    c = rows[:, nc:nc + 4].copy().view('<f4').reshape(-1)
    m = rows[:, nc + 4:].copy().view('<u2')
    return codes, c, m


def quant_act_i8g(x):
    """SPEC.md:45-48 quant_act_i8g over rows of x [M][n] -> (xq int8, sx f32 [M], mx u16 [M][G])."""
    x = np.asarray(x, dtype=F32)
    M, n = x.shape
    G = n // GROUP
    xg = x.reshape(M, G, GROUP)
    amax = np.abs(xg).max(axis=-1)                       # order-free; |x| >= +0 so -0 never wins
    s_g = (amax / F32(127)).astype(F32)
    smax = s_g.max(axis=-1)
    with np.errstate(divide='ignore', invalid='ignore', over='ignore'):
        sx = np.where(smax == 0, F32(1), smax / F32(65535)).astype(F32)
        m = np.rint((s_g / sx[:, None]).astype(F32))
        m = np.where(m < 1, F32(1), np.where(m > 65535, F32(65535), m))
        mx = np.where(np.isnan(m), 0, m).astype(np.uint16)  # Rust `as u16`: NaN -> 0
        eff = (sx[:, None] * mx.astype(F32)).astype(F32)
        inv = (F32(1) / eff).astype(F32)
        v = np.rint((xg * inv[:, :, None]).astype(F32))
    v = np.where(v < -127, F32(-127), np.where(v > 127, F32(127), v))
    xq = np.where(np.isnan(v), 0, v).astype(np.int8)     # Rust `as i8`: NaN -> 0
    return xq.reshape(M, n), sx, mx


def quant_act_i8(x):
    """SPEC.md:49-50 quant_act_i8: per row s = amax/127 (1 if amax == 0), q = clamp(rint(x/s))."""
    x = np.asarray(x, dtype=F32)
    amax = np.abs(x).max(axis=-1)
    with np.errstate(divide='ignore', invalid='ignore', over='ignore'):
        s = np.where(amax == 0, F32(1), amax / F32(127)).astype(F32)
        inv = (F32(1) / s).astype(F32)
        v = np.rint((x * inv[:, None]).astype(F32))
    v = np.where(v < -127, F32(-127), np.where(v > 127, F32(127), v))
    return np.where(np.isnan(v), 0, v).astype(np.int8), s


def gemm_acc(codes, m, xq, mx):
    """SPEC.md:58-60 exact integer acc[t][n] (int64) = sum_g (m[n,g]*mx[t,g]) * sum_{k in g} wq*xq."""
    N, K = codes.shape
    M = xq.shape[0]
    G = K // GROUP
    w = codes.astype(np.int64).reshape(N, G, GROUP)
    x = xq.astype(np.int64).reshape(M, G, GROUP)
    part = np.einsum('tgk,ngk->tng', x, w)               # |part| < 2^21
    mult = mx.astype(np.int64)[:, None, :] * m.astype(np.int64)[None, :, :]
    return (part * mult).sum(axis=-1)                     # exact in int64 (< 2^61)


def gemm(rows, bits, k, xq, sx, mx):
    """SPEC.md:58-61 y[t][n] = (float32(acc) * c[n]) * sx[t]."""
    codes, c, m = split_rows(rows, bits, k)
    if mx is None:
        mx = np.ones((xq.shape[0], k // GROUP), np.uint16)
    acc = gemm_acc(codes, m, xq, mx)
    f = acc.astype(F32)                                   # int64 -> fp32, round to nearest even
    return ((f * c[None, :]).astype(F32) * sx[:, None]).astype(F32)


def quantize_rows(w, bits):
    """SPEC.md:38-41 + quantize.rs:33-85: per group the best of 11 scales by sequential f64 squared error."""
    w = np.asarray(w, dtype=F32)
    N, K = w.shape
    G = K // GROUP
    qmax = float((1 << (bits - 1)) - 1)
    wd = w.astype(np.float64).reshape(N, G, GROUP)
    amax = np.abs(wd).max(axis=-1)
    base = amax / qmax
    best_err = np.full((N, G), np.inf)
    best = base.copy()
    with np.errstate(divide='ignore', invalid='ignore'):
        for step in range(11):
            s = base * (0.80 + 0.02 * step)
            q = np.clip(np.rint(wd / s[..., None]), -qmax, qmax)
            d = q * s[..., None] - wd
            err = np.add.accumulate(d * d, axis=-1)[..., -1]   # sequential sum, index order
            better = err < best_err
            best_err = np.where(better, err, best_err)
            best = np.where(better, s, best)
    scales = np.where(amax == 0, 1.0, best)
    smax = scales.max(axis=-1)
    c = (smax / 65535.0).astype(F32)
    m = np.clip(np.rint(scales / c.astype(np.float64)[:, None]), 1.0, 65535.0).astype(np.uint16)
    eff = c.astype(np.float64)[:, None] * m.astype(np.float64)
    codes = np.clip(np.rint(wd / eff[..., None]), -qmax, qmax).astype(np.int8).reshape(N, K)
    out = np.concatenate([pack_codes(codes, bits), c.reshape(N, 1).view(np.uint8),
                          m.astype('<u2').view(np.uint8)], axis=-1)
    return out
