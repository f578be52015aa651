"""Pins of the mixer oracle (oracle/mixer_oracle.c) against what the mathematics fixes (CPU only).

Each check is chosen so that a plausible mistake in the restatement fails it: l2norm vs rmsnorm, the rope
rotation's sign and halves, rint ties and the int16 clamp, the softmax fixed point's numerator/denominator, the
grouped-query head mapping (h // rep, not h % n_kv), causality and the cache position of each token, the orientation
of the Gated DeltaNet state ([dk][dv]) and the order of its update, the conv window's age order, and argmax ties.
"""
import ctypes

import numpy as np
import pytest

import oracle

f32 = np.float32


def L():
    return oracle.lib()


def P(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def test_l2norm_closed_form():
    x = np.array([3, 4], f32)
    y = np.zeros(2, f32)
    L().ora_l2norm(P(x), 0.0, 2, P(y))
    inv = f32(1) / np.sqrt(f32(25))            # 1/5, not 1/sqrt(25/2) as rmsnorm would give
    assert y.tolist() == [f32(3) * inv, f32(4) * inv]
    z = np.zeros(4, f32)
    L().ora_l2norm(P(z), 1e-6, 4, P(y := np.ones(4, f32)))
    assert (y == 0).all()                      # eps keeps the zero row finite


def test_rope_rotation():
    x = np.array([2, 3, 5, 7], f32)            # half = 2: pairs (x0, x2), (x1, x3)
    cs, sn = np.array([0, 1], f32), np.array([1, 0], f32)
    L().ora_rope(P(x), P(cs), P(sn), 2)
    assert x.tolist() == [-5, 3, 2, 7]          # pair 0 rotated by +90 degrees: (a, b) -> (-b, a); pair 1 untouched


def test_quant_v_ties_and_clamp():
    v = np.array([0.5, 1.5, 2.5, -0.5, -1.5, 40000, -40000, 32767.4], f32)
    q = np.zeros(8, np.int16)
    L().ora_quant_v(P(v), 1.0, 8, P(q))
    assert q.tolist() == [0, 2, 2, 0, -2, 32767, -32767, 32767]
    q2 = np.zeros(2, np.int16)
    L().ora_quant_v(P(np.array([1.0, -3.0], f32)), 2.0, 2, P(q2))
    assert q2.tolist() == [2, -6]


def _head(qq, sq, kq, sk, vq, vs):
    hd = len(qq)
    o = np.zeros(hd, f32)
    L().ora_attn_head(P(qq), sq, P(kq), P(sk), P(vq), len(sk), hd, 1, vs, hd, P(o))
    return o


def test_attn_head_single_key_and_two_keys():
    rng = np.random.default_rng(1)
    hd = 8
    qq = rng.integers(-127, 128, hd).astype(np.int8)
    kq = rng.integers(-127, 128, (3, hd)).astype(np.int8)
    vq = rng.integers(-30000, 30000, (3, hd)).astype(np.int16)
    sk = np.array([0.01, 0.02, 0.015], f32)
    # one key: pq = 2^24, o = (f32(2^24 v) / f32(2^24)) * vs = v * vs exactly
    o = _head(qq, f32(0.03), kq[:1], sk[:1], vq[:1], f32(0.5))
    assert o.tolist() == (vq[0].astype(f32) * f32(0.5)).tolist()
    # three keys: integer numerator and denominator from the fixed-point weights (python ints)
    s = [(f32(int(np.dot(qq.astype(np.int64), kq[j].astype(np.int64)))) * f32(0.03)) * sk[j] for j in range(3)]
    mx = max(s)
    pq = [int(np.rint(f32(L().ora_exp_f(f32(sj - mx))) * f32(16777216.0))) for sj in s]
    num = [sum(pq[j] * int(vq[j][i]) for j in range(3)) for i in range(hd)]
    want = [f32(f32(n) / f32(sum(pq))) * f32(0.5) for n in num]
    assert _head(qq, f32(0.03), kq, sk, vq, f32(0.5)).tolist() == want
    assert pq[int(np.argmax(s))] == 1 << 24


def _attention(n_h, n_kv, hd, M, pos0, qg, k, v, cache=None, rot=4, cap=8, vscale=None):
    rng = np.random.default_rng(5)
    q_norm = (1 + 0.1 * rng.standard_normal(hd)).astype(f32)
    k_norm = (1 + 0.1 * rng.standard_normal(hd)).astype(f32)
    v_scale = np.array(vscale if vscale is not None else [1 / 1024] * n_kv, f32)
    v_inv = (f32(1) / v_scale).astype(f32)
    half = rot // 2
    pos = np.arange(cap, dtype=np.float64)[:, None] * (1.0 / 10000 ** (np.arange(half) / half))[None, :]
    cos, sin = np.cos(pos).astype(f32), np.sin(pos).astype(f32)
    if cache is None:
        cache = (np.zeros((cap, n_kv, hd), np.int8), np.zeros((cap, n_kv), f32), np.zeros((cap, n_kv, hd), np.int16))
    kq, sk, vq = cache
    o = np.zeros((M, n_h, hd), f32)
    L().ora_attention(P(q_norm), P(k_norm), P(v_scale), P(v_inv), P(kq), P(sk), P(vq), P(qg), P(k), P(v), P(cos),
                      P(sin), rot, 1e-6, M, pos0, n_h, n_kv, hd, P(o))
    return o, cache


def _sig(x):
    return np.array([L().ora_sigmoid_f(f32(t)) for t in x.ravel()], f32).reshape(x.shape)


def test_attention_single_position_gqa_mapping():
    """At position 0 every head sees one key, so o = vq * v_scale * sigmoid(gate) of its own kv head: head h reads
    kv head h // rep."""
    rng = np.random.default_rng(2)
    n_h, n_kv, hd = 4, 2, 8
    qg = rng.standard_normal((1, n_h, 2 * hd)).astype(f32)
    k = rng.standard_normal((1, n_kv, hd)).astype(f32)
    v = (rng.standard_normal((1, n_kv, hd)) * 0.1).astype(f32)
    vs = [1 / 1024, 1 / 512]
    o, (_, _, vq) = _attention(n_h, n_kv, hd, 1, 0, qg, k, v, vscale=vs)
    for h in range(n_h):
        kvh = h // 2
        want = (vq[0, kvh].astype(f32) * f32(vs[kvh])) * _sig(qg[0, h, hd:])
        assert o[0, h].tolist() == want.tolist(), h
    assert not np.array_equal(o[0, 1], o[0, 2])       # h % n_kv would pair heads 0, 2 and 1, 3


def test_attention_batch_equals_token_by_token():
    """Causality and cache positions: two tokens at once give the outputs and cache rows of two single steps."""
    rng = np.random.default_rng(3)
    n_h, n_kv, hd = 2, 1, 8
    qg = rng.standard_normal((2, n_h, 2 * hd)).astype(f32)
    k = rng.standard_normal((2, n_kv, hd)).astype(f32)
    v = (rng.standard_normal((2, n_kv, hd)) * 0.1).astype(f32)
    o2, c2 = _attention(n_h, n_kv, hd, 2, 0, qg, k, v)
    oa, ca = _attention(n_h, n_kv, hd, 1, 0, qg[:1].copy(), k[:1].copy(), v[:1].copy())
    ob, cb = _attention(n_h, n_kv, hd, 1, 1, qg[1:].copy(), k[1:].copy(), v[1:].copy(), cache=ca)
    assert np.array_equal(o2[0], oa[0]) and np.array_equal(o2[1], ob[0])
    for x, y in zip(c2, cb):
        assert np.array_equal(x, y)
    assert not np.array_equal(o2[1], oa[0])


def test_gdn_head_step_closed_form():
    """From a zero state one step gives S[i][j] = k[i] * (v[j] * beta) and o[j] = S[0][j] q[0] + S[1][j] q[1]
    (dk = 2 != dv = 3 fixes the orientation); a second step decays, subtracts the memory and adds again."""
    k = np.array([0.6, -0.8], f32)
    q = np.array([0.25, 0.5], f32)
    v = np.array([1.0, -2.0, 0.5], f32)
    beta, decay = f32(0.75), f32(0.9)
    s = np.zeros((2, 3), f32)
    o = np.zeros(3, f32)
    L().ora_gdn_head_step(P(s), 2, 3, P(k), P(q), P(v), beta, decay, P(o))
    S = np.zeros((2, 3), f32)
    for j in range(3):
        delta = (v[j] - f32(0)) * beta
        S[:, j] = f32(0) + k * delta
    assert np.array_equal(s, S)
    assert o.tolist() == [(S[0, j] * q[0]) + (S[1, j] * q[1]) for j in range(3)]
    v2 = np.array([0.1, 0.2, 0.3], f32)
    L().ora_gdn_head_step(P(s), 2, 3, P(k), P(q), P(v2), beta, decay, P(o))
    for j in range(3):
        col = S[:, j] * decay
        kv = (col[0] * k[0]) + (col[1] * k[1])
        delta = (v2[j] - kv) * beta
        S[:, j] = col + k * delta
    assert np.array_equal(s, S)


def test_gdn_conv_window_order_and_decay():
    win = np.array([1, 2, 3, 4], f32)           # oldest first, the current input last
    assert L().ora_gdn_conv(P(win), P(np.array([0, 0, 0, 1], f32))) == L().ora_silu_f(4.0)
    assert L().ora_gdn_conv(P(win), P(np.array([1, 0, 0, 0], f32))) == L().ora_silu_f(1.0)
    assert L().ora_gdn_decay(3.0, -3.0, 0.0) == 1.0                # A = 0: no decay
    assert L().ora_gdn_decay(20.0, 5.0, 1.0) == L().ora_exp_f(-25.0)   # softplus(25) = 25 above its threshold


def _gdn(M, qkv, z, a, b, state=None, n_k=1, n_v=2, dk=4, dv=4):
    rng = np.random.default_rng(9)
    conv_dim = 2 * n_k * dk + n_v * dv
    conv_w = (rng.standard_normal((conv_dim, 4)) * 0.5).astype(f32)
    A = np.array([0.5, 1.5][:n_v], f32)
    dt = np.array([0.1, -0.2][:n_v], f32)
    norm = (1 + 0.1 * rng.standard_normal(dv)).astype(f32)
    if state is None:
        state = (np.zeros((3, conv_dim), f32), np.zeros((n_v, dk, dv), f32))
    cs, S = state
    on = np.zeros((M, n_v, dv), f32)
    L().ora_gdn(P(conv_w), P(A), P(dt), P(norm), P(cs), P(S), P(qkv), P(z), P(a), P(b), 1e-6, M, n_k, n_v, dk, dv,
                P(on))
    return on, state


def test_gdn_batch_equals_token_by_token():
    """The conv window and the recurrent state carry from call to call exactly as within one call."""
    rng = np.random.default_rng(4)
    n_k, n_v, dk, dv = 1, 2, 4, 4
    conv_dim = 2 * n_k * dk + n_v * dv
    qkv = rng.standard_normal((3, conv_dim)).astype(f32)
    z = rng.standard_normal((3, n_v, dv)).astype(f32)
    a = rng.standard_normal((3, n_v)).astype(f32)
    b = rng.standard_normal((3, n_v)).astype(f32)
    o3, s3 = _gdn(3, qkv, z, a, b)
    o1, s1 = _gdn(1, qkv[:1].copy(), z[:1].copy(), a[:1].copy(), b[:1].copy())
    o2, s2 = _gdn(2, qkv[1:].copy(), z[1:].copy(), a[1:].copy(), b[1:].copy(), state=s1)
    assert np.array_equal(o3[:1], o1) and np.array_equal(o3[1:], o2)
    assert np.array_equal(s3[0], s2[0]) and np.array_equal(s3[1], s2[1])
    assert not np.array_equal(o3[0], o3[1])


def test_argmax_first_of_ties():
    for x, want in (([1, 3, 3, 2], 1), ([-np.inf, -5], 1), ([0.0, -0.0], 0), ([2, 1], 0)):
        a = np.array(x, f32)
        assert L().ora_argmax(P(a), len(a)) == want
