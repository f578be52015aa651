"""det_attention / det_gdn / det_argmax through the C ABI against the oracle (oracle/mixer_oracle.c), bit for bit:
outputs, the KV cache rows (kq, sk, vq), the conv window and the recurrent state, over batches of tokens fed in
order (prefill, then single-token steps), at the 4B-class shapes (attention 16 heads over 4 kv heads of 256 dims
with 64 rotary dims; Gated DeltaNet 16 k heads, 32 v heads, dk = dv = 128) and small ones.  The reference backend
(cpu.rs:212-383) is what the oracle restates.
"""
import ctypes

import numpy as np
import pytest

import oracle
from det_amd import ffi

pytestmark = pytest.mark.gpu
f32 = np.float32


def P(a):
    return a.ctypes.data_as(ctypes.c_void_p)


def rope_tables(cap, half, theta=10000000.0):
    pos = np.arange(cap, dtype=np.float64)[:, None]
    inv = 1.0 / theta ** (np.arange(half, dtype=np.float64) / max(half, 1))
    return np.cos(pos * inv).astype(f32), np.sin(pos * inv).astype(f32)


def check_attention(n_h, n_kv, hd, rot, steps, cap, seed, v_amp=0.05, zero_k=False):
    rng = np.random.default_rng(seed)
    q_norm = (1 + 0.2 * rng.standard_normal(hd)).astype(f32)
    k_norm = (1 + 0.2 * rng.standard_normal(hd)).astype(f32)
    v_scale = (np.array([1 / 1024, 1 / 256, 1 / 2048, 1 / 512] * n_kv)[:n_kv]).astype(f32)
    v_inv = (f32(1) / v_scale).astype(f32)
    cos, sin = rope_tables(cap, rot // 2)
    dev = {n: ffi.Buf.upload(a) for n, a in (('qn', q_norm), ('kn', k_norm), ('vs', v_scale), ('vi', v_inv),
                                             ('cos', cos), ('sin', sin))}
    layer = ffi.AttnLayer(dev['qn'].ptr, dev['kn'].ptr, dev['vs'].ptr, dev['vi'].ptr)
    kq_d, sk_d, vq_d = ffi.Buf((cap, n_kv, hd), np.int8), ffi.Buf((cap, n_kv), f32), ffi.Buf((cap, n_kv, hd), np.int16)
    kv = ffi.KvCache(kq_d.ptr, sk_d.ptr, vq_d.ptr, cap, None, None)
    kq, sk, vq = np.zeros((cap, n_kv, hd), np.int8), np.zeros((cap, n_kv), f32), np.zeros((cap, n_kv, hd), np.int16)
    pos = 0
    L = oracle.lib()
    for M in steps:
        print(f'attention n_h={n_h} n_kv={n_kv} hd={hd} rot={rot} pos0={pos} M={M}', flush=True)
        qg = rng.standard_normal((M, n_h, 2 * hd)).astype(f32)
        k = rng.standard_normal((M, n_kv, hd)).astype(f32)
        v = (rng.standard_normal((M, n_kv, hd)) * v_amp).astype(f32)
        if zero_k:
            k[0, 0] = 0
        bufs = [ffi.Buf.upload(a) for a in (qg, k, v)]
        o_d = ffi.Buf((M, n_h, hd), f32)
        ffi.attention(layer, kv, bufs[0], bufs[1], bufs[2], dev['cos'], dev['sin'], rot, 1e-6, M, pos, n_h, n_kv, hd, o_d)
        o = np.zeros((M, n_h, hd), f32)
        L.ora_attention(P(q_norm), P(k_norm), P(v_scale), P(v_inv), P(kq), P(sk), P(vq), P(qg), P(k), P(v), P(cos),
                        P(sin), rot, 1e-6, M, pos, n_h, n_kv, hd, P(o))
        got = o_d.download()
        assert np.array_equal(got.view(np.uint32), o.view(np.uint32)), f'o differs at M={M} pos0={pos}'
        pos += M
        assert np.array_equal(kq_d.download()[:pos], kq[:pos])
        assert np.array_equal(sk_d.download()[:pos].view(np.uint32), sk[:pos].view(np.uint32))
        assert np.array_equal(vq_d.download()[:pos], vq[:pos])


def test_attention_4b_shape_prefill_then_decode():
    check_attention(16, 4, 256, 64, [37, 1, 1, 5], 64, seed=1)


def test_attention_4b_shape_decode_over_many_key_chunks():
    """Decode steps whose keys span many 32-key chunks, and batches spanning 256-key chunks."""
    check_attention(16, 4, 256, 64, [300, 1, 1, 3, 200, 1], 600, seed=6)


def test_attention_head_dim_128_batches():
    """hd = 128: the matrix-core batch path and the wave-per-row prep at two lanes' values each, GQA rep 4."""
    check_attention(8, 2, 128, 32, [40, 1, 7, 70], 128, seed=7)


def test_attention_long_prefill_chunks():
    """More than one 1024-key chunk in the weight pass, and the last cache row."""
    check_attention(2, 1, 64, 16, [1100, 1], 1101, seed=2)


def test_attention_small_heads_clamped_values_zero_key():
    check_attention(4, 2, 8, 4, [3, 1, 2], 8, seed=3, v_amp=100.0, zero_k=True)


def check_gdn(n_k, n_v, dk, dv, steps, seed):
    rng = np.random.default_rng(seed)
    cd = 2 * n_k * dk + n_v * dv
    conv_w = (rng.standard_normal((cd, 4)) * 0.5).astype(f32)
    A = (np.abs(rng.standard_normal(n_v)) + 0.1).astype(f32)
    dt = (rng.standard_normal(n_v) * 0.5).astype(f32)
    norm = (1 + 0.1 * rng.standard_normal(dv)).astype(f32)
    dev = {n: ffi.Buf.upload(a) for n, a in (('conv', conv_w), ('A', A), ('dt', dt), ('norm', norm))}
    layer = ffi.GdnLayer(dev['conv'].ptr, dev['A'].ptr, dev['dt'].ptr, dev['norm'].ptr)
    cs_d, S_d = ffi.Buf((3, cd), f32), ffi.Buf((n_v, dk, dv), f32)
    state = ffi.GdnState(cs_d.ptr, S_d.ptr)
    cs, S = np.zeros((3, cd), f32), np.zeros((n_v, dk, dv), f32)
    L = oracle.lib()
    for M in steps:
        print(f'gdn n_k={n_k} n_v={n_v} dk={dk} dv={dv} M={M}', flush=True)
        qkv = rng.standard_normal((M, cd)).astype(f32)
        z = rng.standard_normal((M, n_v, dv)).astype(f32)
        a = rng.standard_normal((M, n_v)).astype(f32)
        b = rng.standard_normal((M, n_v)).astype(f32)
        bufs = [ffi.Buf.upload(x) for x in (qkv, z, a, b)]
        on_d = ffi.Buf((M, n_v, dv), f32)
        scratch = ffi.Buf(ffi.gdn_scratch_bytes(M, n_k, n_v, dk, dv), np.uint8)
        ffi.gdn(layer, state, bufs[0], bufs[1], bufs[2], bufs[3], 1e-6, M, n_k, n_v, dk, dv, on_d, scratch)
        on = np.zeros((M, n_v, dv), f32)
        L.ora_gdn(P(conv_w), P(A), P(dt), P(norm), P(cs), P(S), P(qkv), P(z), P(a), P(b), 1e-6, M, n_k, n_v, dk, dv,
                  P(on))
        assert np.array_equal(on_d.download().view(np.uint32), on.view(np.uint32)), f'on differs at M={M}'
        assert np.array_equal(cs_d.download().view(np.uint32), cs.view(np.uint32))
        assert np.array_equal(S_d.download().view(np.uint32), S.view(np.uint32))


def test_gdn_4b_shape_prefill_then_decode():
    check_gdn(16, 32, 128, 128, [19, 1, 70, 1, 2], seed=4)


@pytest.mark.parametrize('n_k,n_v,dk,dv', [(1, 2, 4, 4), (2, 4, 8, 16), (1, 2, 16, 8), (1, 1, 32, 24),
                                           (2, 2, 64, 40), (1, 1, 128, 20), (1, 2, 64, 256)])
def test_gdn_small_shapes(n_k, n_v, dk, dv):
    # 33 and 64 tokens span two token chunks of the recurrence (a partial and a full second one)
    check_gdn(n_k, n_v, dk, dv, [1, 2, 5, 33, 64, 1], seed=5)


@pytest.mark.parametrize('V', [1, 5, 1000, 248320])
def test_argmax_first_of_ties(V):
    rng = np.random.default_rng(V)
    x = rng.standard_normal((3, V)).astype(f32)
    if V > 4:
        x[1, 2] = x[1, 4] = 100.0          # a tie: the lower index wins
        x[2, :] = -np.inf
        x[2, V - 1] = 0.0
    xd = ffi.Buf.upload(x)
    out = ffi.Buf(3, np.int32)
    ffi.argmax(xd, 3, V, out)
    L = oracle.lib()
    want = [L.ora_argmax(P(np.ascontiguousarray(x[m])), V) for m in range(3)]
    assert out.download().tolist() == want


def test_argmax_nan_and_signed_zero():
    """The spec's scan (l[i] > l[best]): a NaN at index 0 is kept, later NaNs are passed over, -0 equals +0."""
    rows = [[np.nan, 1.0, 2.0, 0.5], [-0.0, 0.0, -1.0, -0.0], [1.0, np.nan, 3.0, 3.0], [-np.inf, np.nan, -np.inf, -np.inf],
            [0.0, -0.0, np.nan, 0.0]]
    x = np.array(rows, dtype=f32)
    out = ffi.Buf(len(rows), np.int32)
    ffi.argmax(ffi.Buf.upload(x), len(rows), 4, out)
    L = oracle.lib()
    want = [L.ora_argmax(P(np.ascontiguousarray(r)), 4) for r in x]
    assert want == [0, 0, 2, 0, 0]
    assert out.download().tolist() == want
