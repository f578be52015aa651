"""The model runner (det_model.h; the reference's Model + qwen35::forward) end to end on the GPU against an oracle
forward, bit for bit: a synthetic qwen35 float model (one Gated DeltaNet layer with 2 key / 4 value heads of 128,
one attention layer with 2 heads over 1 kv head of 128 dims and 64 rotary dims, SwiGLU MLPs, untied head) is
converted by the library's det_convert; the oracle side reads the converter restatement's bytes
(tests/gguf_ref.convert_ref, byte-identical to det_convert's output by tests/test_convert.py) and runs
qwen35.rs:8-172 with the oracle's ops (rmsnorm_quant, gemm, attention, gdn, quant, silu_mul_quant, argmax).
Logits after a batched prefill, after prefill chunks of max_batch and after single-token decode steps, and a
greedy generation, must match exactly."""
import ctypes
import os

import numpy as np
import pytest

import oracle
from det_amd import ffi, gguf
from tests import gguf_ref as R
from tests.test_convert import synthetic_model, write_model

pytestmark = pytest.mark.gpu
f32 = np.float32
BITS = '6,output=8,ssm_alpha=8,ssm_beta=8'
CTX = 40


def P(a):
    return a.ctypes.data_as(ctypes.c_void_p)


class OracleModel:
    """qwen35::forward (qwen35.rs:8-172) and Model::forward / embed_rows (model.rs:390-466) over the oracle."""

    def __init__(self, data, ctx=CTX, fast=False):
        """data: the det GGUF's bytes.  fast: the GEMMs on det's x86 GEMM restated in C (oracle/x86_gemm.c, pinned
        bit for bit to the scalar oracle) instead of the scalar oracle."""
        self.ctx, self.fast, self.x86 = ctx, fast, {}
        kv, self.t = R.read_gguf(data)
        a = lambda k: kv['qwen35.' + k][1]
        self.h, self.ff = a('embedding_length'), a('feed_forward_length')
        self.n_h, self.n_kv, self.hd, self.rot = (a('attention.head_count'), a('attention.head_count_kv'),
                                                  a('attention.key_length'), a('rope.dimension_count'))
        self.eps = f32(a('attention.layer_norm_rms_epsilon'))
        self.n_k, self.n_v, self.dk = a('ssm.group_count'), a('ssm.time_step_rank'), a('ssm.state_size')
        self.dv = a('ssm.inner_size') // self.n_v
        n_layers = a('block_count') - kv.get('qwen35.nextn_predict_layers', (0, 0))[1]
        self.attn = [(i + 1) % a('full_attention_interval') == 0 for i in range(n_layers)]
        self.vs = np.array(kv['det.v_scale'][1][1], f32)
        self.vocab = self.t['token_embd.weight'][0][1]
        self.cd = 2 * self.n_k * self.dk + self.n_v * self.dv
        self.reset()

    def reset(self):
        self.pos = 0
        self.kv = [(np.zeros((self.ctx, self.n_kv, self.hd), np.int8), np.zeros((self.ctx, self.n_kv), f32),
                    np.zeros((self.ctx, self.n_kv, self.hd), np.int16)) if at else None for at in self.attn]
        self.gs = [None if at else (np.zeros((3, self.cd), f32), np.zeros((self.n_v, self.dk, self.dv), f32))
                   for at in self.attn]

    def vec(self, name):
        dims, ty, data = self.t[name]
        return R.f32s(ty, data, int(np.prod(dims)))

    def gemm(self, name, xq, sx, mx, y=None, acc=False):
        dims, ty, data = self.t[name]
        K, N = dims
        bits = {v: b for b, v in R.DET.items()}[ty]
        rows = np.frombuffer(data, np.uint8).reshape(N, -1)
        if not self.fast:
            return oracle.gemm(rows, N, K, bits, xq, sx, mx, y=y, accumulate=acc)
        if name not in self.x86:
            self.x86[name] = oracle.X86Linear(rows, N, K, bits)
        v = self.x86[name].gemm(xq, sx, mx)
        return (y + v).astype(f32) if acc else v

    def forward(self, ids):
        t = len(ids)
        emb = self.t['token_embd.weight']
        x = np.stack([R.f32s(emb[1], emb[2][2 * self.h * i:2 * self.h * (i + 1)], self.h) for i in ids]).astype(f32)
        L = oracle.lib()
        cos, sin = self.vec('rope_cos').reshape(-1, self.rot // 2), self.vec('rope_sin').reshape(-1, self.rot // 2)
        ai = 0
        for li, at in enumerate(self.attn):
            b = f'blk.{li}.'
            xq, sx, mx = oracle.rmsnorm_quant(x, self.vec(b + 'attn_norm.weight'), self.eps)
            if at:
                qg = self.gemm(b + 'attn_q.weight', xq, sx, mx)
                k = self.gemm(b + 'attn_k.weight', xq, sx, mx)
                v = self.gemm(b + 'attn_v.weight', xq, sx, mx)
                vs = self.vs[ai * self.n_kv:(ai + 1) * self.n_kv].copy()
                ai += 1
                vi = (f32(1) / vs).astype(f32)
                kq, sk, vq = self.kv[li]
                o = np.zeros((t, self.n_h * self.hd), f32)
                L.ora_attention(P(self.vec(b + 'attn_q_norm.weight')), P(self.vec(b + 'attn_k_norm.weight')), P(vs),
                                P(vi), P(kq), P(sk), P(vq), P(qg), P(k), P(v), P(cos), P(sin), self.rot, self.eps, t,
                                self.pos, self.n_h, self.n_kv, self.hd, P(o))
                oq, so, mo = oracle.quant(o)
                x = self.gemm(b + 'attn_output.weight', oq, so, mo, y=x, acc=True)
            else:
                qkv = self.gemm(b + 'attn_qkv.weight', xq, sx, mx)
                z = self.gemm(b + 'attn_gate.weight', xq, sx, mx)
                aa = self.gemm(b + 'ssm_alpha.weight', xq, sx, mx)
                bb = self.gemm(b + 'ssm_beta.weight', xq, sx, mx)
                cs, S = self.gs[li]
                on = np.zeros((t, self.n_v * self.dv), f32)
                A = (-self.vec(b + 'ssm_a')).astype(f32)
                L.ora_gdn(P(self.vec(b + 'ssm_conv1d.weight')), P(A), P(self.vec(b + 'ssm_dt.bias')),
                          P(self.vec(b + 'ssm_norm.weight')), P(cs), P(S), P(qkv), P(z), P(aa), P(bb), self.eps, t,
                          self.n_k, self.n_v, self.dk, self.dv, P(on))
                oq, so, mo = oracle.quant(on)
                x = self.gemm(b + 'ssm_out.weight', oq, so, mo, y=x, acc=True)
            xq, sx, mx = oracle.rmsnorm_quant(x, self.vec(b + 'post_attention_norm.weight'), self.eps)
            g = self.gemm(b + 'ffn_gate.weight', xq, sx, mx)
            u = self.gemm(b + 'ffn_up.weight', xq, sx, mx)
            hq, sh, mh = oracle.silu_mul_quant(g, u)
            x = self.gemm(b + 'ffn_down.weight', hq, sh, mh, y=x, acc=True)
        xq, sx, mx = oracle.rmsnorm_quant(x[t - 1:], self.vec('output_norm.weight'), self.eps)
        self.pos += t
        return self.gemm('output.weight', xq, sx, mx)[0]


class Runner:
    """det_model.h through ctypes."""

    def __init__(self, path, ctx, batch):
        L = ffi.lib()
        c = ctypes
        for name, (res, args) in {'det_model_load': (c.c_void_p, [c.c_char_p, c.c_int, c.c_int]),
                                  'det_model_free': (None, [c.c_void_p]), 'det_model_last_error': (c.c_char_p, []),
                                  'det_model_vocab': (c.c_int, [c.c_void_p]), 'det_model_pos': (c.c_int, [c.c_void_p]),
                                  'det_model_reset': (None, [c.c_void_p]),
                                  'det_model_forward': (c.c_int, [c.c_void_p, c.c_void_p, c.c_int]),
                                  'det_model_prefill': (c.c_int, [c.c_void_p, c.c_void_p, c.c_int]),
                                  'det_model_logits': (c.c_int, [c.c_void_p, c.c_void_p]),
                                  'det_model_argmax': (c.c_int, [c.c_void_p]),
                                  'det_model_generate': (c.c_int, [c.c_void_p, c.c_void_p, c.c_int, c.c_int, c.c_void_p,
                                                                   c.c_int, c.c_void_p])}.items():
            getattr(L, name).restype, getattr(L, name).argtypes = res, args
        self.L = L
        self.m = L.det_model_load(os.fsencode(str(path)), ctx, batch)
        if not self.m:
            raise RuntimeError(L.det_model_last_error().decode())
        self.vocab = L.det_model_vocab(self.m)

    def check(self, rc):
        if rc < 0:
            raise RuntimeError(self.L.det_model_last_error().decode())
        return rc

    def prefill(self, ids):
        a = np.array(ids, np.int32)
        self.check(self.L.det_model_prefill(self.m, P(a), len(a)))

    def logits(self):
        out = np.zeros(self.vocab, f32)
        self.check(self.L.det_model_logits(self.m, P(out)))
        return out

    def __del__(self):
        if getattr(self, 'm', None):
            self.L.det_model_free(self.m)


@pytest.fixture(scope='module')
def model_files(tmp_path_factory):
    d = tmp_path_factory.mktemp('e2e')
    model = synthetic_model(seed=7)
    src, dst = d / 'm-BF16.gguf', d / 'm-det.gguf'
    write_model(src, model)
    gguf.convert(src, dst, BITS, CTX)
    ref = R.convert_ref(model, BITS, CTX)
    assert dst.read_bytes() == ref
    return dst, ref


def same(a, b):
    return np.array_equal(np.asarray(a, f32).view(np.uint32), np.asarray(b, f32).view(np.uint32))


def test_prefill_chunks_and_decode(model_files):
    path, ref = model_files
    print('e2e: prefill 11 tokens in batches of 8, then 4 decode steps', flush=True)
    run, ora = Runner(path, CTX, 8), OracleModel(ref)
    rng = np.random.default_rng(1)
    prompt = rng.integers(0, ora.vocab, 11).tolist()
    run.prefill(prompt)
    ora.forward(prompt[:8])
    want = ora.forward(prompt[8:])
    assert same(run.logits(), want), 'logits after the prefill'
    for step in range(4):
        nxt = int(rng.integers(0, ora.vocab))
        run.prefill([nxt])
        assert same(run.logits(), ora.forward([nxt])), f'logits after decode step {step}'
    assert run.L.det_model_pos(run.m) == 15
    # reset: the same prompt again gives the same logits
    run.L.det_model_reset(run.m)
    ora.reset()
    run.prefill(prompt[:5])
    assert same(run.logits(), ora.forward(prompt[:5]))


def test_greedy_generation(model_files):
    path, ref = model_files
    print('e2e: greedy generation of 6 tokens after a 7-token prompt', flush=True)
    run, ora = Runner(path, CTX, 16), OracleModel(ref)
    prompt = [3, 141, 59, 26, 5, 35, 89]
    out = np.zeros(6, np.int32)
    pa = np.array(prompt, np.int32)
    n = run.check(run.L.det_model_generate(run.m, P(pa), len(pa), 6, None, 0, P(out)))
    assert n == 6
    logits = ora.forward(prompt)
    want = []
    for i in range(6):
        nxt = int(oracle.lib().ora_argmax(P(logits), len(logits)))
        want.append(nxt)
        if i + 1 < 6:
            logits = ora.forward([nxt])
    assert out.tolist() == want


def test_errors(model_files, tmp_path):
    path, _ = model_files
    run = Runner(path, 8, 4)
    with pytest.raises(RuntimeError, match='batch of 5 tokens'):
        run.prefill_one = run.check(run.L.det_model_forward(run.m, P(np.zeros(5, np.int32)), 5))
    with pytest.raises(RuntimeError, match='outside the embedding table'):
        run.check(run.L.det_model_forward(run.m, P(np.array([run.vocab], np.int32)), 1))
    run.prefill([1, 2, 3, 4])
    run.prefill([1, 2, 3, 4])
    with pytest.raises(RuntimeError, match='exceed the context of 8'):
        run.check(run.L.det_model_forward(run.m, P(np.array([1], np.int32)), 1))
    with pytest.raises(RuntimeError, match='rope tables cover 40 positions, context 64 requested'):
        Runner(path, 64, 4)
