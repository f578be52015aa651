"""BASELINE configs[4] parity: the random-init qwen35 of the 4B architecture (32 layers, hidden 2560, FFN 9728, 16
q / 4 kv heads of 256 with 64 rotary dims, GDN 16 key / 32 value heads of 128, vocab 248320) written as a bf16 GGUF
(seed 5, bench.write_qwen35_bf16), converted by the library's det_convert with det's defaults (W6, W8 head and GDN
a|b, --no-calibrate), then run by the model runner (det_model.h): a 512-token prompt of uniform ids (seed 11)
prefilled in one batch, then greedy decoding.

The oracle forward (tests/test_model_e2e.OracleModel: qwen35.rs:8-172 over the oracle's ops, GEMMs on det's x86
GEMM restated in C, equal to the scalar oracle by tests/test_model_oracle.py) reads the converted file.  That file is
det_convert's output, byte-exact to the converter's restatement on the synthetic models of tests/test_convert.py;
here a row sample of every quantized tensor kind is re-quantized from the bf16 source by the oracle's quantizer.
Checked bit for bit: the logits after the 512-token prefill, the logits after each of the first 3 greedy decode
steps (one token per forward), and the 128 greedy tokens of det_model_generate from the same prompt.
Progress lines are appended to test_model_4b.log in the output folder that travels back from a GPU run (the test
runs for minutes).
"""
import os
import time

import numpy as np
import pytest

import bench
import oracle
from det_amd import gguf
from tests import gguf_ref as R
from tests.test_model_e2e import OracleModel, Runner, P, same

pytestmark = pytest.mark.gpu

N_DECODE = 128
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def log(msg, t0=[time.time()]):
    line = f'[{time.time() - t0[0]:7.1f}s] {msg}'
    print(line, flush=True)
    d = os.path.join(ROOT, 'gpurun_out')          # a file that keeps growing shows a long run is alive
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, 'test_model_4b.log'), 'a') as f:
        f.write(line + '\n')


@pytest.mark.long
@pytest.mark.timeout(1500)
def test_qwen35_4b_prefill_512_and_greedy_decode(tmp_path):
    cfg = dict(bench.QWEN35_4B)
    src, dst = tmp_path / 'q35-4b-BF16.gguf', tmp_path / 'q35-4b-det.gguf'
    log('writing the bf16 source')
    bench.write_qwen35_bf16(str(src), cfg, seed=5, progress=log)
    log(f'converting ({os.path.getsize(src) / 1e9:.2f} GB)')
    gguf.convert(str(src), str(dst), None, cfg['ctx'])
    data = dst.read_bytes()
    log(f'converted ({len(data) / 1e9:.2f} GB); quantization spot check')
    check_rows_against_source(str(src), data)
    os.remove(src)

    prompt = np.random.default_rng(11).integers(0, cfg['vocab'], 512).tolist()
    log('GPU: load and prefill 512')
    run = Runner(dst, cfg['ctx'], 512)
    run.prefill(prompt)
    got0 = run.logits()
    log('oracle: prefill 512')
    ora = OracleModel(data, ctx=cfg['ctx'], fast=True)
    want = ora.forward(prompt)
    assert same(got0, want), 'logits after the 512-token prefill'
    toks = []
    for step in range(N_DECODE):
        nxt = int(oracle.lib().ora_argmax(P(want), len(want)))
        toks.append(nxt)
        if step + 1 == N_DECODE:
            break
        want = ora.forward([nxt])
        if step < 3:
            run.prefill([nxt])
            assert same(run.logits(), want), f'logits after decode step {step}'
        if step % 16 == 0:
            log(f'oracle: decode step {step}')
    log('GPU: greedy generation of 128 tokens from the same prompt')
    run.L.det_model_reset(run.m)
    out = np.zeros(N_DECODE, np.int32)
    pa = np.array(prompt, np.int32)
    n = run.check(run.L.det_model_generate(run.m, P(pa), len(pa), N_DECODE, None, 0, P(out)))
    assert n == N_DECODE
    assert out.tolist() == toks, 'greedy tokens'
    log('done')


def check_rows_against_source(src_path, det_data):
    """Rows of several quantized tensors, re-quantized from the bf16 source by the oracle's quantizer, equal the
    converted file's rows (the GDN value-head reorder of qkv is avoided: the rows checked are the q/k rows)."""
    with open(src_path, 'rb') as f:
        head = f.read(1 << 20)
    kv_s, st = read_table(head)
    data_start = st.pop('__data__')
    _, dt = R.read_gguf(det_data)
    with open(src_path, 'rb') as f:
        for name, row_ids in (('output.weight', (0, 124160, 248319)), ('blk.0.ffn_down.weight', (0, 2559)),
                              ('blk.3.attn_q.weight', (0, 8191)), ('blk.5.ffn_up.weight', (17, 9727)),
                              ('blk.0.attn_qkv.weight', (0, 4095))):
            dims, ty, data = dt[name]
            K, N = dims
            bits = {v: b for b, v in R.DET.items()}[ty]
            rows = np.frombuffer(data, np.uint8).reshape(N, -1)
            sdims, sty, soff = st[name]
            assert sty == 30 and sdims == [K, N]
            for r in row_ids:
                f.seek(data_start + soff + 2 * K * r)
                b16 = np.frombuffer(f.read(2 * K), np.uint16)
                w = (b16.astype(np.uint32) << 16).view(np.float32).reshape(1, K)
                assert (oracle.quantize_rows(w, bits)[0] == rows[r]).all(), f'{name} row {r}'


def read_table(head):
    """GGUF v3 header and tensor table (name -> (dims, type, offset)) of a file's first bytes; '__data__' is the
    data section's start (gguf.rs:261-300)."""
    import struct
    pos = 4
    ver, nt, nkv = struct.unpack_from('<IQQ', head, pos)
    pos += 20
    assert ver == 3

    def string():
        nonlocal pos
        (n,) = struct.unpack_from('<Q', head, pos)
        s = head[pos + 8:pos + 8 + n].decode()
        pos += 8 + n
        return s
    kv = {}
    for _ in range(nkv):
        k = string()
        (ty,) = struct.unpack_from('<I', head, pos)
        pos += 4
        if ty == 8:
            kv[k] = string()
        else:
            kv[k] = struct.unpack_from('<f' if ty == 6 else '<I', head, pos)[0]
            pos += 4
    t = {}
    for _ in range(nt):
        name = string()
        (nd,) = struct.unpack_from('<I', head, pos)
        pos += 4
        dims = list(struct.unpack_from(f'<{nd}Q', head, pos))
        pos += 8 * nd
        ty, off = struct.unpack_from('<IQ', head, pos)
        pos += 12
        t[name] = (dims, ty, off)
    t['__data__'] = pos + (-pos % 32)
    return kv, t
