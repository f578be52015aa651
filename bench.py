"""Benchmark of det's quantized-linear path on one MI355X (BASELINE.json metric and configs).

    python bench.py [--gpus 1] [--steps K] [--warmup W]

Workload (the prefill config; configs[0] rides along as the decode line):
  * step = one W6 x int8 GEMM, K=2560 -> N=9728, M=512 tokens (det_gemm_ex, GemmOut::Write), weights seeded
    N(0, 0.02) quantized by det's rules on the device (det_quantize_rows), activations N(0,1) with every 37th row
    x1e-3 and one all-zero row quantized by det_quant.  `value` = int8 TOPS (2*M*N*K per step).
  * the other configs[1] shapes (W6 M=64, W8 head K=2560 -> N=248320 at M=1 and 512) and configs[0] (W6 M=1 decode)
    are timed the same way and reported under "shapes", decode lines in GB/s of algorithmic bytes.
Inputs are resident in HBM before timing.  Each shape rotates over enough weight copies (> 512 MB in total) that
no launch finds its weights in the 256 MB Infinity Cache.  Kernel time comes from HIP events on the null stream
(the stream det's kernels run on) around the timed launches.
The CPU baseline (rank 0, N=1) times det's x86 GEMM algorithm restated in C (oracle/x86_gemm.c) on the same
quantized weights: the W6 M=512 GEMM on all host threads (at most 16) and on one, and the M=1 GEMVs of the W6
linear and the W8 head, each for a few seconds.
"""
import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

from det_amd import ffi  # noqa: E402

HBM_PEAK_GBS = 8000.0
# the kernel det_gemm_ex runs for the bench's M = 512 line (DET_PREFILL=streamk selects the stream-K kernel) and its
# grid (total threads, as rocprofv3 reports it) for the committed traffic summary
if os.environ.get('DET_PREFILL') == 'streamk':
    PREFILL_KERNEL, PREFILL_GRID = 'k_prefill<6>', 512 * 256
else:
    PREFILL_KERNEL, PREFILL_GRID = 'k_prefill2<6>', ((9728 + 63) // 64) * 4 * 256
INT8_PEAK_TOPS = 5000.0
ROTATE_BYTES = 600 << 20


class HipEvents:
    """hipEventRecord / hipEventElapsedTime on the null stream."""

    def __init__(self):
        self.h = ctypes.CDLL('libamdhip64.so')
        self.h.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.h.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.h.hipEventSynchronize.argtypes = [ctypes.c_void_p]
        self.h.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]

    def event(self):
        e = ctypes.c_void_p()
        assert self.h.hipEventCreate(ctypes.byref(e)) == 0
        return e

    def record(self, e):
        assert self.h.hipEventRecord(e, None) == 0

    def elapsed_ms(self, a, b):
        assert self.h.hipEventSynchronize(b) == 0
        ms = ctypes.c_float()
        assert self.h.hipEventElapsedTime(ctypes.byref(ms), a, b) == 0
        return ms.value


def row_bytes(bits, K):
    return K // 32 * {8: 32, 6: 24, 4: 16}[bits] + 4 + 2 * (K // 128)


def algo_bytes(N, K, M, bits):
    """Algorithmic bytes of one GEMM: packed weights with c and m, xq, mx, sx, y (Write)."""
    return N * row_bytes(bits, K) + M * K + 2 * M * (K // 128) + 4 * M + 4 * M * N


def make_linear_copies(N, K, bits, seed, min_bytes):
    """Quantize seeded N(0, 0.02) weights on the device and repack them into enough copies to exceed min_bytes.
    Returns the linears and the det rows (host copy, for the CPU baseline on the same weights)."""
    w = (np.random.default_rng(seed).standard_normal((N, K), dtype=np.float32) * np.float32(0.02))
    wd = ffi.Buf.upload(w)
    del w
    rows = ffi.quantize_rows(wd, N, K, bits)
    wd.free()
    one = N * row_bytes(bits, K)
    copies = max(1, -(-min_bytes // one))
    lins = [ffi.Linear(None, K, bits, rows_on_device=(rows, N)) for _ in range(copies)]
    host_rows = rows.download()
    rows.free()
    return lins, host_rows


def make_acts(M, K, seed):
    x = np.random.default_rng(seed).standard_normal((M, K), dtype=np.float32)
    x[::37] *= np.float32(1e-3)
    if M > 1:
        x[M // 2] = 0.0
    xb = ffi.Buf.upload(x)
    xq, sx, mx = ffi.Buf((M, K), np.int8), ffi.Buf(M, np.float32), ffi.Buf((M, K // 128), np.uint16)
    ffi.quant(xb, M, K, xq, sx, mx)
    return xq, sx, mx


def time_gemm(ev, lins, xq, sx, mx, M, y, steps, warmup):
    for i in range(warmup):
        ffi.gemm(lins[i % len(lins)], xq, sx, mx, M, write=y)
    ffi.lib().det_sync()
    a, b = ev.event(), ev.event()
    t0 = time.perf_counter()
    ev.record(a)
    for i in range(steps):
        ffi.gemm(lins[i % len(lins)], xq, sx, mx, M, write=y)
    ev.record(b)
    ms = ev.elapsed_ms(a, b)
    ffi.lib().det_sync()
    wall = time.perf_counter() - t0
    return ms / steps, wall


def read_floor(ev, nbytes, steps=200, grids=(512, 1024, 2048, 4096)):
    """The fastest plain streaming read (det_test_read) of `nbytes`, rotating over copies that exceed the Infinity
    Cache, over a few grid sizes: the floor a single-pass read of a GEMV's weight bytes can reach at that size.
    Returns (us, GB/s, grid)."""
    nb = (nbytes + 15) // 16 * 16
    copies = max(1, -(-ROTATE_BYTES // nb))
    bufs = [ffi.Buf(nb, np.uint8) for _ in range(copies)]
    sink = ffi.Buf(max(grids), np.uint32)
    L = ffi.lib()
    best = None
    for grid in grids:
        for i in range(10):
            L.det_test_read(bufs[i % copies].ptr, nb, grid, sink.ptr, None)
        a, b = ev.event(), ev.event()
        ev.record(a)
        for i in range(steps):
            L.det_test_read(bufs[i % copies].ptr, nb, grid, sink.ptr, None)
        ev.record(b)
        us = ev.elapsed_ms(a, b) * 1e3 / steps
        if best is None or us < best[0]:
            best = (us, nbytes / us / 1e3, grid)
    for b_ in bufs:
        b_.free()
    sink.free()
    return best


def shape_line(name, N, K, M, bits, ms):
    ops = 2.0 * M * N * K
    byt = algo_bytes(N, K, M, bits)
    tops = ops / (ms * 1e-3) / 1e12
    gbs = byt / (ms * 1e-3) / 1e9
    ai = ops / byt
    bound_tops = min(INT8_PEAK_TOPS, ai * HBM_PEAK_GBS / 1e3)
    bound = 'hbm' if bound_tops < INT8_PEAK_TOPS else 'mfma'
    return {'shape': name, 'bits': bits, 'M': M, 'N': N, 'K': K, 'us': round(ms * 1e3, 3), 'TOPS': round(tops, 2),
            'GBps': round(gbs, 1), 'bound': bound,
            'frac_of_bound': round((gbs / HBM_PEAK_GBS) if bound == 'hbm' else (tops / INT8_PEAK_TOPS), 4)}


def committed_traffic(kernel, grid):
    """HBM bytes per launch of `kernel` at `grid` from the committed FETCH_SIZE/WRITE_SIZE summary (scaled by the
    copy calibration), or None when the summary has no such row."""
    path = os.path.join(ROOT, 'profiles', 'gemm_hbm_traffic.md')
    if not os.path.exists(path):
        return None
    for line in open(path):
        cols = [c.strip().strip('`') for c in line.split('|')]
        if len(cols) > 6 and cols[1] == kernel and cols[2] == str(grid):
            return int(cols[6])
    return None


def cpu_model():
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('model name'):
                return line.split(':', 1)[1].strip()
    except OSError:
        pass
    return 'unknown'


def cpu_flags():
    try:
        for line in open('/proc/cpuinfo'):
            if line.startswith('flags'):
                return set(line.split(':', 1)[1].split())
    except OSError:
        pass
    return set()


def cpu_host_acts(M, K, seed):
    """The bench's activations (N(0,1), every 37th row x1e-3, one zero row) quantized by the oracle."""
    import oracle
    x = np.random.default_rng(seed).standard_normal((M, K), dtype=np.float32)
    x[::37] *= np.float32(1e-3)
    if M > 1:
        x[M // 2] = 0.0
    return oracle.quant(x)


def time_cpu(X, xq, sx, mx, threads, vnni, target_s):
    X.gemm(xq, sx, mx, vnni=vnni, threads=threads)            # warm-up
    reps, t0 = 0, time.perf_counter()
    while True:
        X.gemm(xq, sx, mx, vnni=vnni, threads=threads)
        reps += 1
        dt = time.perf_counter() - t0
        if dt > target_s:
            return dt / reps, reps, dt


def cpu_baseline(rows6, rows_head, target_s=5.0):
    """det's x86 backend GEMM (crates/det/src/x86/gemm.rs: strips of 8 rows, vpdpbusd on AVX-VNNI, else
    vpmaddubsw + vpmaddwd; restated in oracle/x86_gemm.c, checked bit for bit against the scalar oracle) on the
    GPU line's own quantized weights: the W6 M=512 GEMM on all of the host's threads (at most 16; `value`) and on
    one thread, and the M=1 decode GEMVs of the W6 linear and the W8 head in GB/s of algorithmic bytes, each
    repeated for about `target_s` seconds (det bench --gemm's figures, main.rs:343-423)."""
    import oracle
    threads = min(os.cpu_count() or 1, 16)
    threads = int(os.environ.get('OMP_NUM_THREADS', threads))
    vnni = oracle.has_vnni()
    K, M, N, NH = 2560, 512, 9728, 248320
    X6 = oracle.X86Linear(rows6, N, K, 6)
    xq, sx, mx = cpu_host_acts(M, K, 2)
    per, reps, dt = time_cpu(X6, xq, sx, mx, threads, vnni, target_s)
    tops = 2.0 * M * N * K / per / 1e12
    per1, reps1, dt1 = time_cpu(X6, xq, sx, mx, 1, vnni, target_s)
    xq1, sx1, mx1 = cpu_host_acts(1, K, 4)
    perd, _, _ = time_cpu(X6, xq1, sx1, mx1, threads, vnni, target_s / 2)
    XH = oracle.X86Linear(rows_head, NH, K, 8)
    perh, _, _ = time_cpu(XH, xq1, sx1, mx1, threads, vnni, target_s / 2)
    del XH
    flags = cpu_flags()
    return {'value': round(tops, 4), 'unit': 'TOPS', 'cores': threads, 'kind': 'port',
            'cpu': cpu_model(), 'nproc': os.cpu_count(), 'avx_vnni': 'avx_vnni' in flags,
            'avx512_vnni': 'avx512_vnni' in flags, 'path': 'AVX-VNNI vpdpbusd' if vnni else 'AVX2 vpmaddubsw',
            'w6_m512_tops_1_thread': round(2.0 * M * N * K / per1 / 1e12, 4),
            'w6_m1_gbps': round(algo_bytes(N, K, 1, 6) / perd / 1e9, 2),
            'w8_head_m1_gbps': round(algo_bytes(NH, K, 1, 8) / perh / 1e9, 2),
            'sample': f"det's x86 GEMM algorithm (crates/det/src/x86/gemm.rs) restated in C on the GPU line's "
                      f"weights: the whole W6 K=2560 N=9728 M=512 GEMM {reps} times in {dt:.1f} s on {threads} "
                      f"threads and {reps1} times in {dt1:.1f} s on 1 thread; M=1 GEMVs of it and of the W8 head"}


# ---------------------------------------------------------------- end to end
QWEN35_4B = dict(hidden=2560, layers=32, interval=4, ff=9728, heads=16, kv=4, hd=256, rot=64, nk=16, nv=32, dk=128,
                 dv=128, vocab=248320, ctx=640)


def write_qwen35_bf16(path, cfg, seed, progress=None):
    """A random-init qwen35 float GGUF of the given architecture (weights seeded N(0, 0.02), norms 1 + N(0, 0.02),
    ssm_a negative), BF16 matrices and F32 vectors, streamed to disk tensor by tensor."""
    import struct
    H, FF, V = cfg['hidden'], cfg['ff'], cfg['vocab']
    cd = 2 * cfg['nk'] * cfg['dk'] + cfg['nv'] * cfg['dv']
    qd, kvd, od = 2 * cfg['heads'] * cfg['hd'], cfg['kv'] * cfg['hd'], cfg['heads'] * cfg['hd']
    ts = [('token_embd.weight', [H, V], 'w'), ('output_norm.weight', [H], 'n'), ('output.weight', [H, V], 'w')]
    for i in range(cfg['layers']):
        b = f'blk.{i}.'
        ts += [(b + 'attn_norm.weight', [H], 'n'), (b + 'post_attention_norm.weight', [H], 'n'),
               (b + 'ffn_gate.weight', [H, FF], 'w'), (b + 'ffn_up.weight', [H, FF], 'w'),
               (b + 'ffn_down.weight', [FF, H], 'w')]
        if (i + 1) % cfg['interval'] == 0:
            ts += [(b + 'attn_q.weight', [H, qd], 'w'), (b + 'attn_k.weight', [H, kvd], 'w'),
                   (b + 'attn_v.weight', [H, kvd], 'w'), (b + 'attn_output.weight', [od, H], 'w'),
                   (b + 'attn_q_norm.weight', [cfg['hd']], 'n'), (b + 'attn_k_norm.weight', [cfg['hd']], 'n')]
        else:
            ts += [(b + 'attn_qkv.weight', [H, cd], 'w'), (b + 'attn_gate.weight', [H, cfg['nv'] * cfg['dv']], 'w'),
                   (b + 'ssm_alpha.weight', [H, cfg['nv']], 'w'), (b + 'ssm_beta.weight', [H, cfg['nv']], 'w'),
                   (b + 'ssm_out.weight', [cfg['nv'] * cfg['dv'], H], 'w'), (b + 'ssm_conv1d.weight', [4, cd], 'c'),
                   (b + 'ssm_a', [cfg['nv']], 'a'), (b + 'ssm_dt.bias', [cfg['nv']], 'c'),
                   (b + 'ssm_norm.weight', [cfg['dv']], 'n')]
    U32, F32, STR = 4, 6, 8
    kv = [('general.architecture', STR, 'qwen35'), ('qwen35.block_count', U32, cfg['layers']),
          ('qwen35.full_attention_interval', U32, cfg['interval']), ('qwen35.embedding_length', U32, H),
          ('qwen35.feed_forward_length', U32, FF), ('qwen35.attention.head_count', U32, cfg['heads']),
          ('qwen35.attention.head_count_kv', U32, cfg['kv']), ('qwen35.attention.key_length', U32, cfg['hd']),
          ('qwen35.attention.layer_norm_rms_epsilon', F32, 1e-6), ('qwen35.rope.dimension_count', U32, cfg['rot']),
          ('qwen35.rope.freq_base', F32, 10000000.0), ('qwen35.context_length', U32, cfg['ctx']),
          ('qwen35.ssm.state_size', U32, cfg['dk']), ('qwen35.ssm.time_step_rank', U32, cfg['nv']),
          ('qwen35.ssm.group_count', U32, cfg['nk']), ('qwen35.ssm.inner_size', U32, cfg['nv'] * cfg['dv']),
          ('qwen35.ssm.conv_kernel', U32, 4)]
    sizes = [int(np.prod(d)) * (2 if k == 'w' else 4) for _, d, k in ts]
    head = bytearray(b'GGUF') + struct.pack('<IQQ', 3, len(ts), len(kv))
    for key, ty, v in kv:
        head += struct.pack('<Q', len(key)) + key.encode() + struct.pack('<I', ty)
        head += (struct.pack('<Q', len(v)) + v.encode()) if ty == STR else struct.pack('<f' if ty == F32 else '<I', v)
    off = 0
    for (name, dims, kind), nb in zip(ts, sizes):
        head += struct.pack('<Q', len(name)) + name.encode() + struct.pack('<I', len(dims))
        head += b''.join(struct.pack('<Q', d) for d in dims) + struct.pack('<IQ', 30 if kind == 'w' else 0, off)
        off += nb + (-nb % 32)
    head += bytes(-len(head) % 32)
    # every tensor is drawn in chunks of CHUNK values, chunk j of tensor idx from its own generator [seed, idx, j], so
    # the chunks can be drawn by a pool of threads (numpy's generators release the GIL) and written in file order
    CHUNK = 1 << 24
    jobs = []
    for idx, ((name, dims, kind), nb) in enumerate(zip(ts, sizes)):
        n = int(np.prod(dims))
        for j, lo in enumerate(range(0, n, CHUNK)):
            jobs.append((idx, j, kind, min(CHUNK, n - lo), lo + CHUNK >= n, nb))

    def draw(job):
        idx, j, kind, n, last, nb = job
        a = np.random.default_rng([seed, idx, j]).standard_normal(n, dtype=np.float32) * np.float32(0.02)
        if kind == 'n':
            a = a + np.float32(1)
        elif kind == 'a':
            a = -np.abs(a) - np.float32(1)
        data = (a.view(np.uint32) >> 16).astype(np.uint16).tobytes() if kind == 'w' else a.tobytes()
        return data + (bytes(-nb % 32) if last else b'')

    from concurrent.futures import ThreadPoolExecutor
    workers = max(1, min(16, os.cpu_count() or 1))
    with open(path, 'wb') as f, ThreadPoolExecutor(workers) as pool:
        f.write(head)
        pending = []
        for job in jobs:
            pending.append((job, pool.submit(draw, job)))
            if len(pending) > 2 * workers:             # bounded memory: at most ~2 chunks per worker in flight
                done, fut = pending.pop(0)
                f.write(fut.result())
                report(done, progress, len(ts))
        for done, fut in pending:
            f.write(fut.result())
            report(done, progress, len(ts))


def report(job, progress, nt):
    idx, j = job[0], job[1]
    if idx % 40 == 0 and j == 0:
        msg = f'e2e: writing tensor {idx} of {nt}'
        if progress:
            progress(msg)
        else:
            print(msg, file=sys.stderr, flush=True)


def e2e(args):
    """the 4B-architecture model converted by det convert, prefill 512 ids, greedy decode 128."""
    import tempfile
    from det_amd import gguf, model
    cfg = dict(QWEN35_4B)
    L = ffi.lib()
    assert L.det_init() == 0
    tmp = tempfile.mkdtemp(prefix='det_e2e_')
    src, dst = os.path.join(tmp, 'q35-4b-BF16.gguf'), os.path.join(tmp, 'q35-4b-det-w6.gguf')
    t0 = time.time()
    write_qwen35_bf16(src, cfg, seed=5)
    t1 = time.time()
    print(f'e2e: bf16 source written ({os.path.getsize(src) / 1e9:.2f} GB, {t1 - t0:.1f} s)', file=sys.stderr, flush=True)
    gguf.convert(src, dst, None, cfg['ctx'])
    os.remove(src)
    t2 = time.time()
    print(f'e2e: det convert done ({os.path.getsize(dst) / 1e9:.2f} GB, {t2 - t1:.1f} s)', file=sys.stderr, flush=True)
    m = model.Model(dst, cfg['ctx'], 512)
    t3 = time.time()
    print(f'e2e: model loaded ({t3 - t2:.1f} s)', file=sys.stderr, flush=True)
    prompt = np.random.default_rng(11).integers(0, cfg['vocab'], 512).tolist()
    m.prefill(prompt)                              # warm-up pass (code objects, caches), then the measured one
    m.generate([], 4)
    m.reset()
    L.det_sync()
    a = time.perf_counter()
    m.prefill(prompt)
    L.det_sync()
    b = time.perf_counter()
    toks = m.generate([], args.decode)
    L.det_sync()
    c = time.perf_counter()
    os.remove(dst)
    os.rmdir(tmp)
    out = {'metric': 'end-to-end qwen35 4B-architecture: prefill and greedy decode tokens/s, 1 MI355X',
           'prefill_tok_s': round(512 / (b - a), 1), 'decode_tok_s': round(len(toks) / (c - b), 2),
           'prefill_ms': round((b - a) * 1e3, 2), 'decode_ms_per_token': round((c - b) * 1e3 / max(len(toks), 1), 3),
           'tokens': toks[:8], 'n_decoded': len(toks), 'unit': 'tokens/s', 'higher_is_better': True,
           'data': 'synthetic (random-init weights, seed 5; prompt of 512 uniform ids, seed 11)',
           'config': {'workload': 'BASELINE configs[4]', **cfg,
                      'bits': '6,output=8,ssm_alpha=8,ssm_beta=8 (det convert default, --no-calibrate)',
                      'max_batch': 512},
           'setup_s': {'write_bf16': round(t1 - t0, 1), 'convert': round(t2 - t1, 1), 'load': round(t3 - t2, 1)}}
    print(json.dumps(out), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument('--gpus', type=int, default=1)
    ap.add_argument('--steps', type=int, default=200)
    ap.add_argument('--warmup', type=int, default=20)
    ap.add_argument('--no-cpu', action='store_true')
    ap.add_argument('--only-main', action='store_true')
    ap.add_argument('--copy-calibration', action='store_true',
                    help='only run a plain device-to-device copy of 1 GiB, 10 times (scales FETCH_SIZE/WRITE_SIZE)')
    ap.add_argument('--e2e', action='store_true',
                    help='BASELINE configs[4] instead: the 4B-architecture model end to end (prefill / decode tokens/s)')
    ap.add_argument('--decode', type=int, default=128, help='tokens decoded by --e2e')
    args = ap.parse_args()
    if args.e2e:
        e2e(args)
        return
    if args.copy_calibration:
        L = ffi.lib()
        a, b = ffi.Buf(1 << 30, np.uint8), ffi.Buf(1 << 30, np.uint8)
        for _ in range(10):
            L.det_memcpy(b.ptr, a.ptr, 1 << 30, None)
        L.det_sync()
        print(json.dumps({'copy_bytes_per_launch': 1 << 30, 'launches': 10}))
        return
    if args.gpus != 1 or int(os.environ.get('WORLD_SIZE', '1')) != 1:
        print('bench.py: this build measures one GPU only (the path shards along N with an all-gather of y; '
              'no multi-GPU figure is produced)', file=sys.stderr)
        sys.exit(2)

    L = ffi.lib()
    assert L.det_init() == 0
    device = L.det_device_name().decode()
    ev = HipEvents()
    K, N6, NH = 2560, 9728, 248320

    lin6, rows6 = make_linear_copies(N6, K, 6, 1, ROTATE_BYTES)
    rows_head = None
    xq, sx, mx = make_acts(512, K, 2)
    y = ffi.Buf((512, NH), np.float32)
    ms, wall = time_gemm(ev, lin6, xq, sx, mx, 512, y, args.steps, args.warmup)
    main_line = shape_line('w6_9728x2560', N6, K, 512, 6, ms)

    shapes = [main_line]
    if not args.only_main:
        for M in (1, 64):
            xq_m, sx_m, mx_m = make_acts(M, K, 3 + M)
            msm, _ = time_gemm(ev, lin6, xq_m, sx_m, mx_m, M, y, max(args.steps, 200), args.warmup)
            shapes.append(shape_line('w6_9728x2560', N6, K, M, 6, msm))
        for l in lin6:
            for b in (l.wq, l.c, l.m):
                b.free()
        linh, rows_head = make_linear_copies(NH, K, 8, 4, ROTATE_BYTES)
        for M in (1, 512):
            xq_m, sx_m, mx_m = make_acts(M, K, 5 + M)
            msm, _ = time_gemm(ev, linh, xq_m, sx_m, mx_m, M, y, max(10, args.steps // 10), max(2, args.warmup // 10))
            shapes.append(shape_line('w8_head_248320x2560', NH, K, M, 8, msm))

    tops = main_line['TOPS']
    out = {
        'metric': 'W6xint8 GEMM: decode HBM GB/s, prefill int8 TOPS (% roofline), 1 MI355X',
        'value': tops, 'unit': 'TOPS', 'n_gpus': 1, 'steps': args.steps, 'warmup': args.warmup,
        'ms_per_step': round(ms, 6), 'higher_is_better': True, 'scaling': 'weak', 'vs_baseline': None,
        'dtype': 'int8xint6->int32/int64, fp32 epilogue', 'data': 'synthetic (seeded Gaussian weights/activations)',
        'config': {'workload': 'BASELINE configs[1]: W6 prefill GEMM K=2560 N=9728 M=512 (det_gemm_ex Write)',
                   'M': 512, 'N': N6, 'K': K, 'bits': 6, 'device': device},
        'roofline': {'bound': 'mfma', 'achieved': tops, 'peak': INT8_PEAK_TOPS, 'unit': 'TFLOP/s',
                     'frac': round(tops / INT8_PEAK_TOPS, 4),
                     'traffic': committed_traffic(PREFILL_KERNEL, PREFILL_GRID),
                     'traffic_source': 'profiles/gemm_hbm_traffic.md (FETCH_SIZE x2 + WRITE_SIZE x1 per launch)',
                     'algorithmic_bytes_per_launch': algo_bytes(N6, K, 512, 6),
                     'kernel': PREFILL_KERNEL, 'algorithmic_ops_per_launch': 2 * 512 * N6 * K},
        'shapes': shapes,
        'timed_wall_s': round(wall, 4),
    }
    dec = [s for s in shapes if s['M'] == 1]
    if dec:
        out['decode'] = {}
        for s_ in dec:
            wbytes = s_['N'] * row_bytes(s_['bits'], s_['K'])
            fus, fgbs, fgrid = read_floor(ev, wbytes)
            out['decode'][s_['shape']] = {
                'GBps': s_['GBps'], 'frac_of_hbm_peak': s_['frac_of_bound'], 'us': s_['us'],
                'read_floor_us': round(fus, 3), 'read_floor_GBps': round(fgbs, 1), 'read_floor_grid': fgrid,
                'frac_of_read_floor': round(fus / s_['us'], 4)}
    if not args.no_cpu:
        if rows_head is None:
            rows_head = np.zeros((NH, row_bytes(8, K)), np.uint8)
        out['cpu_baseline'] = cpu_baseline(rows6, rows_head)
    print(json.dumps(out), flush=True)


if __name__ == '__main__':
    main()
