"""The stream-K prefill kernel (k_prefill, selected by DET_PREFILL=streamk) against the oracle, bit for bit, on
the GPU: the reference suite's M > 64 cases, the BASELINE W6 9728 x 2560 shape at M = 65, 100, 512, a W8 and a W4
shape with split tiles, Accumulate and fused Parts outputs, and mx = NULL.  The kernel has not run on a GPU yet,
so this module is skipped unless DET_TEST_STREAMK=1: it runs in a child process with DET_PREFILL=streamk."""
import os
import subprocess
import sys
import textwrap

import pytest

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(os.environ.get('DET_TEST_STREAMK') != '1',
                                 reason='stream-K prefill kernel not yet run on a GPU (opt-in: DET_TEST_STREAMK=1)')]
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))

BODY = textwrap.dedent('''
    import sys
    sys.path.insert(0, ROOT)
    import numpy as np, oracle
    from det_amd import ffi
    from tests.helpers import same_f32
    fails = []
    def run(name, rows, N, K, bits, M, seed, widths=None, acc=False, use_mx=True):
        rng = oracle.Rng(seed)
        xq, sx, mx = oracle.quant(rng.acts_x(M, K))
        if not use_mx:
            mx = None
        lin = ffi.Linear(rows, K, bits, widths=widths)
        xb, sb = ffi.Buf.upload(xq), ffi.Buf.upload(sx)
        mb = ffi.Buf.upload(mx) if mx is not None else None
        print(name, 'W%d N=%d K=%d M=%d' % (bits, N, K, M), flush=True)
        if widths:
            outs = [ffi.Buf((M, w), np.float32) for w in widths]
            ffi.gemm(lin, xb, sb, mb, M, parts=outs)
            want = oracle.gemm(rows, N, K, bits, xq, sx, mx, widths=widths)
            for p, (o, w) in enumerate(zip(outs, want)):
                d = same_f32(w, o.download())
                if d: fails.append('%s part %d: %s' % (name, p, d))
            return
        y0 = np.asarray(rng.acts_x(M, N), np.float32) if acc else np.zeros((M, N), np.float32)
        y = ffi.Buf.upload(y0)
        if acc:
            ffi.gemm(lin, xb, sb, mb, M, accumulate=y)
        else:
            ffi.gemm(lin, xb, sb, mb, M, write=y)
        want = oracle.gemm(rows, N, K, bits, xq, sx, mx, y=y0 if acc else None, accumulate=acc)
        d = same_f32(want, y.download())
        if d: fails.append('%s: %s' % (name, d))
    rng = oracle.Rng(11)
    for bits in (8, 6, 4):
        rows = rng.fake_rows(bits, 640, 2560)
        for M in (65, 100, 300):
            run('conformance', rows, 640, 2560, bits, M, 100 + M)
        run('accumulate', rows, 640, 2560, bits, 100, 7, acc=True)
        run('no mx', rows, 640, 2560, bits, 130, 8, use_mx=False)
        r2 = rng.fake_rows(bits, 200, 5120)
        run('split tiles', r2, 200, 5120, bits, 200, 9)
    rows = rng.fake_rows(6, 9728, 2560)
    for M in (65, 100, 512):
        run('baseline', rows, 9728, 2560, 6, M, 200 + M)
    r3 = rng.fake_rows(4, 300, 1024)
    run('parts', r3, 300, 1024, 4, 150, 12, widths=[100, 36, 164])
    print('FAILS', len(fails))
    for f in fails:
        print(f)
    sys.exit(1 if fails else 0)
''')


def test_streamk_prefill_parity():
    env = dict(os.environ, DET_PREFILL='streamk')
    r = subprocess.run([sys.executable, '-u', '-c', f'ROOT = {ROOT!r}\n' + BODY], env=env, capture_output=True,
                       text=True, timeout=900)
    print(r.stdout[-4000:], r.stderr[-4000:])
    assert r.returncode == 0, r.stdout[-4000:] + r.stderr[-4000:]
