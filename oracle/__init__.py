"""CPU oracle for det's quantized-linear path (TEST INFRASTRUCTURE ONLY).

`det_oracle.c` restates the reference's Rust (crates/det/src/spec, quantize.rs, cpu.rs) in scalar C;
`spec_np.py` restates docs/SPEC.md independently in numpy.  Only tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg may import this package; the product (det_amd) never does.
"""
import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, 'libdet_oracle.so')
SRC = os.path.join(HERE, 'det_oracle.c')
MIXER_SRC = os.path.join(HERE, 'mixer_oracle.c')

CFLAGS = ['-O2', '-fPIC', '-shared', '-ffp-contract=off', '-fno-fast-math', '-fopenmp', '-Wall']


X86_SRC = os.path.join(HERE, 'x86_gemm.c')


def build():
    """Compile the C restatement (gcc, default MXCSR: no -ffast-math, no FMA contraction) together with the
    restatement of det's x86 GEMM (x86_gemm.c, built once for AVX2 and once for AVX2 + AVX-VNNI)."""
    import tempfile
    with tempfile.TemporaryDirectory() as tmp:
        objs = []
        for vnni, isa in ((0, ['-mavx2']), (1, ['-mavx2', '-mavxvnni'])):
            o = os.path.join(tmp, f'x86_{vnni}.o')
            subprocess.check_call(['gcc', '-O3', '-fPIC', '-fopenmp', '-Wall', '-c', f'-DXVNNI={vnni}'] + isa +
                                  ['-o', o, X86_SRC])
            objs.append(o)
        subprocess.check_call(['gcc'] + CFLAGS + ['-o', LIB_PATH, SRC, MIXER_SRC] + objs + ['-lm'])


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        P = ctypes.c_void_p
        i, f, sz, u64p = ctypes.c_int, ctypes.c_float, ctypes.c_size_t, ctypes.POINTER(ctypes.c_uint64)
        sig = {
            'ora_fmax': (f, [f, f]), 'ora_rint': (f, [f]), 'ora_i64_to_f32': (f, [ctypes.c_int64]),
            'ora_exp_f': (f, [f]), 'ora_log_f': (f, [f]), 'ora_softplus_f': (f, [f]),
            'ora_sigmoid_f': (f, [f]), 'ora_silu_f': (f, [f]), 'ora_treesum': (f, [P, i]),
            'ora_quant_act_i8': (f, [P, i, P]), 'ora_quant_act_i8g': (f, [P, i, P, P]),
            'ora_quant': (None, [P, i, i, P, P, P]),
            'ora_rmsnorm_quant': (None, [P, P, f, i, i, P, P, P]),
            'ora_silu_mul_quant': (None, [P, P, i, i, P, P, P]),
            'ora_row_bytes': (sz, [i, i]), 'ora_unpack_row': (None, [P, i, i, P]),
            'ora_pack': (None, [P, i, i, P]),
            'ora_gemm_row': (f, [P, f, P, P, f, P, i]),
            'ora_gemm_acc': (ctypes.c_int64, [P, P, P, P, i]),
            'ora_gemm': (None, [P, i, i, i, P, P, P, i, P, i, i, P, P]),
            'ora_quantize_row': (None, [P, i, i, P]), 'ora_quantize_rows': (None, [P, i, i, i, P]),
            'ora_rng_next': (ctypes.c_uint64, [u64p]), 'ora_rng_unit': (f, [u64p]),
            'ora_rng_byte': (ctypes.c_uint8, [u64p]), 'ora_rng_below': (ctypes.c_uint64, [u64p, ctypes.c_uint64]),
            'ora_rng_denorm': (f, [u64p]), 'ora_rng_units': (None, [u64p, P, sz]),
            'ora_fake_rows': (None, [u64p, i, i, i, P]), 'ora_acts_x': (None, [u64p, i, i, P]),
            'ora_rmsnorm': (None, [P, P, f, i, P]),
            'ora_l2norm': (None, [P, f, i, P]), 'ora_rope': (None, [P, P, P, i]),
            'ora_quant_v': (None, [P, f, i, P]),
            'ora_attn_head': (None, [P, f, P, P, P, i, i, i, f, i, P]),
            'ora_attention': (None, [P, P, P, P, P, P, P, P, P, P, P, P, i, f, i, i, i, i, i, P]),
            'ora_gdn_conv': (f, [P, P]), 'ora_gdn_decay': (f, [f, f, f]),
            'ora_gdn_head_step': (None, [P, i, i, P, P, P, f, f, P]),
            'ora_gdn': (None, [P, P, P, P, P, P, P, P, P, P, f, i, i, i, i, i, P]),
            'ora_argmax': (i, [P, i]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def row_bytes(bits, k):
    return int(lib().ora_row_bytes(bits, k))


def quant(x, group=True):
    """Cpu::quant (cpu.rs:130-140): rows of x -> (xq, sx, mx); group=False is quant_act_i8 (mx None)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    M, n = x.shape
    xq = np.zeros((M, n), np.int8)
    sx = np.zeros(M, np.float32)
    mx = np.zeros((M, n // 128), np.uint16) if group else None
    lib().ora_quant(_p(x), M, n, _p(xq), _p(sx), _p(mx))
    return xq, sx, mx


def rmsnorm_quant(x, w, eps):
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    M, n = x.shape
    xq, sx, mx = np.zeros((M, n), np.int8), np.zeros(M, np.float32), np.zeros((M, n // 128), np.uint16)
    lib().ora_rmsnorm_quant(_p(x), _p(w), eps, M, n, _p(xq), _p(sx), _p(mx))
    return xq, sx, mx


def silu_mul_quant(g, u):
    g = np.ascontiguousarray(g, dtype=np.float32)
    u = np.ascontiguousarray(u, dtype=np.float32)
    M, n = g.shape
    xq, sx, mx = np.zeros((M, n), np.int8), np.zeros(M, np.float32), np.zeros((M, n // 128), np.uint16)
    lib().ora_silu_mul_quant(_p(g), _p(u), M, n, _p(xq), _p(sx), _p(mx))
    return xq, sx, mx


def unpack_row(packed, bits, k):
    packed = np.ascontiguousarray(packed, dtype=np.uint8)
    out = np.zeros(k, np.int8)
    lib().ora_unpack_row(_p(packed), bits, k, _p(out))
    return out


def pack(codes, bits):
    codes = np.ascontiguousarray(codes, dtype=np.int8)
    out = np.zeros(codes.size // 32 * {8: 32, 6: 24, 4: 16}[bits], np.uint8)
    lib().ora_pack(_p(codes), codes.size, bits, _p(out))
    return out


def gemm(rows, N, K, bits, xq, sx, mx, y=None, accumulate=False, widths=None):
    """Cpu::gemm (cpu.rs:142-185).  widths (fused parts) -> list of part outputs, else y [M][N]."""
    rows = np.ascontiguousarray(rows, dtype=np.uint8)
    xq = np.ascontiguousarray(xq, dtype=np.int8)
    sx = np.ascontiguousarray(sx, dtype=np.float32)
    mx = None if mx is None else np.ascontiguousarray(mx, dtype=np.uint16)
    M = xq.shape[0]
    if widths is not None and len(widths) > 1:
        outs = [np.zeros((M, w), np.float32) for w in widths]
        offs = np.cumsum([0] + list(widths[:-1])).astype(np.int32)
        ptrs = (ctypes.c_void_p * len(outs))(*[o.ctypes.data for o in outs])
        lib().ora_gemm(_p(rows), N, K, bits, _p(xq), _p(sx), _p(mx), M, None, 0, len(outs), _p(offs),
                       ctypes.cast(ptrs, ctypes.c_void_p))
        return outs
    if y is None:
        y = np.zeros((M, N), np.float32)
    else:
        y = np.ascontiguousarray(y, dtype=np.float32).copy()
    lib().ora_gemm(_p(rows), N, K, bits, _p(xq), _p(sx), _p(mx), M, _p(y), 1 if accumulate else 0, 0, None, None)
    return y


def quantize_rows(w, bits):
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    out = np.zeros((N, row_bytes(bits, K)), np.uint8)
    lib().ora_quantize_rows(_p(w), N, K, bits, _p(out))
    return out


class Rng:
    """The conformance xorshift64 (conformance.rs:35-59), state kept in C for bulk draws."""

    def __init__(self, seed):
        self.s = ctypes.c_uint64(seed)

    def _sp(self):
        return ctypes.byref(self.s)

    def next(self):
        return int(lib().ora_rng_next(self._sp()))

    def unit(self):
        return float(lib().ora_rng_unit(self._sp()))

    def byte(self):
        return int(lib().ora_rng_byte(self._sp()))

    def below(self, n):
        return int(lib().ora_rng_below(self._sp(), n))

    def denorm(self):
        return np.float32(lib().ora_rng_denorm(self._sp()))

    def units(self, n):
        out = np.zeros(n, np.float32)
        lib().ora_rng_units(self._sp(), _p(out), n)
        return out

    def fake_rows(self, bits, n, k):
        """conformance.rs:104-120 fake_gguf rows."""
        out = np.zeros((n, row_bytes(bits, k)), np.uint8)
        lib().ora_fake_rows(self._sp(), bits, n, k, _p(out))
        return out

    def acts_x(self, m, k):
        """conformance.rs:147-156 acts() before quantization."""
        out = np.zeros((m, k), np.float32)
        lib().ora_acts_x(self._sp(), m, k, _p(out))
        return out


class X86Linear:
    """det's x86 backend GEMM (crates/det/src/x86/gemm.rs) restated in C: the CPU baseline's timed path."""

    def __init__(self, rows, N, K, bits):
        L = lib()
        L.ora_x86_repack.restype = ctypes.c_void_p
        L.ora_x86_repack.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.ora_x86_gemm.argtypes = [ctypes.c_void_p] * 4 + [ctypes.c_int, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.ora_x86_free.argtypes = [ctypes.c_void_p]
        rows = np.ascontiguousarray(rows, dtype=np.uint8)
        self.N, self.K, self.bits = N, K, bits
        self.h = L.ora_x86_repack(_p(rows), N, K, bits)

    def gemm(self, xq, sx, mx, vnni=None, threads=0):
        if vnni is None:
            vnni = has_vnni()
        xq = np.ascontiguousarray(xq, dtype=np.int8)
        sx = np.ascontiguousarray(sx, dtype=np.float32)
        mx = None if mx is None else np.ascontiguousarray(mx, dtype=np.uint16)
        M = xq.shape[0]
        y = np.zeros((M, self.N), np.float32)
        lib().ora_x86_gemm(self.h, _p(xq), _p(sx), _p(mx), M, _p(y), int(vnni), threads)
        return y

    def __del__(self):
        if getattr(self, 'h', None):
            lib().ora_x86_free(self.h)
            self.h = None


def has_vnni():
    """AVX-VNNI (the VEX vpdpbusd det's x86 backend uses, x86/mod.rs:41-52) on this CPU."""
    return bool(lib().ora_x86_has_vnni())
