"""ctypes bindings of include/det_hip.h, plus a small host-side mirror of det's Backend operations
(reference crates/det/src/backend.rs:203-265: linear / quant / gemm with GemmOut::{Write, Accumulate, Parts} /
rmsnorm_quant / silu_mul_quant, and Buf ownership through det_malloc / det_free) used by tests and bench.py.

Fails loudly when the HIP library is missing: there is no CPU path here.
"""
import ctypes
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, 'libdet_hip.so')
HEADER = os.path.join(os.path.dirname(HERE), 'include', 'det_hip.h')

_lib = None


class QLinear(ctypes.Structure):
    """det_qlinear (det_hip.h; det_cuda.h:27-32)."""
    _fields_ = [('wq', ctypes.c_void_p), ('c', ctypes.c_void_p), ('m', ctypes.c_void_p),
                ('N', ctypes.c_int), ('K', ctypes.c_int), ('bits', ctypes.c_int)]


class AttnLayer(ctypes.Structure):
    """det_attn_layer (det_hip.h; det_cuda.h:60-65)."""
    _fields_ = [('q_norm', ctypes.c_void_p), ('k_norm', ctypes.c_void_p), ('v_scale', ctypes.c_void_p),
                ('v_inv_scale', ctypes.c_void_p)]


class KvCache(ctypes.Structure):
    """det_kv_cache (det_hip.h; det_cuda.h:66-67)."""
    _fields_ = [('kq', ctypes.c_void_p), ('sk', ctypes.c_void_p), ('vq', ctypes.c_void_p), ('capacity', ctypes.c_int),
                ('vlo', ctypes.c_void_p), ('vhi', ctypes.c_void_p)]


class GdnLayer(ctypes.Structure):
    """det_gdn_layer (det_hip.h; det_cuda.h:85-90)."""
    _fields_ = [('conv', ctypes.c_void_p), ('A', ctypes.c_void_p), ('dt_bias', ctypes.c_void_p),
                ('norm', ctypes.c_void_p)]


class GdnState(ctypes.Structure):
    """det_gdn_state (det_hip.h; det_cuda.h:91)."""
    _fields_ = [('conv_state', ctypes.c_void_p), ('S', ctypes.c_void_p)]


def header_symbols():
    """Function names declared in include/det_hip.h."""
    text = open(HEADER).read()
    text = re.sub(r'//.*', '', text)
    return sorted(set(re.findall(r'\b(det_[a-z0-9_]+)\s*\(', text)))


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f'{LIB_PATH} is missing: build it with `python -m det_amd.build` (no CPU fallback exists)')
    L = ctypes.CDLL(LIB_PATH)
    P, i, f, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    szp = ctypes.POINTER(ctypes.c_size_t)
    sig = {
        'det_init': (i, []), 'det_device_name': (ctypes.c_char_p, []), 'det_malloc': (P, [sz]),
        'det_free': (None, [P]), 'det_allocated_bytes': (sz, []), 'det_sync': (None, []), 'det_flush': (None, []),
        'det_memset': (None, [P, i, sz, P]), 'det_memcpy': (None, [P, P, sz, P]), 'det_hip_stream': (P, []),
        'det_linear_sizes': (None, [i, i, i, szp, szp, szp]),
        'det_linear_repack': (None, [P, i, i, i, P, P, P, P]),
        'det_quantize_rows': (None, [P, i, i, i, P, P]),
        'det_quant': (None, [P, i, i, P, P, P, P]),
        'det_rmsnorm_quant': (None, [P, P, f, i, i, P, P, P, P, P]),
        'det_silu_mul_quant': (None, [P, P, i, i, P, P, P, P, P]),
        'det_gemm': (None, [ctypes.POINTER(QLinear), P, P, P, i, P, P]),
        'det_gemm_ex': (None, [ctypes.POINTER(QLinear), P, P, P, i, P, i, i, P, P, P]),
        'det_gemm_scratch_bytes': (sz, [i, i]), 'det_gemm_set_scratch': (None, [P, sz]),
        'det_test_prim': (None, [i, P, i, i, P, P]),
        'det_test_gemv_silu0': (None, [ctypes.POINTER(QLinear), P, P, P, i, P, P, P]),
        'det_test_mul_quant': (None, [P, P, i, i, P, P, P, P]),
        'det_test_read': (None, [P, sz, i, P, P]),
        'det_attention': (None, [ctypes.POINTER(AttnLayer), ctypes.POINTER(KvCache), P, P, P, P, P, i, f, i, i, i, i,
                                 i, P, P, P]),
        'det_attn_scratch_bytes': (sz, [i, i, i]),
        'det_gdn': (None, [ctypes.POINTER(GdnLayer), ctypes.POINTER(GdnState), P, P, P, P, f, i, i, i, i, i, P, P, P]),
        'det_gdn_scratch_bytes': (sz, [i, i, i, i, i]),
        'det_argmax': (None, [P, i, i, P, P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _lib = L
    return L


def linear_sizes(N, K, bits):
    a, b, c = ctypes.c_size_t(), ctypes.c_size_t(), ctypes.c_size_t()
    lib().det_linear_sizes(N, K, bits, ctypes.byref(a), ctypes.byref(b), ctypes.byref(c))
    return a.value, b.value, c.value


# ---------------------------------------------------------------- device buffers (Buf<T>, backend.rs:13-134)
class Buf:
    """A det_malloc'd device array (zero-initialised) that frees itself with det_free."""

    def __init__(self, shape, dtype):
        self.shape = tuple(shape) if isinstance(shape, (tuple, list)) else (int(shape),)
        self.dtype = np.dtype(dtype)
        self.nbytes = int(np.prod(self.shape)) * self.dtype.itemsize
        self.ptr = lib().det_malloc(max(self.nbytes, 16))
        if not self.ptr:
            raise MemoryError(f'det_malloc({self.nbytes}) failed')

    @classmethod
    def upload(cls, arr):
        arr = np.ascontiguousarray(arr)
        b = cls(arr.shape, arr.dtype)
        lib().det_memcpy(b.ptr, arr.ctypes.data, arr.nbytes, None)
        return b

    def write(self, arr):
        arr = np.ascontiguousarray(arr, dtype=self.dtype)
        assert arr.nbytes <= self.nbytes
        lib().det_memcpy(self.ptr, arr.ctypes.data, arr.nbytes, None)

    def download(self):
        out = np.empty(self.shape, self.dtype)
        lib().det_memcpy(out.ctypes.data, self.ptr, self.nbytes, None)
        lib().det_sync()
        return out

    def free(self):
        if self.ptr:
            lib().det_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def ptr(b):
    return None if b is None else b.ptr


# ---------------------------------------------------------------- Backend mirror
class Linear:
    """Backend::linear (backend.rs:229-231): det rows (one or more tensors fused along N, all of one K and width)
    uploaded and repacked on the device into the tiled layout of det_hip.h."""

    def __init__(self, rows, K, bits, widths=None, rows_on_device=None):
        if rows_on_device is None:
            rows = np.ascontiguousarray(rows, dtype=np.uint8)
            N = rows.shape[0]
            dev_rows = Buf.upload(rows)
        else:
            dev_rows, N = rows_on_device
        self.N, self.K, self.bits = N, K, bits
        self.widths = list(widths) if widths is not None else [N]
        assert sum(self.widths) == N
        wb, cb, mb = linear_sizes(N, K, bits)
        self.wq, self.c, self.m = Buf(wb, np.uint8), Buf(cb // 4, np.float32), Buf(mb // 2, np.uint16)
        lib().det_linear_repack(dev_rows.ptr, N, K, bits, self.wq.ptr, self.c.ptr, self.m.ptr, None)
        if rows_on_device is None:
            lib().det_sync()
            dev_rows.free()
        self.q = QLinear(self.wq.ptr, self.c.ptr, self.m.ptr, N, K, bits)


def quantize_rows(w_dev, N, K, bits):
    """det_quantize_rows on a device fp32 [N][K] buffer -> device det rows."""
    rb = K // 32 * {8: 32, 6: 24, 4: 16}[bits] + 4 + 2 * (K // 128)
    rows = Buf((N, rb), np.uint8)
    lib().det_quantize_rows(w_dev.ptr, N, K, bits, rows.ptr, None)
    return rows


def quant(x, M, n, xq, sx, mx):
    """Backend::quant (backend.rs:245): mx None selects per-row quant_act_i8."""
    lib().det_quant(x.ptr, M, n, xq.ptr, sx.ptr, ptr(mx), None)


def rmsnorm_quant(x, w, eps, M, n, xq, sx, mx, y=None):
    lib().det_rmsnorm_quant(x.ptr, w.ptr, eps, M, n, ptr(y), ptr(xq), ptr(sx), ptr(mx), None)


def silu_mul_quant(g, u, M, n, hq, sh, mh, h=None):
    lib().det_silu_mul_quant(g.ptr, u.ptr, M, n, ptr(h), ptr(hq), ptr(sh), ptr(mh), None)


def gemm(lin, xq, sx, mx, M, write=None, accumulate=None, parts=None):
    """Backend::gemm (backend.rs:246-254) with exactly one of GemmOut::Write / Accumulate / Parts."""
    if parts is not None:
        assert len(parts) == len(lin.widths)
        offs = (ctypes.c_int * len(parts))(*np.cumsum([0] + lin.widths[:-1]).tolist())
        dsts = (ctypes.c_void_p * len(parts))(*[p.ptr for p in parts])
        lib().det_gemm_ex(ctypes.byref(lin.q), xq.ptr, sx.ptr, ptr(mx), M, None, 0, len(parts),
                          ctypes.cast(offs, ctypes.c_void_p), ctypes.cast(dsts, ctypes.c_void_p), None)
    elif accumulate is not None:
        lib().det_gemm_ex(ctypes.byref(lin.q), xq.ptr, sx.ptr, ptr(mx), M, accumulate.ptr, 1, 0, None, None, None)
    else:
        lib().det_gemm_ex(ctypes.byref(lin.q), xq.ptr, sx.ptr, ptr(mx), M, write.ptr, 0, 0, None, None, None)


def test_prim(op, x, M, n):
    """det_test_prim on a host fp32 array -> host result (out has M entries for op 11, else M*n)."""
    xb = Buf.upload(np.ascontiguousarray(x, dtype=np.float32))
    out = Buf(M if op == 11 else M * n, np.float32)
    lib().det_test_prim(op, xb.ptr, M, n, out.ptr, None)
    return out.download()


def attention(layer, kv, qg, k, v, rope_cos, rope_sin, rot, eps, M, pos0, n_h, n_kv, hd, o):
    """Backend::attention (backend.rs; cpu.rs:212-285) over det_attention.  layer: AttnLayer, kv: KvCache."""
    scratch = Buf(lib().det_attn_scratch_bytes(M, n_h, hd), np.uint8)
    lib().det_attention(ctypes.byref(layer), ctypes.byref(kv), qg.ptr, k.ptr, v.ptr, rope_cos.ptr, rope_sin.ptr, rot,
                        eps, M, pos0, n_h, n_kv, hd, o.ptr, scratch.ptr, None)


def gdn(layer, state, qkv, z, a, b, eps, M, n_k, n_v, dk, dv, on, scratch):
    """Backend::gdn (backend.rs; cpu.rs:287-383) over det_gdn.  scratch: a Buf of det_gdn_scratch_bytes()."""
    lib().det_gdn(ctypes.byref(layer), ctypes.byref(state), qkv.ptr, z.ptr, a.ptr, b.ptr, eps, M, n_k, n_v, dk, dv,
                  on.ptr, scratch.ptr, None)


def gdn_scratch_bytes(M, n_k, n_v, dk, dv):
    return lib().det_gdn_scratch_bytes(M, n_k, n_v, dk, dv)


def argmax(logits, M, V, out):
    """Backend::argmax (backend.rs; spec/sample.rs:6-14) over det_argmax: out[m] = first index of the max."""
    lib().det_argmax(logits.ptr, M, V, out.ptr, None)
