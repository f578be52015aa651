"""GGUF container and `det convert` over det_gguf.h (ctypes).

    python -m det_amd.gguf convert <float.gguf> [--out det.gguf] [--bits 6,ffn_down=8,...] [--rope-positions N]
    python -m det_amd.gguf info <model.gguf>

`convert` is the reference's `det convert --no-calibrate` (crates/det-cli/src/main.rs:517-524, convert.rs): the
linears are quantized on the GPU.  The calibration pass (`det calibrate`) needs the model forward, which this
build does not have.
"""
import ctypes
import os
import sys

import numpy as np

from . import ffi

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARRAY, U64, I64, F64 = range(13)
TYPE_F32, TYPE_F16, TYPE_BF16, TYPE_DET4, TYPE_DET6, TYPE_DET8 = 0, 1, 30, 0xDE04, 0xDE06, 0xDE08
DEFAULT_BITS = '6,output=8,ssm_alpha=8,ssm_beta=8'

_bound = False


def _lib():
    global _bound
    L = ffi.lib()
    if not _bound:
        P, c = ctypes.c_void_p, ctypes
        sig = {
            'det_gguf_last_error': (c.c_char_p, []),
            'det_gguf_open': (P, [c.c_char_p]),
            'det_gguf_close': (None, [P]),
            'det_gguf_data_start': (c.c_uint64, [P]),
            'det_gguf_alignment': (c.c_uint64, [P]),
            'det_gguf_n_kv': (c.c_uint64, [P]),
            'det_gguf_kv_key': (c.c_char_p, [P, c.c_uint64]),
            'det_gguf_kv_type': (c.c_uint32, [P, c.c_uint64]),
            'det_gguf_find_kv': (c.c_int64, [P, c.c_char_p]),
            'det_gguf_get_u64': (c.c_int, [P, c.c_char_p, c.POINTER(c.c_uint64)]),
            'det_gguf_get_f32': (c.c_int, [P, c.c_char_p, c.POINTER(c.c_float)]),
            'det_gguf_get_str': (c.c_char_p, [P, c.c_char_p]),
            'det_gguf_get_array': (c.c_int, [P, c.c_char_p, c.POINTER(c.c_uint32), c.POINTER(c.c_uint64)]),
            'det_gguf_array_u64': (c.c_int, [P, c.c_char_p, c.c_uint64, c.POINTER(c.c_uint64)]),
            'det_gguf_array_f64': (c.c_int, [P, c.c_char_p, c.c_uint64, c.POINTER(c.c_double)]),
            'det_gguf_array_str': (c.c_char_p, [P, c.c_char_p, c.c_uint64]),
            'det_gguf_n_tensors': (c.c_uint64, [P]),
            'det_gguf_find_tensor': (c.c_int64, [P, c.c_char_p]),
            'det_gguf_tensor_name': (c.c_char_p, [P, c.c_uint64]),
            'det_gguf_tensor_type': (c.c_uint32, [P, c.c_uint64]),
            'det_gguf_tensor_dims': (c.c_int, [P, c.c_uint64, c.POINTER(c.c_uint64)]),
            'det_gguf_tensor_offset': (c.c_uint64, [P, c.c_uint64]),
            'det_gguf_tensor_bytes': (c.c_uint64, [P, c.c_uint64]),
            'det_gguf_tensor_data': (P, [P, c.c_uint64]),
            'det_convert': (c.c_int, [c.c_char_p, c.c_char_p, c.c_char_p, c.c_int64]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype, f.argtypes = res, args
        _bound = True
    return L


class GgufError(RuntimeError):
    pass


def _err():
    return GgufError(_lib().det_gguf_last_error().decode())


class Tensor:
    def __init__(self, g, i):
        L = _lib()
        self.name = L.det_gguf_tensor_name(g.h, i).decode()
        self.type = L.det_gguf_tensor_type(g.h, i)
        dims = (ctypes.c_uint64 * 4)()
        n = L.det_gguf_tensor_dims(g.h, i, dims)
        self.dims = [int(dims[j]) for j in range(n)]
        self.offset = L.det_gguf_tensor_offset(g.h, i)
        self.nbytes = L.det_gguf_tensor_bytes(g.h, i)
        self._ptr = L.det_gguf_tensor_data(g.h, i)
        self._g = g

    def bytes(self):
        """The tensor's stored bytes (a copy)."""
        return np.ctypeslib.as_array((ctypes.c_uint8 * self.nbytes).from_address(self._ptr)).copy()


class Gguf:
    """Gguf::open (crates/det/src/gguf.rs:208-300) over the library's reader."""

    def __init__(self, path):
        self.h = _lib().det_gguf_open(os.fsencode(path))
        if not self.h:
            raise _err()
        L = _lib()
        self.data_start = L.det_gguf_data_start(self.h)
        self.alignment = L.det_gguf_alignment(self.h)
        self.keys = [L.det_gguf_kv_key(self.h, i).decode() for i in range(L.det_gguf_n_kv(self.h))]
        self.tensors = [Tensor(self, i) for i in range(L.det_gguf_n_tensors(self.h))]

    def close(self):
        if self.h:
            _lib().det_gguf_close(self.h)
            self.h = None

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def __del__(self):
        self.close()

    def kv_type(self, key):
        i = _lib().det_gguf_find_kv(self.h, key.encode())
        return None if i < 0 else _lib().det_gguf_kv_type(self.h, i)

    def u64(self, key):
        v = ctypes.c_uint64()
        return v.value if _lib().det_gguf_get_u64(self.h, key.encode(), ctypes.byref(v)) else None

    def f32(self, key):
        v = ctypes.c_float()
        return v.value if _lib().det_gguf_get_f32(self.h, key.encode(), ctypes.byref(v)) else None

    def str(self, key):
        s = _lib().det_gguf_get_str(self.h, key.encode())
        return None if s is None else s.decode()

    def array(self, key):
        """(element type, [values]) with numbers as u64 / f64 where they convert, strings as str."""
        L = _lib()
        et, n = ctypes.c_uint32(), ctypes.c_uint64()
        if not L.det_gguf_get_array(self.h, key.encode(), ctypes.byref(et), ctypes.byref(n)):
            return None
        out = []
        for j in range(n.value):
            if et.value == STR:
                out.append(L.det_gguf_array_str(self.h, key.encode(), j).decode())
            elif et.value in (F32, F64):
                d = ctypes.c_double()
                L.det_gguf_array_f64(self.h, key.encode(), j, ctypes.byref(d))
                out.append(d.value)
            else:
                u = ctypes.c_uint64()
                out.append(u.value if L.det_gguf_array_u64(self.h, key.encode(), j, ctypes.byref(u)) else None)
        return et.value, out

    def tensor(self, name):
        i = _lib().det_gguf_find_tensor(self.h, name.encode())
        return None if i < 0 else self.tensors[i]


def convert(src, dst, bits=None, rope_positions=0):
    """det convert --no-calibrate (convert.rs:170-402), linears quantized on the GPU."""
    rc = _lib().det_convert(os.fsencode(src), os.fsencode(dst), None if bits is None else bits.encode(), int(rope_positions))
    if rc != 0:
        raise _err()


def main(argv):
    if len(argv) >= 2 and argv[0] == 'convert':
        src, out, bits, rope = argv[1], None, None, 0
        i = 2
        while i < len(argv):
            if argv[i] == '--out':
                out = argv[i + 1]; i += 2
            elif argv[i] == '--bits':
                bits = argv[i + 1]; i += 2
            elif argv[i] == '--rope-positions':
                rope = int(argv[i + 1]); i += 2
            else:
                raise SystemExit(f'unknown option {argv[i]}')
        if out is None:
            # default_output (convert.rs:404-413): <stem minus its float suffix>-det-w<default bits>.gguf
            stem = os.path.splitext(os.path.basename(src))[0]
            for suf in ('-00001-of-00002', '-BF16', '-bf16', '-F16', '-f16'):
                while stem.endswith(suf):
                    stem = stem[:-len(suf)]
            default = '6'
            for item in (bits or DEFAULT_BITS).split(','):     # the last plain width is the default (Bits::parse)
                if item.strip() and '=' not in item:
                    default = item.strip()
            out = os.path.join(os.path.dirname(src), f'{stem}-det-w{default}.gguf')
        convert(src, out, bits, rope)
        return 0
    if len(argv) == 2 and argv[0] == 'info':
        with Gguf(argv[1]) as g:
            print(f'{len(g.keys)} metadata keys, {len(g.tensors)} tensors, data at {g.data_start}')
            for t in g.tensors:
                print(f'  {t.name}: type {t.type:#x} dims {t.dims} {t.nbytes} bytes at {t.offset}')
        return 0
    print(__doc__)
    return 2


if __name__ == '__main__':
    sys.exit(main(sys.argv[1:]))
