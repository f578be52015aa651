"""The library's GGUF reader (det_gguf.h, replacing crates/det/src/gguf.rs) on files written by the test-side
writer: every metadata value type, arrays, the alignment key, every tensor type det accepts, and the reference's
error cases (gguf.rs:208-300).  CPU only: the reader is host code."""
import struct

import numpy as np
import pytest

import oracle
from det_amd import gguf
from tests import gguf_ref as R


def sample_file(path, alignment=64):
    kv = [('general.architecture', R.STR, 'qwen35'), ('a.u8', R.U8, 200), ('a.i8', R.I8, -5), ('a.u16', R.U16, 65000),
          ('a.i16', R.I16, 1234), ('a.u32', R.U32, 4000000000), ('a.i32', R.I32, -7), ('a.i32p', R.I32, 77),
          ('a.f32', R.F32, 0.1), ('a.bool', R.BOOL, True), ('a.u64', R.U64, 1 << 40), ('a.i64', R.I64, -(1 << 40)),
          ('a.f64', R.F64, 2.5), ('a.strs', R.ARRAY, (R.STR, ['x', 'yz', ''])), ('a.u32s', R.ARRAY, (R.U32, [1, 2, 3])),
          ('a.f32s', R.ARRAY, (R.F32, [0.5, -1.25])), ('a.empty', R.ARRAY, (R.U8, [])),
          ('general.alignment', R.U32, alignment), ('a.dup', R.U32, 1), ('a.dup', R.U32, 2)]
    rng = np.random.default_rng(3)
    rows = oracle.Rng(5).fake_rows(6, 5, 256)
    f = rng.standard_normal(256).astype(np.float32)
    h = rng.standard_normal((3, 64)).astype(np.float16).astype(np.float32)
    b = (rng.standard_normal((2, 32)).astype(np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)
    tensors = [('v.f32', [256], R.T_F32, f.tobytes()), ('m.f16', [64, 3], R.T_F16, R.to_bytes(h, R.T_F16)),
               ('m.bf16', [32, 2], R.T_BF16, R.to_bytes(b, R.T_BF16)), ('lin.w6', [256, 5], R.DET[6], rows.tobytes())]
    R.write_gguf(path, kv, tensors, alignment)
    return kv, tensors


def test_reader_roundtrip(tmp_path):
    p = tmp_path / 'm.gguf'
    kv, tensors = sample_file(p)
    with gguf.Gguf(p) as g:
        assert g.keys == [k for k, _, _ in kv]
        assert g.alignment == 64 and g.data_start % 64 == 0
        assert g.str('general.architecture') == 'qwen35'
        assert g.u64('a.u8') == 200 and g.u64('a.u16') == 65000 and g.u64('a.u32') == 4000000000
        assert g.u64('a.u64') == 1 << 40 and g.u64('a.i32p') == 77
        assert g.u64('a.i8') is None and g.u64('a.i32') is None and g.u64('a.i64') is None   # negative: no u64
        assert g.u64('a.bool') is None and g.u64('a.f32') is None
        assert g.f32('a.f32') == np.float32(0.1) and g.f32('a.f64') == 2.5 and g.f32('a.u32') == np.float32(4e9)
        assert g.kv_type('a.bool') == R.BOOL and g.kv_type('a.strs') == R.ARRAY
        assert g.array('a.strs') == (R.STR, ['x', 'yz', ''])
        assert g.array('a.u32s') == (R.U32, [1, 2, 3])
        assert g.array('a.f32s') == (R.F32, [0.5, -1.25])
        assert g.array('a.empty') == (R.U8, [])
        assert g.u64('a.dup') == 2                              # the last of equal keys (gguf.rs:244-248)
        assert g.str('missing') is None and g.array('a.u8') is None
        assert [t.name for t in g.tensors] == [t[0] for t in tensors]
        off = 0
        for t, (name, dims, ty, data) in zip(g.tensors, tensors):
            assert (t.dims, t.type, t.offset, t.nbytes) == (dims, ty, off, len(data))
            assert t.bytes().tobytes() == data
            off += len(data) + (-len(data) % 64)
        assert g.tensor('lin.w6').type == 0xDE06 and g.tensor('nope') is None


def corrupt(tmp_path, name, mutate):
    p = tmp_path / 'base.gguf'
    sample_file(p, alignment=32)
    b = bytearray(p.read_bytes())
    q = tmp_path / name
    q.write_bytes(mutate(b))
    return q


@pytest.mark.parametrize('name,mutate,msg', [
    ('magic', lambda b: b'GGUX' + b[4:], 'not a GGUF file'),
    ('version', lambda b: b[:4] + struct.pack('<I', 4) + b[8:], 'unsupported GGUF version 4'),
    ('truncated', lambda b: b[:40], 'truncated GGUF header'),
    ('empty', lambda b: b'', 'truncated GGUF header'),
    ('tail', lambda b: b[:-100], 'does not fit the file'),
])
def test_reader_errors(tmp_path, name, mutate, msg):
    with pytest.raises(gguf.GgufError, match=msg):
        gguf.Gguf(corrupt(tmp_path, name, mutate))


def test_reader_bad_tensors(tmp_path):
    for dims, ty, nbytes, msg in (([64], 2, 64, 'unsupported type Q4_0'), ([48, 1], R.DET[6], 64, 'unsupported type DET_W6'),
                                  ([32, 2, 2], R.T_F32, 512, 'does not fit the file')):
        p = tmp_path / 'bad.gguf'
        R.write_gguf(p, [('k', R.U32, 1)], [('t', dims, ty, bytes(nbytes))])
        with pytest.raises(gguf.GgufError, match=msg):
            gguf.Gguf(p)
    p = tmp_path / 'badval.gguf'
    p.write_bytes(b'GGUF' + struct.pack('<IQQ', 3, 0, 1) + struct.pack('<Q', 1) + b'k' + struct.pack('<I', 13) + bytes(8))
    with pytest.raises(gguf.GgufError, match='unknown GGUF value type 13'):
        gguf.Gguf(p)
