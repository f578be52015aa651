"""GGUF writer and a restatement of `det convert` in Python (TEST INFRASTRUCTURE).

`write_gguf` restates the container format (crates/det/src/gguf.rs:361-418: magic, version 3, metadata, tensor table,
padding to the alignment).  `convert_ref` restates convert.rs:170-402 and config.rs:32-93 step by step with the
oracle's quantizer (the C restatement of quantize.rs), libm cos/sin/pow through Python's math module for the
rotary tables, and this writer; the library's det_convert must reproduce its output byte for byte.
"""
import math
import struct

import numpy as np

import oracle

U8, I8, U16, I16, U32, I32, F32, BOOL, STR, ARRAY, U64, I64, F64 = range(13)
T_F32, T_F16, T_BF16 = 0, 1, 30
DET = {4: 0xDE04, 6: 0xDE06, 8: 0xDE08}
_FMT = {U8: '<B', I8: '<b', U16: '<H', I16: '<h', U32: '<I', I32: '<i', F32: '<f', BOOL: '<?', U64: '<Q', I64: '<q',
        F64: '<d'}


def _value(out, ty, v):
    if ty == STR:
        b = v.encode()
        out += struct.pack('<Q', len(b)) + b
    elif ty == ARRAY:
        et, items = v
        out += struct.pack('<IQ', et, len(items))
        for e in items:
            _value(out, et, e)
    elif ty == F32 and isinstance(v, (bytes, bytearray)):
        out += v                                            # exact bits
    else:
        out += struct.pack(_FMT[ty], v)


def header(kv, tensors, alignment=32):
    """kv: [(key, type, value)]; tensors: [(name, dims, type, offset)]."""
    out = bytearray(b'GGUF') + struct.pack('<IQQ', 3, len(tensors), len(kv))
    for k, ty, v in kv:
        kb = k.encode()
        out += struct.pack('<Q', len(kb)) + kb + struct.pack('<I', ty)
        _value(out, ty, v)
    for name, dims, ty, off in tensors:
        nb = name.encode()
        out += struct.pack('<Q', len(nb)) + nb + struct.pack('<I', len(dims))
        out += b''.join(struct.pack('<Q', d) for d in dims) + struct.pack('<IQ', ty, off)
    out += bytes(-len(out) % alignment)
    return bytes(out)


def write_gguf(path, kv, tensors, alignment=32):
    """tensors: [(name, dims, type, data bytes)] laid out in order, each padded to the alignment."""
    infos, blobs, off = [], [], 0
    for name, dims, ty, data in tensors:
        infos.append((name, dims, ty, off))
        blobs.append(data + bytes(-len(data) % alignment))
        off += len(blobs[-1])
    with open(path, 'wb') as f:
        f.write(header(kv, infos, alignment))
        for b in blobs:
            f.write(b)


def to_bytes(a, ty):
    a = np.ascontiguousarray(a, np.float32)
    if ty == T_F32:
        return a.tobytes()
    if ty == T_F16:
        return a.astype(np.float16).tobytes()
    return (a.view(np.uint32) >> 16).astype(np.uint16).tobytes()      # BF16 by truncation (values chosen exact)


def f32s(ty, data, n):
    """spec/tensor.rs:73-104 for the float types."""
    if ty == T_F32:
        return np.frombuffer(data, np.float32, n).copy()
    if ty == T_F16:
        return np.frombuffer(data, np.float16, n).astype(np.float32)
    return (np.frombuffer(data, np.uint16, n).astype(np.uint32) << 16).view(np.float32)


def head_perm(n_k, n_v, width, offset, total):
    """convert.rs:149-161."""
    rep = n_v // n_k
    p = list(range(total))
    for h2 in range(n_v):
        h = (h2 % rep) * n_k + h2 // rep
        for j in range(width):
            p[offset + h2 * width + j] = offset + h * width + j
    return p


def bits_of(spec, linear):
    default, per = 6, []
    for item in (x.strip() for x in spec.split(',')):
        if not item:
            continue
        if '=' in item:
            n, v = item.split('=', 1)
            per.append((n, int(v)))
        else:
            default = int(item)
    for n, v in per:
        if n == linear:
            return v
    return default


def convert_ref(model, bits='6,output=8,ssm_alpha=8,ssm_beta=8', rope_positions=None):
    """model: {'kv': [(key, type, value)], 'tensors': {name: (dims, type, data)}} as written to the source file.
    Returns the det GGUF bytes det convert writes."""
    kv = {k: v for k, _, v in model['kv']}
    T = model['tensors']
    arch = kv['general.architecture']
    a = lambda s: kv[f'{arch}.{s}']
    n_layers = a('block_count') - kv.get(f'{arch}.nextn_predict_layers', 0)
    interval = a('full_attention_interval')
    attention = [(i + 1) % interval == 0 for i in range(n_layers)]
    n_k, n_v, dk = a('ssm.group_count'), a('ssm.time_step_rank'), a('ssm.state_size')
    dv = a('ssm.inner_size') // n_v
    kd, conv_dim = n_k * dk, 2 * n_k * dk + n_v * dv
    rot, theta = a('rope.dimension_count'), float(np.float32(a('rope.freq_base')))
    n_pos = rope_positions or kv.get(f'{arch}.context_length', 32768)
    n_kv = a('attention.head_count_kv')

    def floats(name):
        dims, ty, data = T[name]
        return f32s(ty, data, int(np.prod(dims)))

    plan = []                                              # (name, dims, type, bytes)
    copy = lambda name: plan.append((name, T[name][0], T[name][1], T[name][2]))

    def quant(name, src=None, rows=None, cols=None):
        src = src or name
        k, n = T[src][0][0], T[src][0][1]
        w = floats(src).reshape(n, k)
        if rows is not None:
            w = w[rows]
        if cols is not None:
            w = w[:, cols]
        b = bits_of(bits, name.split('.')[-2] if name.count('.') else name)
        plan.append((name, [k, n], DET[b], oracle.quantize_rows(np.ascontiguousarray(w), b).tobytes()))

    copy('token_embd.weight')
    copy('output_norm.weight')
    quant('output.weight', src='output.weight' if 'output.weight' in T else 'token_embd.weight')
    half = rot // 2
    inv = [math.pow(theta, -(2 * i) / rot) for i in range(half)]
    for use_cos in (True, False):
        f = math.cos if use_cos else math.sin
        tab = np.array([[f(pos * inv[i]) for i in range(half)] for pos in range(n_pos)], np.float64).astype(np.float32)
        plan.append(('rope_cos' if use_cos else 'rope_sin', [half, n_pos], T_F32, tab.tobytes()))
    for i in range(n_layers):
        n = lambda s: f'blk.{i}.{s}'
        copy(n('attn_norm.weight'))
        copy(n('post_attention_norm.weight'))
        for s in ('ffn_gate', 'ffn_up', 'ffn_down'):
            quant(n(f'{s}.weight'))
        if attention[i]:
            for s in ('attn_q', 'attn_k', 'attn_v', 'attn_output'):
                quant(n(f'{s}.weight'))
            copy(n('attn_q_norm.weight'))
            copy(n('attn_k_norm.weight'))
        else:
            vrows = head_perm(n_k, n_v, dv, 2 * kd, conv_dim)
            heads = head_perm(n_k, n_v, 1, 0, n_v)
            quant(n('attn_qkv.weight'), rows=vrows)
            quant(n('attn_gate.weight'), rows=head_perm(n_k, n_v, dv, 0, n_v * dv))
            quant(n('ssm_alpha.weight'), rows=heads)
            quant(n('ssm_beta.weight'), rows=heads)
            quant(n('ssm_out.weight'), cols=head_perm(n_k, n_v, dv, 0, n_v * dv))
            for name, perm in (('ssm_conv1d.weight', vrows), ('ssm_a', heads), ('ssm_dt.bias', heads)):
                dims = T[n(name)][0]
                v = floats(n(name))
                inner = dims[0] if len(dims) > 1 else 1
                v = v.reshape(-1, inner)[perm].reshape(-1)
                plan.append((n(name), dims, T_F32, v.astype(np.float32).tobytes()))
            copy(n('ssm_norm.weight'))
    out_kv = [(k, t, v) for k, t, v in model['kv'] if not k.startswith('split.') and k != 'det.v_scale']
    n_att = sum(attention)
    out_kv.append(('det.v_scale', ARRAY, (F32, [1.0 / 1024.0] * (n_att * n_kv))))
    infos, blobs, off = [], [], 0
    for name, dims, ty, data in plan:
        infos.append((name, dims, ty, off))
        blobs.append(data + bytes(-len(data) % 32))
        off += len(blobs[-1])
    return header(out_kv, infos, 32) + b''.join(blobs)


def read_gguf(data):
    """A GGUF file's bytes -> ({key: (type, value)}, {name: (dims, type, data bytes)}) (gguf.rs:208-300 restated
    for the test side: the oracle model reads the converter restatement's output through this, not the library)."""
    pos = 0

    def take(n):
        nonlocal pos
        b = data[pos:pos + n]
        pos += n
        return b

    def u32():
        return struct.unpack('<I', take(4))[0]

    def u64():
        return struct.unpack('<Q', take(8))[0]

    def string():
        return take(u64()).decode()

    def value(ty):
        if ty == STR:
            return string()
        if ty == ARRAY:
            et, n = u32(), u64()
            return (et, [value(et) for _ in range(n)])
        fmt = _FMT[ty]
        return struct.unpack(fmt, take(struct.calcsize(fmt)))[0]

    assert take(4) == b'GGUF'
    u32()
    n_t, n_kv = u64(), u64()
    kv = {}
    for _ in range(n_kv):
        k = string()
        ty = u32()
        kv[k] = (ty, value(ty))
    infos = []
    for _ in range(n_t):
        name = string()
        dims = [u64() for _ in range(u32())]
        infos.append((name, dims, u32(), u64()))
    align = kv.get('general.alignment', (U32, 32))[1]
    start = (pos + align - 1) // align * align
    tensors = {}
    for name, dims, ty, off in infos:
        k = dims[0]
        rb = 4 * k if ty == T_F32 else 2 * k if ty in (T_F16, T_BF16) else oracle.row_bytes({v: b for b, v in DET.items()}[ty], k)
        rows = int(np.prod(dims[1:])) if len(dims) > 1 else 1
        tensors[name] = (dims, ty, data[start + off:start + off + rb * rows])
    return kv, tensors
