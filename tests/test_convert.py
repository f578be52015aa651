"""`det convert` (det_convert, det_gguf.h; the reference's convert.rs + config.rs, `--no-calibrate`) on the GPU,
byte for byte against the Python restatement of the conversion (tests/gguf_ref.py) on a synthetic qwen35 float
model: one GDN layer (value-head permutations with 2 key heads and 4 value heads) and one attention layer, an
extra next-token-prediction block that convert skips, BF16 / F16 / F32 sources, tied and untied heads, the
default and custom width presets, explicit rotary lengths and a split source."""
import numpy as np
import pytest

from det_amd import gguf
from tests import gguf_ref as R

pytestmark = pytest.mark.gpu

H, V, FF = 256, 320, 384
NK, NV, DK, DV = 2, 4, 128, 128
HEADS, NKV, HD, ROT = 2, 1, 128, 64


def bf16_exact(a):
    return (np.ascontiguousarray(a, np.float32).view(np.uint32) & 0xFFFF0000).view(np.float32)


def synthetic_model(seed=1, tied=False):
    rng = np.random.default_rng(seed)
    g = lambda *s: (rng.standard_normal(s).astype(np.float32) * np.float32(0.02))
    kv = [('general.architecture', R.STR, 'qwen35'), ('general.name', R.STR, 'synthetic'),
          ('qwen35.block_count', R.U32, 3), ('qwen35.nextn_predict_layers', R.U32, 1),
          ('qwen35.full_attention_interval', R.U32, 2), ('qwen35.embedding_length', R.U32, H),
          ('qwen35.feed_forward_length', R.U32, FF), ('qwen35.attention.head_count', R.U32, HEADS),
          ('qwen35.attention.head_count_kv', R.U32, NKV), ('qwen35.attention.key_length', R.U32, HD),
          ('qwen35.attention.layer_norm_rms_epsilon', R.F32, 1e-6), ('qwen35.rope.dimension_count', R.U32, ROT),
          ('qwen35.rope.freq_base', R.F32, 10000000.0), ('qwen35.context_length', R.U32, 40),
          ('qwen35.ssm.state_size', R.U32, DK), ('qwen35.ssm.time_step_rank', R.U32, NV),
          ('qwen35.ssm.group_count', R.U32, NK), ('qwen35.ssm.inner_size', R.U32, NV * DV),
          ('qwen35.ssm.conv_kernel', R.U32, 4), ('det.v_scale', R.ARRAY, (R.F32, [0.5])),
          ('tokenizer.ggml.tokens', R.ARRAY, (R.STR, [f't{i}' for i in range(V)]))]
    T = {}

    def add(name, dims, ty, a):
        a = bf16_exact(a) if ty == R.T_BF16 else a
        T[name] = (dims, ty, R.to_bytes(a, ty))
    add('token_embd.weight', [H, V], R.T_BF16, g(V, H))
    add('output_norm.weight', [H], R.T_F32, 1 + g(H))
    if not tied:
        add('output.weight', [H, V], R.T_BF16, g(V, H))
    conv_dim = 2 * NK * DK + NV * DV
    for i, attn in ((0, False), (1, True)):
        n = lambda s: f'blk.{i}.{s}'
        add(n('attn_norm.weight'), [H], R.T_F32, 1 + g(H))
        add(n('post_attention_norm.weight'), [H], R.T_F32, 1 + g(H))
        add(n('ffn_gate.weight'), [H, FF], R.T_F16, g(FF, H))
        add(n('ffn_up.weight'), [H, FF], R.T_BF16, g(FF, H))
        add(n('ffn_down.weight'), [FF, H], R.T_F32, g(H, FF))
        if attn:
            add(n('attn_q.weight'), [H, 2 * HEADS * HD], R.T_BF16, g(2 * HEADS * HD, H))
            add(n('attn_k.weight'), [H, NKV * HD], R.T_BF16, g(NKV * HD, H))
            add(n('attn_v.weight'), [H, NKV * HD], R.T_F16, g(NKV * HD, H))
            add(n('attn_output.weight'), [HEADS * HD, H], R.T_BF16, g(H, HEADS * HD))
            add(n('attn_q_norm.weight'), [HD], R.T_F32, 1 + g(HD))
            add(n('attn_k_norm.weight'), [HD], R.T_F32, 1 + g(HD))
        else:
            add(n('attn_qkv.weight'), [H, conv_dim], R.T_BF16, g(conv_dim, H))
            add(n('attn_gate.weight'), [H, NV * DV], R.T_BF16, g(NV * DV, H))
            add(n('ssm_alpha.weight'), [H, NV], R.T_F32, g(NV, H))
            add(n('ssm_beta.weight'), [H, NV], R.T_F32, g(NV, H))
            add(n('ssm_out.weight'), [NV * DV, H], R.T_BF16, g(H, NV * DV))
            add(n('ssm_conv1d.weight'), [4, conv_dim], R.T_F32, g(conv_dim, 4))
            add(n('ssm_a'), [NV], R.T_F32, -np.abs(g(NV)) - 1)
            add(n('ssm_dt.bias'), [NV], R.T_F32, g(NV))
            add(n('ssm_norm.weight'), [DV], R.T_F32, 1 + g(DV))
    add('blk.2.attn_norm.weight', [H], R.T_F32, 1 + g(H))      # the next-token-prediction block: not converted
    return {'kv': kv, 'tensors': T}


def write_model(path, model):
    R.write_gguf(path, model['kv'], [(k, d, t, b) for k, (d, t, b) in model['tensors'].items()])


@pytest.mark.parametrize('tied,bits,rope', [(False, None, 0), (True, '4,ffn_down=8,output=6,attn_qkv=8', 24),
                                             (False, '8', 7)])
def test_convert_bytes(tmp_path, tied, bits, rope):
    model = synthetic_model(tied=tied)
    src, dst = tmp_path / 'm-BF16.gguf', tmp_path / 'm-det.gguf'
    write_model(src, model)
    print(f'convert tied={tied} bits={bits} rope={rope}', flush=True)
    gguf.convert(src, dst, bits, rope)
    want = R.convert_ref(model, bits or R_DEFAULT, rope or None)
    got = dst.read_bytes()
    assert len(got) == len(want)
    if got != want:
        i = next(j for j in range(len(want)) if got[j] != want[j])
        pytest.fail(f'first difference at byte {i} of {len(want)}')
    with gguf.Gguf(dst) as g:                                  # and the library reads its own output
        head = {None: 0xDE08, '4,ffn_down=8,output=6,attn_qkv=8': 0xDE06, '8': 0xDE08}[bits]
        assert g.tensor('output.weight').type == head
        assert g.array('det.v_scale') == (R.F32, [1.0 / 1024.0])


R_DEFAULT = '6,output=8,ssm_alpha=8,ssm_beta=8'


def test_convert_split_source(tmp_path):
    """A source split over two files (split.count, -0000N-of-00002 names) converts to the same bytes."""
    model = synthetic_model(seed=2)
    names = list(model['tensors'])
    kv = model['kv'] + [('split.count', R.U16, 2)]
    for part, sel in ((1, names[:9]), (2, names[9:])):
        R.write_gguf(tmp_path / f'm-{part:05d}-of-00002.gguf', kv if part == 1 else [('split.count', R.U16, 2)],
                     [(k,) + model['tensors'][k] for k in sel])
    dst = tmp_path / 'out.gguf'
    gguf.convert(tmp_path / 'm-00001-of-00002.gguf', dst)
    assert dst.read_bytes() == R.convert_ref(model)


def test_convert_errors(tmp_path):
    model = synthetic_model()
    src = tmp_path / 'm.gguf'
    write_model(src, model)
    for bits, msg in (('5', 'bit width 5 is not 4, 6 or 8'), ('6,ffn_down=x', 'bad bit width "x"')):
        with pytest.raises(gguf.GgufError, match=msg):
            gguf.convert(src, tmp_path / 'o.gguf', bits)
    del model['tensors']['blk.1.attn_k.weight']
    write_model(src, model)
    with pytest.raises(gguf.GgufError, match='missing tensor blk.1.attn_k.weight'):
        gguf.convert(src, tmp_path / 'o.gguf')
