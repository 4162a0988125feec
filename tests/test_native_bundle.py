"""seedplane-bundle/2 conversion and loading (host side; reference: seedplane/native_bundle.py:62-137 and its unit
tests tests/test_core.py:178-200).  Quantized matrices are checked against the oracle's closed-form dequantisers."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle.quant_ref import dequant_q4, dequant_q8, unpack_q4
from seedplane_amd import native_bundle
from seedplane_amd.presets import preset
from seedplane_amd.synth import make_weights, write_bundle


def tiny_qwen2(directory, seed=0):
    """The 2-layer test model of the reference (L 2, H 128, 2 / 1 heads, head_dim 64, I 256, V 50; randn * 0.05,
    embedding x 20, unit norms) written as a BF16 safetensors checkpoint.  Returns the fp32 tensors."""
    cfg, w = make_weights(preset('tiny'), 'f32', seed=seed)
    write_bundle(directory, cfg, {k: v.to(torch.bfloat16) for k, v in w.items()})
    return w


def test_convert_layout_roundtrip_and_plan(tmp_path):
    w = tiny_qwen2(tmp_path)
    out = tmp_path / 'out.sp'
    m = native_bundle.convert(tmp_path, out, shard=8, halo=4, sinks=2)
    assert m['format'] == 'seedplane-bundle/2' and m['plan'] == {'shard': 8, 'halo': 4, 'sinks': 2}
    assert all(t['offset'] % native_bundle.ALIGN == 0 for t in m['tensors'].values())
    blob = np.fromfile(out / 'weights.spw', dtype=np.uint8)
    t = m['tensors']['1.qkv_w']
    got = blob[t['offset']:t['offset'] + t['bytes']].view('<f2').reshape(t['shape']).astype(np.float32)
    p = 'model.layers.1.self_attn.'
    ref = torch.cat([w[p + 'q_proj.weight'], w[p + 'k_proj.weight'], w[p + 'v_proj.weight']]).to(torch.bfloat16).float()
    assert np.abs(got - ref.numpy().astype(np.float16).astype(np.float32)).max() < 1e-12
    assert json.loads((out / 'seedplane.json').read_text())['weights']['sha256'] == m['weights']['sha256']
    assert m['weights']['sha256'] == native_bundle.sha256_file(out / 'weights.spw')
    assert m['quantization'] is None and m['arch']['tied_embeddings']


def test_keeps_v1_plan_and_rejects_bad_plans(tmp_path):
    tiny_qwen2(tmp_path)
    (tmp_path / 'seedplane.json').write_text(json.dumps({'format': 'seedplane-bundle/1', 'source': 'tiny',
                                                         'plan': {'shard': 16, 'halo': 8, 'sinks': 1}}))
    m = native_bundle.convert(tmp_path, tmp_path / 'a.sp')
    assert (m['plan'], m['source']) == ({'shard': 16, 'halo': 8, 'sinks': 1}, 'tiny')
    with pytest.raises(ValueError):
        native_bundle.convert(tmp_path, tmp_path / 'b.sp', shard=native_bundle.MAX_WINDOW, halo=200)
    for args in ((0, 1, 0), (1, -1, 0), (1, 0, -1)):
        with pytest.raises(ValueError):
            native_bundle.convert(tmp_path, tmp_path / 'c.sp', *((None,) + args))


def test_q8_quantizer_error_bound_and_exact_codes():
    rng = np.random.default_rng(0)
    w = rng.normal(0, 0.05, (48, 256)).astype(np.float32)
    w[3, 32:64] = 0.0                                     # an all-zero block
    codes, scales = native_bundle.quantize_q8(w)
    assert codes.dtype == np.int8 and codes.min() >= -127 and codes.max() <= 127
    deq = dequant_q8(torch.from_numpy(codes), torch.from_numpy(scales)).numpy()
    s = np.repeat(scales.astype(np.float32), 32, axis=1)
    # rint to the nearest code: half a step, plus the clip at 127 when the fp16 scale rounded down (< 2^-11 rel.)
    assert np.all(np.abs(deq - w) <= s * (0.5 + 127 * 2.0 ** -11) + 1e-12)
    assert np.all(deq[3, 32:64] == 0)
    # weights that are codes x a power of two come back exactly
    c = rng.integers(-127, 128, (16, 64)).astype(np.float32)
    c[:, ::32] = 127                                      # every block reaches the full code range
    codes2, scales2 = native_bundle.quantize_q8(c * 2.0 ** -9)
    assert np.array_equal(codes2.astype(np.float32), c) and np.all(scales2 == np.float16(2.0 ** -9))


def test_q4_quantizer_error_bound_packing_and_constant_groups():
    rng = np.random.default_rng(1)
    w = rng.normal(0, 0.05, (32, 128)).astype(np.float32)
    w[0, :32] = 0.25                                      # constant groups: positive, negative, zero
    w[1, :32] = -0.5
    w[2, :32] = 0.0
    packed, scales, zeros = native_bundle.quantize_q4(w)
    assert packed.shape == (32, 64) and packed.dtype == np.uint8
    deq = dequant_q4(torch.from_numpy(packed), torch.from_numpy(scales), torch.from_numpy(zeros)).numpy()
    s = np.repeat(scales.astype(np.float32), 32, axis=1)
    assert np.all(np.abs(deq - w) <= s * 0.6 + 1e-7)
    # a constant group is 15 (or 0 - 15) steps of fp16(|c| / 15): only the scale's fp16 rounding remains
    for r in (0, 1):
        assert np.all(np.abs(deq[r, :32] - w[r, :32]) <= np.abs(w[r, :32]) * 2.0 ** -11)
    assert np.all(deq[2, :32] == 0)
    # packing: even k in the low nibble (the layout the engine's int4 GEMV and the oracle read)
    codes = unpack_q4(torch.from_numpy(packed)).numpy()
    assert np.array_equal(packed, (codes[:, 0::2] | (codes[:, 1::2] << 4)).astype(np.uint8))
    # (code - zero) * scale with an integer zero and a power-of-two scale comes back exactly
    c = rng.integers(0, 16, (8, 64)).astype(np.float32)
    c[:, ::32], c[:, 1::32] = 0, 15
    p2, s2, z2 = native_bundle.quantize_q4((c - 3.0) * 2.0 ** -6)
    assert np.array_equal(unpack_q4(torch.from_numpy(p2)).numpy().astype(np.float32), c)
    assert np.all(s2 == np.float16(2.0 ** -6)) and np.all(z2 == np.float16(3.0))


@pytest.mark.parametrize('bits', [8, 4])
def test_quantized_bundle_roundtrip(tmp_path, bits):
    w = tiny_qwen2(tmp_path)
    out = tmp_path / f'q{bits}.sp'
    m = native_bundle.convert(tmp_path, out, bits=bits)
    assert m['quantization'] == {'method': 'seedplane', 'bits': bits, 'group_size': 32}
    cfg, t = native_bundle.load(out)
    assert cfg['quantization_config'] == {'quant_method': 'seedplane', 'bits': bits, 'group_size': 32}
    assert (cfg['num_hidden_layers'], cfg['hidden_size'], cfg['vocab_size']) == (2, 128, 50)
    for name in ('model.layers.1.self_attn.k_proj', 'model.layers.0.mlp.down_proj', 'model.embed_tokens'):
        src = w[name + '.weight'].to(torch.bfloat16).float().numpy()
        if bits == 8:
            c, s = native_bundle.quantize_q8(src)
            assert np.array_equal(t[name + '.qweight'].numpy(), c) and np.array_equal(t[name + '.scales'].numpy(), s)
        else:
            c, s, z = native_bundle.quantize_q4(src)
            assert np.array_equal(t[name + '.qweight'].numpy(), c) and np.array_equal(t[name + '.qzeros'].numpy(), z)
    b = w['model.layers.1.self_attn.v_proj.bias'].to(torch.bfloat16).float()
    assert torch.equal(t['model.layers.1.self_attn.v_proj.bias'], b)


def test_prequantized_checkpoint_is_copied_code_for_code(tmp_path):
    cfg, w = make_weights(preset('tiny'), 'q4', seed=3)
    src = write_bundle(tmp_path / 'hf', cfg, w)
    native_bundle.convert(src, tmp_path / 'b.sp')
    cfg2, t = native_bundle.load(tmp_path / 'b.sp')
    assert cfg2['quantization_config']['bits'] == 4
    for k, v in w.items():
        assert torch.equal(t[k].to(v.dtype), v), k
    with pytest.raises(ValueError):
        native_bundle.convert(src, tmp_path / 'c.sp', bits=8)


def test_load_rejects_tampered_or_foreign_bundles(tmp_path):
    tiny_qwen2(tmp_path)
    out = tmp_path / 'out.sp'
    native_bundle.convert(tmp_path, out)
    native_bundle.load(out)
    data = bytearray((out / 'weights.spw').read_bytes())
    data[1000] ^= 1
    (out / 'weights.spw').write_bytes(bytes(data))
    with pytest.raises(ValueError, match='SHA-256'):
        native_bundle.load(out)
    native_bundle.load(out, verify=False)                 # the check can be skipped explicitly
    man = json.loads((out / 'seedplane.json').read_text())
    (out / 'seedplane.json').write_text(json.dumps(dict(man, format='seedplane-bundle/1')))
    with pytest.raises(ValueError, match='format'):
        native_bundle.load(out)
    (out / 'seedplane.json').write_text(json.dumps(man))
    (out / 'weights.spw').unlink()
    with pytest.raises(FileNotFoundError):
        native_bundle.load(out)
    with pytest.raises(FileNotFoundError):
        native_bundle.load(tmp_path / 'nothing')


def test_reference_float_bundles_load_and_quantized_bundles_fail_closed(tmp_path):
    # the reference converter writes engine 'seedplane-native-qwen2/1' with the same tensor table: it loads here.  A
    # quantized bundle carries a format string the reference runtime refuses (qwen_vk.cpp:68 checks it), and a
    # seedplane-bundle/2 holding integer codes is rejected here
    tiny_qwen2(tmp_path)
    out = tmp_path / 'f.sp'
    native_bundle.convert(tmp_path, out)
    man = json.loads((out / 'seedplane.json').read_text())
    (out / 'seedplane.json').write_text(json.dumps(dict(man, engine='seedplane-native-qwen2/1')))
    cfg, t = native_bundle.load(out)
    assert cfg['num_hidden_layers'] == 2 and t['model.embed_tokens.weight'].dtype == torch.float16
    (out / 'seedplane.json').write_text(json.dumps(dict(man, engine='someone-else/1')))
    with pytest.raises(ValueError, match='engine'):
        native_bundle.load(out)
    q = native_bundle.convert(tmp_path, tmp_path / 'q.sp', bits=8)
    assert q['format'] == 'seedplane-bundle/2-quant' and q['format'] != 'seedplane-bundle/2'
    qman = json.loads((tmp_path / 'q.sp' / 'seedplane.json').read_text())
    (tmp_path / 'q.sp' / 'seedplane.json').write_text(json.dumps(dict(qman, format='seedplane-bundle/2')))
    with pytest.raises(ValueError, match='fp16 / fp32'):
        native_bundle.load(tmp_path / 'q.sp')


def test_fused_rows_split_back_to_checkpoint_tensors(tmp_path):
    # every Hugging Face tensor comes back from the bundle (fp16-rounded), fused matrices and the fused bias included
    w = tiny_qwen2(tmp_path)
    native_bundle.convert(tmp_path, tmp_path / 'b.sp')
    cfg, t = native_bundle.load(tmp_path / 'b.sp')
    assert set(t) == set(w)
    for k, v in w.items():
        want = v.to(torch.bfloat16).float()
        got = t[k].float()
        if v.dim() == 2:
            want = want.half().float()
        assert torch.equal(got, want), k
