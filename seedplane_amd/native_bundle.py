"""Native SeedPlane bundle (`seedplane-bundle/2` layout) holding engine-ready, optionally quantized tensors.

    python -m seedplane_amd.native_bundle <hf_dir> <out.sp> [--bits 8|4] [--shard 512 --halo 256 --sinks 4]

Same directory layout and manifest schema as the reference converter (seedplane/native_bundle.py:1-137):

  seedplane.json  architecture, shard plan, tensor table, SHA-256 of the source files and of weights.spw
  weights.spw     engine-ready tensors, each at a 256-byte aligned offset: fused QKV (+ bias), gate / up, down, o,
                  embedding (and head when untied), fp32 norms and biases
  tokenizer.json  (+ tokenizer_config.json, chat_template.jinja, generation_config.json when present)

Extension over the reference: matrices may be stored quantized in the formats the HIP engine runs --
int8 symmetric in blocks of 32 along K with one fp16 scale per block (`q8`: codes int8 [N, K], scales fp16
[N, K/32]) or int4 asymmetric in groups of 32 (`q4`: two codes per byte, even k in the low nibble, [N, K/2] uint8;
fp16 scale and fp16 zero per group), w = (code - zero) * scale.  A source checkpoint that is already quantized this
way (`quantization_config.quant_method == 'seedplane'`, tensors `<name>.qweight/.scales/.qzeros`) is copied code for
code; a float checkpoint is rounded to fp16 (reference behaviour) or quantized with `--bits`.

`load(path)` checks the manifest (format, engine, tensor ranges, SHA-256 of weights.spw unless verify=False) and
returns a Hugging Face style (config, tensors) pair that `Qwen2Engine` loads; `Qwen2Engine(bundle_dir)` does this by
itself when the directory holds a seedplane.json.  Only numpy is needed to convert; safetensors are parsed directly.
"""
import argparse
import hashlib
import json
import shutil
import struct
from pathlib import Path

import numpy as np

FORMAT = 'seedplane-bundle/2'
ENGINE = 'seedplane-hip-qwen2/1'
ALIGN = 256
GROUP = 32
# sinks + halo + shard must fit one column's attention range: 512 chunks of 64 keys (the split-K attention kernels)
MAX_WINDOW = 32768
EXTRA_FILES = ('tokenizer.json', 'tokenizer_config.json', 'chat_template.jinja', 'generation_config.json')
_NP_DTYPE = {'f16': '<f2', 'f32': '<f4', 'i8': 'i1', 'u8': 'u1'}


# ----------------------------------------------------------------------------------------------- source reading
def read_safetensors(path):
    """name -> (dtype, shape, raw uint8 view) without loading the file (native_bundle.py:26-32)."""
    with open(path, 'rb') as f:
        n = struct.unpack('<Q', f.read(8))[0]
        header = json.loads(f.read(n))
    data = np.memmap(path, dtype=np.uint8, mode='r', offset=8 + n)
    return {k: (v['dtype'], v['shape'], data[v['data_offsets'][0]:v['data_offsets'][1]])
            for k, v in header.items() if k != '__metadata__'}


def as_f32(dtype, raw):
    """float32 copy of a floating safetensors buffer; BF16 widens exactly (native_bundle.py:35-39)."""
    if dtype == 'F32':
        return np.frombuffer(raw, dtype='<f4').copy()
    if dtype == 'F16':
        return np.frombuffer(raw, dtype='<f2').astype(np.float32)
    if dtype == 'BF16':
        return (np.frombuffer(raw, dtype='<u2').astype(np.uint32) << 16).view(np.float32)
    raise ValueError(f'unsupported dtype {dtype}')


def sha256_file(path, chunk=1 << 24):
    h = hashlib.sha256()
    with open(path, 'rb') as f:
        while True:
            block = f.read(chunk)
            if not block:
                break
            h.update(block)
    return h.hexdigest()


def validate_plan(plan):
    """shard > 0, halo >= 0, sinks >= 0 and the window within MAX_WINDOW (native_bundle.py:56-59)."""
    s, h, k = plan['shard'], plan['halo'], plan['sinks']
    if s <= 0 or h < 0 or k < 0:
        raise ValueError(f'invalid plan {plan}')
    if s + h + k > MAX_WINDOW:
        raise ValueError(f'sinks + halo + shard = {s + h + k} exceeds the engine window {MAX_WINDOW}')


# ----------------------------------------------------------------------------------------------- quantizers
def quantize_q8(w):
    """int8 block-32 symmetric: scale = fp16(max|w| / 127) per block, code = clip(rint(w / scale), -127, 127).
    Returns (codes int8 [N, K], scales fp16 [N, K/32]); a block of zeros gets scale 0 and codes 0."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % GROUP:
        raise ValueError(f'K = {k} is not a multiple of {GROUP}')
    b = w.reshape(n, k // GROUP, GROUP)
    scale = (np.abs(b).max(axis=2) / np.float32(127.0)).astype(np.float16)
    s32 = scale.astype(np.float32)[..., None]
    with np.errstate(divide='ignore', invalid='ignore'):
        q = np.where(s32 > 0, np.rint(b / np.where(s32 > 0, s32, 1)), 0)
    return np.clip(q, -127, 127).astype(np.int8).reshape(n, k), scale


def quantize_q4(w):
    """int4 group-32 asymmetric: scale = fp16((max - min) / 15), zero = fp16(-min / scale), code =
    clip(rint(w / scale + zero), 0, 15), w ~ (code - zero) * scale.  A constant group c gets scale |c| / 15 (1 if c
    is 0) so that it is still represented.  Returns (packed uint8 [N, K/2] with even k in the low nibble, scales,
    zeros), both fp16 [N, K/32]."""
    w = np.asarray(w, dtype=np.float32)
    n, k = w.shape
    if k % GROUP:
        raise ValueError(f'K = {k} is not a multiple of {GROUP}')
    b = w.reshape(n, k // GROUP, GROUP)
    lo, hi = b.min(axis=2), b.max(axis=2)
    span = hi - lo
    flat = np.where(np.abs(lo) > 0, np.abs(lo), np.float32(1.0)) / np.float32(15.0)
    scale = np.where(span > 0, span / np.float32(15.0), flat).astype(np.float16)
    scale = np.where(scale > 0, scale, np.float16(2.0 ** -24))     # spans below fp16's range: smallest step
    s32 = scale.astype(np.float32)
    zero = np.where(span > 0, -lo / s32, np.where(lo < 0, np.float32(15.0), np.float32(0.0))).astype(np.float16)
    q = np.clip(np.rint(b / s32[..., None] + zero.astype(np.float32)[..., None]), 0, 15).astype(np.uint8)
    q = q.reshape(n, k)
    packed = (q[:, 0::2] | (q[:, 1::2] << 4)).astype(np.uint8)
    return packed, scale, zero


# ----------------------------------------------------------------------------------------------- convert
def convert(src, out, bits=None, shard=None, halo=None, sinks=None):
    """Write the bundle for the Hugging Face Qwen2 checkpoint directory `src` into `out`; returns the manifest."""
    src, out = Path(src), Path(out)
    if not src.is_dir():
        raise FileNotFoundError(f'{src} is not a checkpoint directory')
    cfg = json.loads((src / 'config.json').read_text())
    if cfg.get('model_type') != 'qwen2':
        raise ValueError('the native engine currently supports model_type=qwen2 only')
    v1 = src / 'seedplane.json'
    v1_meta = json.loads(v1.read_text()) if v1.exists() else {}
    plan = dict(v1_meta.get('plan', {'shard': 512, 'halo': 256, 'sinks': 4}))
    for key, val in (('shard', shard), ('halo', halo), ('sinks', sinks)):
        if val is not None:
            plan[key] = val
    validate_plan(plan)

    L, H = cfg['num_hidden_layers'], cfg['hidden_size']
    NH, NKV = cfg['num_attention_heads'], cfg['num_key_value_heads']
    I, V = cfg['intermediate_size'], cfg['vocab_size']
    if H % NH or NH % NKV:
        raise ValueError('invalid Qwen2 head configuration')
    HD = H // NH
    theta = cfg.get('rope_theta', cfg.get('rope_parameters', {}).get('rope_theta', 10000.0))
    sq = cfg.get('quantization_config') or {}
    src_bits = sq.get('bits') if sq.get('quant_method') == 'seedplane' else None
    if src_bits is not None and bits is not None and bits != src_bits:
        raise ValueError(f'checkpoint is already {src_bits}-bit; requantization is not supported')
    bits = src_bits if src_bits is not None else bits
    if bits not in (None, 8, 4):
        raise ValueError('bits must be 8 or 4')

    files = sorted(src.glob('*.safetensors'))
    if not files:
        raise FileNotFoundError(f'no safetensors in {src}')
    t = {}
    for f in files:
        for name, v in read_safetensors(f).items():
            if name in t:
                raise ValueError(f'duplicate tensor {name}')
            t[name] = v
    get = lambda name: as_f32(t[name][0], t[name][2]).reshape(t[name][1])
    raw = lambda name, dt: np.frombuffer(t[name][2], dtype=dt).reshape(t[name][1])
    tied = 'lm_head.weight' not in t and 'lm_head.qweight' not in t

    out.mkdir(parents=True, exist_ok=True)
    table, stats, h = {}, {'fp16_overflow': 0, 'fp16_flushed_to_zero': 0}, hashlib.sha256()
    with open(out / 'weights.spw', 'wb') as w:
        def put(name, arr, dtype):
            arr = np.ascontiguousarray(arr)
            if dtype == 'f16' and arr.dtype != np.float16:
                a32 = arr.astype(np.float32)
                data = a32.astype(np.float16)
                stats['fp16_overflow'] += int((np.abs(a32) > 65504).sum())
                stats['fp16_flushed_to_zero'] += int(((a32 != 0) & (data == 0)).sum())
            else:
                data = arr.astype(_NP_DTYPE[dtype])
            pad = (-w.tell()) % ALIGN
            if pad:
                w.write(b'\0' * pad)
                h.update(b'\0' * pad)
            buf = data.astype(_NP_DTYPE[dtype]).tobytes()
            table[name] = {'dtype': dtype, 'shape': list(data.shape), 'offset': w.tell(), 'bytes': len(buf)}
            w.write(buf)
            h.update(buf)

        def put_matrix(name, parts):
            """Rows of the HF matrices `parts` concatenated (the engine's fused packing, qwen_engine.py:71-76)."""
            if src_bits is not None:            # copy the checkpoint's codes
                put(name, np.concatenate([raw(p + '.qweight', 'i1' if src_bits == 8 else 'u1') for p in parts]),
                    'i8' if src_bits == 8 else 'u8')
                put(name + '.scales', np.concatenate([raw(p + '.scales', '<f2') for p in parts]), 'f16')
                if src_bits == 4:
                    put(name + '.zeros', np.concatenate([raw(p + '.qzeros', '<f2') for p in parts]), 'f16')
                return
            m = np.concatenate([get(p + '.weight') for p in parts])
            if bits is None:
                put(name, m, 'f16')
            elif bits == 8:
                c, s = quantize_q8(m)
                put(name, c, 'i8')
                put(name + '.scales', s, 'f16')
            else:
                c, s, z = quantize_q4(m)
                put(name, c, 'u8')
                put(name + '.scales', s, 'f16')
                put(name + '.zeros', z, 'f16')

        put_matrix('embed', ['model.embed_tokens'])
        if not tied:
            put_matrix('lm_head', ['lm_head'])
        put('final_norm', get('model.norm.weight'), 'f32')
        for l in range(L):
            p = f'model.layers.{l}.'
            att = [p + 'self_attn.q_proj', p + 'self_attn.k_proj', p + 'self_attn.v_proj']
            put_matrix(f'{l}.qkv_w', att)
            put(f'{l}.qkv_b', np.concatenate([get(n + '.bias') for n in att]), 'f32')
            put_matrix(f'{l}.o_w', [p + 'self_attn.o_proj'])
            put_matrix(f'{l}.gate_w', [p + 'mlp.gate_proj'])
            put_matrix(f'{l}.up_w', [p + 'mlp.up_proj'])
            put_matrix(f'{l}.down_w', [p + 'mlp.down_proj'])
            put(f'{l}.in_norm', get(p + 'input_layernorm.weight'), 'f32')
            put(f'{l}.post_norm', get(p + 'post_attention_layernorm.weight'), 'f32')

    for name in EXTRA_FILES:
        if (src / name).exists():
            shutil.copyfile(src / name, out / name)
    manifest = {
        'format': FORMAT, 'engine': ENGINE,
        'source': v1_meta.get('source', str(src)),
        'source_files': {f.name: sha256_file(f) for f in files},
        'plan': plan,
        'arch': {'model_type': 'qwen2', 'layers': L, 'hidden': H, 'heads': NH, 'kv_heads': NKV, 'head_dim': HD,
                 'intermediate': I, 'vocab': V, 'rope_theta': theta, 'rms_norm_eps': cfg.get('rms_norm_eps', 1e-6),
                 'max_positions': cfg.get('max_position_embeddings', 32768), 'tied_embeddings': tied},
        'quantization': None if bits is None else {'method': 'seedplane', 'bits': bits, 'group_size': GROUP},
        'weights': {'file': 'weights.spw', 'sha256': h.hexdigest(), 'align': ALIGN, **stats},
        'tensors': table,
        'note': 'weights converted (fp16 rounding or seedplane int8/int4 quantization), never retrained',
    }
    (out / 'seedplane.json').write_text(json.dumps(manifest, indent=1))
    return manifest


# ----------------------------------------------------------------------------------------------- load
def is_bundle(path):
    return (Path(path) / 'seedplane.json').is_file()


def read_manifest(path):
    p = Path(path) / 'seedplane.json'
    if not p.is_file():
        raise FileNotFoundError(f'{path} has no seedplane.json')
    m = json.loads(p.read_text())
    if m.get('format') != FORMAT:
        raise ValueError(f'unsupported bundle format {m.get("format")!r} (expected {FORMAT})')
    if m.get('engine') != ENGINE:
        raise ValueError(f'bundle was written for engine {m.get("engine")!r}, not {ENGINE}')
    validate_plan(m['plan'])
    return m


def load(path, verify=True):
    """(config, tensors) of a bundle: config in Hugging Face config.json form (with the seedplane
    quantization_config when quantized), tensors as CPU torch tensors under Hugging Face names (fused matrices are
    split back into row views).  With verify, weights.spw must match the manifest's SHA-256."""
    import torch
    path = Path(path)
    m = read_manifest(path)
    wf = path / m['weights']['file']
    if not wf.is_file():
        raise FileNotFoundError(f'{wf} is missing')
    if verify and sha256_file(wf) != m['weights']['sha256']:
        raise ValueError(f'{wf} does not match the SHA-256 in seedplane.json')
    size = wf.stat().st_size
    blob = np.memmap(wf, dtype=np.uint8, mode='c')
    a = m['arch']

    def tensor(name):
        e = m['tensors'].get(name)
        if e is None:
            raise ValueError(f'bundle has no tensor {name}')
        if e['dtype'] not in _NP_DTYPE or e['offset'] % ALIGN or e['offset'] + e['bytes'] > size:
            raise ValueError(f'bad table entry for {name}: {e}')
        arr = blob[e['offset']:e['offset'] + e['bytes']].view(_NP_DTYPE[e['dtype']]).reshape(e['shape'])
        if arr.nbytes != e['bytes']:
            raise ValueError(f'bad table entry for {name}: {e}')
        return torch.from_numpy(arr)

    q = m.get('quantization')
    bits = q['bits'] if q else None

    def matrix(out, name, parts):
        """Split the fused matrix `name` into the HF matrices `parts` = [(hf_name, rows)]."""
        mats = [tensor(name)] + ([tensor(name + '.scales')] if bits else []) + \
               ([tensor(name + '.zeros')] if bits == 4 else [])
        suffix = ['.weight'] if bits is None else ['.qweight', '.scales'] + (['.qzeros'] if bits == 4 else [])
        r0 = 0
        for hf, rows in parts:
            for t, sfx in zip(mats, suffix):
                out[hf + sfx] = t[r0:r0 + rows]
            r0 += rows
        if r0 != mats[0].shape[0]:
            raise ValueError(f'{name} has {mats[0].shape[0]} rows, expected {r0}')

    L, H, NH, NKV, HD = a['layers'], a['hidden'], a['heads'], a['kv_heads'], a['head_dim']
    I, V = a['intermediate'], a['vocab']
    w = {}
    matrix(w, 'embed', [('model.embed_tokens', V)])
    if not a['tied_embeddings']:
        matrix(w, 'lm_head', [('lm_head', V)])
    w['model.norm.weight'] = tensor('final_norm')
    for l in range(L):
        p = f'model.layers.{l}.'
        att = [(p + 'self_attn.q_proj', NH * HD), (p + 'self_attn.k_proj', NKV * HD), (p + 'self_attn.v_proj', NKV * HD)]
        matrix(w, f'{l}.qkv_w', att)
        b = tensor(f'{l}.qkv_b')
        r0 = 0
        for hf, rows in att:
            w[hf + '.bias'] = b[r0:r0 + rows]
            r0 += rows
        matrix(w, f'{l}.o_w', [(p + 'self_attn.o_proj', H)])
        matrix(w, f'{l}.gate_w', [(p + 'mlp.gate_proj', I)])
        matrix(w, f'{l}.up_w', [(p + 'mlp.up_proj', I)])
        matrix(w, f'{l}.down_w', [(p + 'mlp.down_proj', H)])
        w[p + 'input_layernorm.weight'] = tensor(f'{l}.in_norm')
        w[p + 'post_attention_layernorm.weight'] = tensor(f'{l}.post_norm')
    cfg = {'model_type': 'qwen2', 'num_hidden_layers': L, 'hidden_size': H, 'num_attention_heads': NH,
           'num_key_value_heads': NKV, 'intermediate_size': I, 'vocab_size': V, 'rope_theta': a['rope_theta'],
           'rms_norm_eps': a['rms_norm_eps'], 'max_position_embeddings': a['max_positions'],
           'tie_word_embeddings': a['tied_embeddings']}
    if bits:
        cfg['quantization_config'] = {'quant_method': 'seedplane', 'bits': bits, 'group_size': q['group_size']}
    return cfg, w


def main():
    ap = argparse.ArgumentParser(description='convert a Qwen2 checkpoint into a seedplane-bundle/2 directory')
    ap.add_argument('src')
    ap.add_argument('out')
    ap.add_argument('--bits', type=int, choices=[8, 4], default=None)
    ap.add_argument('--shard', type=int)
    ap.add_argument('--halo', type=int)
    ap.add_argument('--sinks', type=int)
    a = ap.parse_args()
    m = convert(a.src, a.out, bits=a.bits, shard=a.shard, halo=a.halo, sinks=a.sinks)
    print(json.dumps({'format': m['format'], 'plan': m['plan'], 'quantization': m['quantization'],
                      'sha256': m['weights']['sha256'], 'tensors': len(m['tensors'])}))


if __name__ == '__main__':
    main()
