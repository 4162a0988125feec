"""On-disk bundles in the reference's `seedplane-bundle/2` layout, extended with the quantized matrices the HIP engine
runs.

    python -m seedplane_amd.native_bundle <hf_dir> <out.sp> [--bits 8|4] [--shard 512 --halo 256 --sinks 4]

A bundle is a directory (format of the reference converter, seedplane/native_bundle.py:62-137, read by
native/vulkan_decode/qwen_vk.cpp:63-85):

  seedplane.json  format, engine, source files with their SHA-256, shard plan, architecture, the tensor table
                  (name -> dtype, shape, byte offset, byte count) and the SHA-256 of weights.spw
  weights.spw     the tensors back to back, each starting at a multiple of 256 bytes: fused QKV weight (+ fp32 bias),
                  o, gate, up, down, fp32 norms, the embedding (and the head when untied)
  tokenizer.json  and the other tokenizer / generation files of the checkpoint, copied when present

Float bundles hold fp16 matrices and are `seedplane-bundle/2` exactly as the reference writes them, so either side
can read the other's.  Quantized bundles hold int8 (blocks of 32 along K, fp16 scale: `<name>` i8 [N, K] +
`<name>.scales` f16 [N, K/32]) or int4 (groups of 32, two codes per byte with even k in the low nibble, fp16 scale and
zero: `<name>` u8 [N, K/2] + `.scales` + `.zeros`, w = (code - zero) * scale) matrices; they carry the format string
`seedplane-bundle/2-quant` and a `quantization` object, so the reference runtime, which checks the format string and
would read the codes as fp16, refuses them instead.

The bundle's contents are described once, by `_layout`: the writer walks it to place tensors and the reader walks
it to split fused matrices back into Hugging Face names.
"""
import argparse
import hashlib
import json
import shutil
from pathlib import Path

import numpy as np

FORMAT = 'seedplane-bundle/2'
FORMAT_QUANT = 'seedplane-bundle/2-quant'
ENGINE = 'seedplane-hip-qwen2/1'
REFERENCE_ENGINE = 'seedplane-native-qwen2/1'       # float bundles written by the reference converter
ALIGN = 256
GROUP = 32
# sinks + halo + shard must fit one column's attention range: 512 chunks of 64 keys (the split-K attention kernels)
MAX_WINDOW = 32768
EXTRA_FILES = ('tokenizer.json', 'tokenizer_config.json', 'chat_template.jinja', 'generation_config.json')
DEFAULT_PLAN = {'shard': 512, 'halo': 256, 'sinks': 4}
_STORE = {'f16': np.dtype('<f2'), 'f32': np.dtype('<f4'), 'i8': np.dtype('i1'), 'u8': np.dtype('u1')}


def sha256_file(path, chunk=1 << 24):
    digest = hashlib.sha256()
    with open(path, 'rb') as f:
        for block in iter(lambda: f.read(chunk), b''):
            digest.update(block)
    return digest.hexdigest()


def check_plan(plan):
    """A shard plan needs shard >= 1, halo >= 0, sinks >= 0, and a window sinks + halo + shard the kernels hold."""
    shard, halo, sinks = (int(plan[k]) for k in ('shard', 'halo', 'sinks'))
    if shard < 1:
        raise ValueError(f'plan {plan}: shard must be at least 1')
    if halo < 0 or sinks < 0:
        raise ValueError(f'plan {plan}: halo and sinks must be non-negative')
    if shard + halo + sinks > MAX_WINDOW:
        raise ValueError(f'plan {plan}: window sinks + halo + shard = {shard + halo + sinks} is larger than '
                         f'{MAX_WINDOW} positions')


# ----------------------------------------------------------------------------------------------- checkpoint input
class Checkpoint:
    """The tensors of a Hugging Face checkpoint directory, memory-mapped.  A safetensors file is an 8-byte
    little-endian header length, a JSON header (name -> dtype, shape, [begin, end) of the data) and the data."""

    def __init__(self, directory):
        self.dir = Path(directory)
        self.files = sorted(self.dir.glob('*.safetensors'))
        if not self.files:
            raise FileNotFoundError(f'no safetensors in {self.dir}')
        self._where = {}
        for path in self.files:
            blob = np.memmap(path, dtype=np.uint8, mode='r')
            head = int.from_bytes(bytes(blob[:8]), 'little')
            body = 8 + head
            for name, info in json.loads(bytes(blob[8:body])).items():
                if name == '__metadata__':
                    continue
                if name in self._where:
                    raise ValueError(f'tensor {name} appears twice in {self.dir}')
                begin, end = info['data_offsets']
                self._where[name] = (info['dtype'], tuple(info['shape']), blob[body + begin:body + end])

    def __contains__(self, name):
        return name in self._where

    def floats(self, name):
        """float32 values of a floating tensor (BF16 widens exactly: its bits are the top half of an fp32)."""
        dtype, shape, buf = self._where[name]
        if dtype == 'BF16':
            out = (buf.view('<u2').astype(np.uint32) << 16).view(np.float32)
        elif dtype == 'F16':
            out = buf.view('<f2').astype(np.float32)
        elif dtype == 'F32':
            out = buf.view('<f4').copy()
        else:
            raise ValueError(f'{name}: dtype {dtype} is not a float type')
        return out.reshape(shape)

    def stored(self, name, dtype):
        """The tensor's bytes viewed as `dtype` (quantized codes, fp16 scales) without conversion."""
        _, shape, buf = self._where[name]
        return buf.view(dtype).reshape(shape)


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


# ----------------------------------------------------------------------------------------------- layout
def _layout(arch):
    """Every tensor of a bundle in file order: (bundle name, [(Hugging Face name, rows)], kind).  kind 'matrix':
    the rows of the named matrices stacked (the engine's fused packing, qwen_engine.py:64-80); 'vector': fp32
    values, several sources concatenated (the fused QKV bias)."""
    L, H, I, V = arch['layers'], arch['hidden'], arch['intermediate'], arch['vocab']
    q_rows, kv_rows = arch['heads'] * arch['head_dim'], arch['kv_heads'] * arch['head_dim']
    yield 'embed', [('model.embed_tokens', V)], 'matrix'
    if not arch['tied_embeddings']:
        yield 'lm_head', [('lm_head', V)], 'matrix'
    yield 'final_norm', [('model.norm.weight', H)], 'vector'
    for l in range(L):
        p = f'model.layers.{l}.'
        attn = [(p + 'self_attn.q_proj', q_rows), (p + 'self_attn.k_proj', kv_rows), (p + 'self_attn.v_proj', kv_rows)]
        yield f'{l}.qkv_w', attn, 'matrix'
        yield f'{l}.qkv_b', [(n + '.bias', r) for n, r in attn], 'vector'
        yield f'{l}.o_w', [(p + 'self_attn.o_proj', H)], 'matrix'
        yield f'{l}.gate_w', [(p + 'mlp.gate_proj', I)], 'matrix'
        yield f'{l}.up_w', [(p + 'mlp.up_proj', I)], 'matrix'
        yield f'{l}.down_w', [(p + 'mlp.down_proj', H)], 'matrix'
        yield f'{l}.in_norm', [(p + 'input_layernorm.weight', H)], 'vector'
        yield f'{l}.post_norm', [(p + 'post_attention_layernorm.weight', H)], 'vector'


# the parts of a stored matrix: (bundle suffix, Hugging Face suffix, dtype) per weight format
_PARTS = {None: [('', '.weight', 'f16')],
          8: [('', '.qweight', 'i8'), ('.scales', '.scales', 'f16')],
          4: [('', '.qweight', 'u8'), ('.scales', '.scales', 'f16'), ('.zeros', '.qzeros', 'f16')]}


class _WeightsFile:
    """Appends tensors to weights.spw, each at an ALIGN-byte boundary, hashing every byte written (padding too) and
    counting the values fp16 cannot hold (overflow) or rounds to zero."""

    def __init__(self, path):
        self.f = open(path, 'wb')
        self.sha = hashlib.sha256()
        self.table = {}
        self.overflow = self.flushed = 0

    def _emit(self, data):
        self.f.write(data)
        self.sha.update(data)

    def add(self, name, values, dtype):
        if dtype == 'f16' and values.dtype != np.float16:
            wide = np.asarray(values, dtype=np.float32)
            values = wide.astype(np.float16)
            self.overflow += int(np.count_nonzero(np.abs(wide) > 65504))
            self.flushed += int(np.count_nonzero((values == 0) & (wide != 0)))
        data = np.ascontiguousarray(values, dtype=_STORE[dtype])
        self._emit(bytes(-self.f.tell() % ALIGN))
        self.table[name] = {'dtype': dtype, 'shape': list(data.shape), 'offset': self.f.tell(), 'bytes': data.nbytes}
        self._emit(data.tobytes())

    def close(self):
        self.f.close()


# ----------------------------------------------------------------------------------------------- convert
def _arch_of(cfg):
    L, H = cfg['num_hidden_layers'], cfg['hidden_size']
    NH, NKV = cfg['num_attention_heads'], cfg['num_key_value_heads']
    if H % NH or NH % NKV:
        raise ValueError('invalid Qwen2 head configuration')
    theta = cfg.get('rope_theta', cfg.get('rope_parameters', {}).get('rope_theta', 10000.0))
    return {'model_type': 'qwen2', 'layers': L, 'hidden': H, 'heads': NH, 'kv_heads': NKV, 'head_dim': H // NH,
            'intermediate': cfg['intermediate_size'], 'vocab': cfg['vocab_size'], 'rope_theta': theta,
            'rms_norm_eps': cfg.get('rms_norm_eps', 1e-6), 'max_positions': cfg.get('max_position_embeddings', 32768),
            'tied_embeddings': None}


def convert(src, out, bits=None, shard=None, halo=None, sinks=None):
    """Write the bundle of the Hugging Face Qwen2 checkpoint directory `src` into `out`; returns the manifest.
    Float matrices are rounded to fp16, or quantized with bits = 8 / 4; a checkpoint that is already quantized in the
    engine's formats (quantization_config.quant_method 'seedplane', `<name>.qweight/.scales/.qzeros`) keeps its
    codes.  The plan and source name of a version-1 seedplane.json in `src` carry over; shard / halo / sinks given
    here replace the plan's values."""
    src, out = Path(src), Path(out)
    if not src.is_dir():
        raise FileNotFoundError(f'{src} is not a checkpoint directory')
    cfg = json.loads((src / 'config.json').read_text())
    if cfg.get('model_type') != 'qwen2':
        raise ValueError('the native engine currently supports model_type=qwen2 only')
    old = json.loads((src / 'seedplane.json').read_text()) if (src / 'seedplane.json').exists() else {}
    plan = {**DEFAULT_PLAN, **old.get('plan', {})}
    plan.update({k: v for k, v in (('shard', shard), ('halo', halo), ('sinks', sinks)) if v is not None})
    check_plan(plan)

    qc = cfg.get('quantization_config') or {}
    held = qc.get('bits') if qc.get('quant_method') == 'seedplane' else None
    if held is not None and bits not in (None, held):
        raise ValueError(f'the checkpoint is already {held}-bit; requantizing is not supported')
    bits = held if held is not None else bits
    if bits not in (None, 8, 4):
        raise ValueError('bits must be 8 or 4')

    ck = Checkpoint(src)
    arch = _arch_of(cfg)
    arch['tied_embeddings'] = 'lm_head.weight' not in ck and 'lm_head.qweight' not in ck
    out.mkdir(parents=True, exist_ok=True)
    wf = _WeightsFile(out / 'weights.spw')
    try:
        for name, sources, kind in _layout(arch):
            if kind == 'vector':
                wf.add(name, np.concatenate([ck.floats(s).reshape(-1) for s, _ in sources]), 'f32')
            elif held is not None:          # codes, scales (and zeros) exactly as the checkpoint holds them
                for suffix, hf_suffix, dtype in _PARTS[held]:
                    wf.add(name + suffix, np.concatenate([ck.stored(s + hf_suffix, _STORE[dtype]) for s, _ in sources]),
                           dtype)
            else:
                rows = np.concatenate([ck.floats(s + '.weight') for s, _ in sources])
                parts = (rows,) if bits is None else quantize_q8(rows) if bits == 8 else quantize_q4(rows)
                for (suffix, _, dtype), values in zip(_PARTS[bits], parts):
                    wf.add(name + suffix, values, dtype)
    finally:
        wf.close()
    for extra in EXTRA_FILES:
        if (src / extra).exists():
            shutil.copyfile(src / extra, out / extra)
    manifest = {
        'format': FORMAT if bits is None else FORMAT_QUANT,
        'engine': ENGINE,
        'source': old.get('source', str(src)),
        'source_files': {f.name: sha256_file(f) for f in ck.files},
        'plan': plan,
        'arch': arch,
        'quantization': None if bits is None else {'method': 'seedplane', 'bits': bits, 'group_size': GROUP},
        'weights': {'file': 'weights.spw', 'sha256': wf.sha.hexdigest(), 'align': ALIGN,
                    'fp16_overflow': wf.overflow, 'fp16_flushed_to_zero': wf.flushed},
        'tensors': wf.table,
        'note': 'weights converted (fp16 rounding or seedplane int8/int4 quantization), never retrained',
    }
    (out / 'seedplane.json').write_text(json.dumps(manifest, indent=1))
    return manifest


# ----------------------------------------------------------------------------------------------- load
def is_bundle(path):
    return path is not None and (Path(path) / 'seedplane.json').is_file()


def read_manifest(path):
    """The bundle's manifest after its identity checks: `seedplane-bundle/2` from this build or from the reference
    converter (fp16 / fp32 tensors only), or `seedplane-bundle/2-quant` from this build; a valid shard plan."""
    p = Path(path) / 'seedplane.json'
    if not p.is_file():
        raise FileNotFoundError(f'{path} has no seedplane.json')
    m = json.loads(p.read_text())
    fmt, engine = m.get('format'), m.get('engine')
    if fmt == FORMAT:
        if engine not in (ENGINE, REFERENCE_ENGINE):
            raise ValueError(f'{FORMAT} bundle of unknown engine {engine!r}')
        odd = sorted({t.get('dtype') for t in m.get('tensors', {}).values()} - {'f16', 'f32'})
        if odd:
            raise ValueError(f'a {FORMAT} bundle holds fp16 / fp32 tensors only, not {odd}')
    elif fmt == FORMAT_QUANT:
        if engine != ENGINE:
            raise ValueError(f'{FORMAT_QUANT} bundle of unknown engine {engine!r}')
    else:
        raise ValueError(f'unsupported bundle format {fmt!r} (expected {FORMAT} or {FORMAT_QUANT})')
    check_plan(m['plan'])
    return m


def load(path, verify=True):
    """(config, tensors) of a bundle: a Hugging Face style config.json dictionary (with the seedplane
    quantization_config when quantized) and CPU torch tensors under Hugging Face names (fused matrices split back
    into row views).  With verify, weights.spw must match the manifest's SHA-256."""
    import torch
    path = Path(path)
    m = read_manifest(path)
    wpath = path / m['weights']['file']
    if not wpath.is_file():
        raise FileNotFoundError(f'{wpath} is missing')
    if verify and sha256_file(wpath) != m['weights']['sha256']:
        raise ValueError(f'{wpath} does not match the SHA-256 in seedplane.json')
    blob = np.memmap(wpath, dtype=np.uint8, mode='c')
    table, arch = m['tensors'], m['arch']
    q = m.get('quantization')
    bits = q['bits'] if q else None

    def tensor(name):
        e = table.get(name)
        if e is None:
            raise ValueError(f'bundle has no tensor {name}')
        dt = _STORE.get(e['dtype'])
        if (dt is None or e['offset'] % ALIGN or e['offset'] + e['bytes'] > blob.size
                or e['bytes'] != int(np.prod(e['shape'])) * dt.itemsize):
            raise ValueError(f'bad table entry for {name}: {e}')
        return torch.from_numpy(blob[e['offset']:e['offset'] + e['bytes']].view(dt).reshape(e['shape']))

    w = {}
    for name, sources, kind in _layout(arch):
        if kind == 'vector':
            flat, at = tensor(name), 0
            for hf, n in sources:
                w[hf] = flat[at:at + n]
                at += n
            if at != flat.shape[0]:
                raise ValueError(f'{name} holds {flat.shape[0]} values, expected {at}')
            continue
        for suffix, hf_suffix, _ in _PARTS[bits]:
            whole, at = tensor(name + suffix), 0
            for hf, rows in sources:
                w[hf + hf_suffix] = whole[at:at + rows]
                at += rows
            if at != whole.shape[0]:
                raise ValueError(f'{name}{suffix} has {whole.shape[0]} rows, expected {at}')
    cfg = {'model_type': 'qwen2', 'num_hidden_layers': arch['layers'], 'hidden_size': arch['hidden'],
           'num_attention_heads': arch['heads'], 'num_key_value_heads': arch['kv_heads'],
           'intermediate_size': arch['intermediate'], 'vocab_size': arch['vocab'], 'rope_theta': arch['rope_theta'],
           'rms_norm_eps': arch['rms_norm_eps'], 'max_position_embeddings': arch['max_positions'],
           'tie_word_embeddings': arch['tied_embeddings']}
    if bits:
        cfg['quantization_config'] = {'quant_method': 'seedplane', 'bits': bits, 'group_size': q['group_size']}
    return cfg, w


def main():
    ap = argparse.ArgumentParser(description='convert a Qwen2 checkpoint into a seedplane bundle directory')
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
