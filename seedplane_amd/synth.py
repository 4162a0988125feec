"""Seeded synthetic Qwen2 weights (random init; no checkpoints are available offline).

Recipes
  'f32'  : randn * 0.05, embedding x 20, norms 1, biases randn * 0.05 -- the reference's tiny_qwen2 fixture recipe
           (tests/test_core.py:146-165), fp32.
  'f16'  : weights and biases ~ N(0, 0.02) in fp16, norms 1.
  'q8'   : int8 codes uniform in [-127, 127], one fp16 scale |N(0, 0.002)| per block of 32 along K; biases
           N(0, 0.02) fp16; norms 1.  Embedding and head are quantized the same way.
  'q4'   : uint4 codes uniform in [0, 15] (two per byte, even k in the low nibble), fp16 scale |N(0, 0.002)| and fp16
           zero uniform in [7, 8) per group of 32 along K; biases N(0, 0.02); norms 1.
Tensor names follow Hugging Face Qwen2; quantized matrices use `<name>.qweight`, `.scales`, `.qzeros` and the
config carries `quantization_config = {'quant_method': 'seedplane', 'bits': 8|4, 'group_size': 32}`.

Generation is chunked: chunk c of tensor t draws from torch.Generator seeded with mix(seed, t, c), so the result is
deterministic and the chunks fill in parallel threads.
"""
import json
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

import torch

from .presets import head_dim

CHUNK = 1 << 22
GROUP = 32


def _mix(*xs):
    h = 0x9E3779B97F4A7C15
    for x in xs:
        h ^= (int(x) + 0x9E3779B97F4A7C15 + ((h << 6) & (2**64 - 1)) + (h >> 2)) & (2**64 - 1)
        h &= 2**64 - 1
    return h & (2**63 - 1)


class _Filler:
    def __init__(self, seed, threads=16):
        self.seed = seed
        self.tid = 0
        self.pool = ThreadPoolExecutor(max_workers=threads)

    def fill(self, out, fn):
        """fn(generator, n) -> flat tensor of n elements; out is filled chunk by chunk."""
        self.tid += 1
        tid = self.tid
        flat = out.view(-1)
        n = flat.numel()

        def job(c):
            lo, hi = c * CHUNK, min(n, (c + 1) * CHUNK)
            g = torch.Generator().manual_seed(_mix(self.seed, tid, c))
            flat[lo:hi] = fn(g, hi - lo)

        list(self.pool.map(job, range((n + CHUNK - 1) // CHUNK)))
        return out

    def normal(self, shape, std, dtype):
        out = torch.empty(shape, dtype=dtype)
        return self.fill(out, lambda g, n: (torch.randn(n, generator=g) * std).to(dtype))

    def abs_normal(self, shape, std, dtype):
        out = torch.empty(shape, dtype=dtype)
        return self.fill(out, lambda g, n: (torch.randn(n, generator=g) * std).abs().to(dtype))

    def randint(self, shape, lo, hi, dtype):
        out = torch.empty(shape, dtype=dtype)
        return self.fill(out, lambda g, n: torch.randint(lo, hi, (n,), generator=g, dtype=torch.int32).to(dtype))

    def uniform(self, shape, lo, hi, dtype):
        out = torch.empty(shape, dtype=dtype)
        return self.fill(out, lambda g, n: (torch.rand(n, generator=g) * (hi - lo) + lo).to(dtype))


def linear_shapes(cfg):
    """(name, out_features, in_features, has_bias) of every projection, plus the embedding/head."""
    H, I, L = cfg['hidden_size'], cfg['intermediate_size'], cfg['num_hidden_layers']
    NH, NKV, HD = cfg['num_attention_heads'], cfg['num_key_value_heads'], head_dim(cfg)
    out = [('model.embed_tokens', cfg['vocab_size'], H, False)]
    if not cfg.get('tie_word_embeddings', True):
        out.append(('lm_head', cfg['vocab_size'], H, False))
    for l in range(L):
        p = f'model.layers.{l}.'
        out += [(p + 'self_attn.q_proj', NH * HD, H, True), (p + 'self_attn.k_proj', NKV * HD, H, True),
                (p + 'self_attn.v_proj', NKV * HD, H, True), (p + 'self_attn.o_proj', H, NH * HD, False),
                (p + 'mlp.gate_proj', I, H, False), (p + 'mlp.up_proj', I, H, False),
                (p + 'mlp.down_proj', H, I, False)]
    return out


def norm_names(cfg):
    names = ['model.norm.weight']
    for l in range(cfg['num_hidden_layers']):
        names += [f'model.layers.{l}.input_layernorm.weight', f'model.layers.{l}.post_attention_layernorm.weight']
    return names


def make_weights(cfg, recipe, seed=0, threads=16, scale_std=0.002):
    """Return (config, tensors) for `recipe` in {'f32', 'f16', 'q8', 'q4'}; tensors are CPU torch tensors.
    `scale_std`: the standard deviation of the |N(0, s)| block scales of 'q8' / 'q4' (0.002 in the recipes above)."""
    cfg = dict(cfg)
    f = _Filler(seed, threads)
    w = {}
    if recipe in ('q8', 'q4'):
        cfg['quantization_config'] = {'quant_method': 'seedplane', 'bits': 8 if recipe == 'q8' else 4,
                                      'group_size': GROUP}
    for name, n, k, has_bias in linear_shapes(cfg):
        if recipe == 'f32':
            t = f.normal((n, k), 0.05, torch.float32)
            if name == 'model.embed_tokens':
                t *= 20
            w[name + '.weight'] = t
        elif recipe == 'f16':
            w[name + '.weight'] = f.normal((n, k), 0.02, torch.float16)
        elif recipe == 'q8':
            w[name + '.qweight'] = f.randint((n, k), -127, 128, torch.int8)
            w[name + '.scales'] = f.abs_normal((n, k // GROUP), scale_std, torch.float16)
        elif recipe == 'q4':
            packed = f.randint((n, k // 2), 0, 256, torch.uint8)   # two uniform nibbles per byte
            w[name + '.qweight'] = packed
            w[name + '.scales'] = f.abs_normal((n, k // GROUP), scale_std, torch.float16)
            w[name + '.qzeros'] = f.uniform((n, k // GROUP), 7.0, 8.0, torch.float16)
        else:
            raise ValueError(f'unknown recipe {recipe}')
        if has_bias:
            w[name + '.bias'] = (f.normal((n,), 0.05, torch.float32) if recipe == 'f32'
                                 else f.normal((n,), 0.02, torch.float16))
    ndt = torch.float32 if recipe == 'f32' else torch.float16
    for name in norm_names(cfg):
        w[name] = torch.ones(cfg['hidden_size'], dtype=ndt)
    f.pool.shutdown()
    return cfg, w


def write_bundle(directory, cfg, tensors):
    """Write config.json + model.safetensors (the layout Qwen2Engine(bundle) reads)."""
    from safetensors.torch import save_file
    d = Path(directory)
    d.mkdir(parents=True, exist_ok=True)
    (d / 'config.json').write_text(json.dumps(cfg))
    save_file({k: v.contiguous() for k, v in tensors.items()}, str(d / 'model.safetensors'))
    return d


def random_prompt(n, vocab, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, vocab, (n,), generator=g).tolist()
