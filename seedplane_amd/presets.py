"""Qwen2 architecture shapes used by the synthetic workloads, as Hugging Face config.json dictionaries.

Shapes: Qwen2-0.5B (hidden 896, 24 layers, 14/2 heads, head_dim 64, SwiGLU 4864, vocab 151936, tied head),
Qwen2-1.5B (1536, 28, 12/2, 128, 8960, 151936, tied), Qwen2-7B (3584, 28, 28/4, 128, 18944, 152064, untied);
RoPE theta 1e6 and RMSNorm eps 1e-6 for all.  `tiny` is the 2-layer test model of the reference's unit tests
(tests/test_core.py:146-165: L=2, H=128, NH=2, NKV=1, HD=64, I=256, V=50).
"""
import copy


def _cfg(layers, hidden, heads, kv_heads, inter, vocab, tie, max_pos=32768):
    return {'model_type': 'qwen2', 'num_hidden_layers': layers, 'hidden_size': hidden,
            'num_attention_heads': heads, 'num_key_value_heads': kv_heads, 'intermediate_size': inter,
            'vocab_size': vocab, 'max_position_embeddings': max_pos, 'rope_theta': 1000000.0,
            'rms_norm_eps': 1e-6, 'tie_word_embeddings': tie}


PRESETS = {
    'qwen2-0.5b': _cfg(24, 896, 14, 2, 4864, 151936, True),
    'qwen2-1.5b': _cfg(28, 1536, 12, 2, 8960, 151936, True),
    'qwen2-7b': _cfg(28, 3584, 28, 4, 18944, 152064, False),
    'tiny': _cfg(2, 128, 2, 1, 256, 50, True, max_pos=512),
}


def preset(name, **overrides):
    """A copy of a preset with keys overridden (e.g. num_hidden_layers=2 for a shortened model)."""
    c = copy.deepcopy(PRESETS[name])
    c.update(overrides)
    return c


def head_dim(cfg):
    return cfg['hidden_size'] // cfg['num_attention_heads']


def param_count(cfg):
    """Parameters read per decoded token (projections + head), excluding the embedding gather."""
    H, I, V, L = cfg['hidden_size'], cfg['intermediate_size'], cfg['vocab_size'], cfg['num_hidden_layers']
    HD = head_dim(cfg)
    NH, NKV = cfg['num_attention_heads'], cfg['num_key_value_heads']
    per_layer = (NH + 2 * NKV) * HD * H + H * NH * HD + 2 * I * H + H * I
    return L * per_layer + V * H
