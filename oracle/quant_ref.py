"""ORACLE (test infrastructure): closed-form dequantisation of the synthetic weight formats.

int8 block-32 symmetric : w[n][k] = float32(code[n][k]) * float32(scale[n][k // 32])
int4 group-32 asymmetric: w[n][k] = (float32(code[n][k]) - float32(zero[n][k // 32])) * float32(scale[n][k // 32])
                          with code[n][2j] = byte[n][j] & 15 and code[n][2j+1] = byte[n][j] >> 4.
Both are single fp32 roundings of exact operands (int8 x fp16 products are exact in fp32).
"""
import torch

GROUP = 32


def unpack_q4(packed):
    """uint8 [N, K/2] -> int codes [N, K] (even k in the low nibble)."""
    p = packed.to(torch.int32)
    lo, hi = p & 15, p >> 4
    return torch.stack([lo, hi], dim=-1).reshape(p.shape[0], p.shape[1] * 2)


def dequant_q8(codes, scales):
    s = scales.float().repeat_interleave(GROUP, dim=1)
    return codes.float() * s


def dequant_q4(packed, scales, zeros):
    c = unpack_q4(packed).float()
    s = scales.float().repeat_interleave(GROUP, dim=1)
    z = zeros.float().repeat_interleave(GROUP, dim=1)
    return (c - z) * s


def dequant_all(cfg, tensors):
    """Float32 weights under Hugging Face names (`<name>.weight`) for any synthetic recipe."""
    q = (cfg.get('quantization_config') or {})
    bits = q.get('bits') if q.get('quant_method') == 'seedplane' else None
    out = {}
    for name, t in tensors.items():
        if name.endswith('.qweight'):
            base = name[:-len('.qweight')]
            if bits == 8:
                out[base + '.weight'] = dequant_q8(t, tensors[base + '.scales'])
            else:
                out[base + '.weight'] = dequant_q4(t, tensors[base + '.scales'], tensors[base + '.qzeros'])
        elif name.endswith('.scales') or name.endswith('.qzeros'):
            continue
        else:
            out[name] = t.float()
    return out
