"""ORACLE (test infrastructure): CPU fp32 restatement of the reference Qwen2 decoder.

Follows seedplane/qwen_engine.py step by step (cited per function) with three generalisations the product path
needs to be checked against:
  * an explicit boolean attention mask per query over cache positions (`forward_masked`), which reduces to the
    reference's `arange(start+q) <= slots` mask (qwen_engine.py:131-135) in `forward`;
  * an optional sliding window: query at cache position p sees positions (p - W, p] (the Hugging Face rule,
    transformers masking_utils sliding_window_overlay: kv_idx > q_idx - sliding_window);
  * weights of any synthetic recipe, dequantized to fp32 once at load (oracle/quant_ref.py);
  * a storage precision (`storage`):
      None   -- fp32 everywhere: the reference at dtype=float32, its CPU default (qwen_engine.py:39-41);
      'fp16' -- the reference at dtype=float16, its GPU default (qwen_engine.py:39-41): weights, residual stream,
                projections, RoPE cos/sin, K/V cache and attention output are fp16 tensors, the norms compute in fp32
                and cast their output (qwen_engine.py:90-92), logits are cast to fp32 (:143).  Emulated as fp32
                arithmetic rounded to fp16 after every reference op (what fp16 GEMMs with fp32 accumulation give);
      'hip'  -- fp16 at every point where a fp16-activation engine may store fp16: normalised GEMV inputs ('x', the
                union of 'xq' before qkv, 'xg' before gate_up and 'xh' before the head), K/V cache ('kv'), attention
                output ('attn'), SwiGLU activation ('act'); fp32 elsewhere (residual stream, projection outputs,
                RoPE, logits);
      a set of those point names -- fp16 at exactly those points (e.g. {'kv'}: only the K/V cache, the rounding
                a fp16 cache mandates).
The cache here is never a ring: it holds every position, and the window is applied through the mask.
"""
import math

import torch
import torch.nn.functional as F

from .quant_ref import dequant_all

HIP_POINTS = frozenset(('x', 'xq', 'xg', 'xh', 'kv', 'attn', 'act'))   # storage points a set may name


class RefCache:
    """qwen_engine.py:18-29: per-layer [1, capacity, kv_heads, head_dim] K and V plus a mutable length."""

    def __init__(self, layers, capacity, kv_heads, head_dim):
        shape = (1, capacity, kv_heads, head_dim)
        self.keys = [torch.zeros(shape) for _ in range(layers)]
        self.values = [torch.zeros(shape) for _ in range(layers)]
        self.length = 0
        self.capacity = capacity


class RefQwen2:
    def __init__(self, cfg, tensors, storage=None):
        """qwen_engine.py:35-80: config fields, inv_freq, fused qkv / gate_up packing, fp32 norms."""
        if storage in (None, 'fp16'):
            points = frozenset()
        elif storage == 'hip':
            points = HIP_POINTS
        elif isinstance(storage, (set, frozenset, tuple, list)) and set(storage) <= HIP_POINTS:
            points = frozenset(storage)
        else:
            raise ValueError(f'unknown storage {storage!r}')
        self.storage = storage if isinstance(storage, (str, type(None))) else points
        self.points = points
        self.cfg = cfg
        self.n_layers = cfg['num_hidden_layers']
        self.n_heads = cfg['num_attention_heads']
        self.n_kv_heads = cfg['num_key_value_heads']
        self.hidden = cfg['hidden_size']
        self.head_dim = self.hidden // self.n_heads
        theta = cfg.get('rope_theta', 10000.0)
        self.inv_freq = 1.0 / (theta ** (torch.arange(0, self.head_dim, 2).float() / self.head_dim))
        self.eps = cfg.get('rms_norm_eps', 1e-6)
        w = dequant_all(cfg, tensors)
        if storage == 'fp16':          # the reference casts every loaded tensor to dtype (qwen_engine.py:59)
            w = {k: v.half().float() for k, v in w.items()}
        self.embed = w['model.embed_tokens.weight']
        self.head = w.get('lm_head.weight', self.embed)
        self.final_norm = w['model.norm.weight'].float()
        self.layers = []
        for l in range(self.n_layers):
            p = f'model.layers.{l}.'
            self.layers.append({
                'in_norm': w[p + 'input_layernorm.weight'].float(),
                'post_norm': w[p + 'post_attention_layernorm.weight'].float(),
                'qkv_w': torch.cat([w[p + 'self_attn.q_proj.weight'], w[p + 'self_attn.k_proj.weight'],
                                    w[p + 'self_attn.v_proj.weight']]),
                'qkv_b': torch.cat([w[p + 'self_attn.q_proj.bias'], w[p + 'self_attn.k_proj.bias'],
                                    w[p + 'self_attn.v_proj.bias']]),
                'o_w': w[p + 'self_attn.o_proj.weight'],
                'gate_up_w': torch.cat([w[p + 'mlp.gate_proj.weight'], w[p + 'mlp.up_proj.weight']]),
                'down_w': w[p + 'mlp.down_proj.weight'],
            })

    def new_cache(self, capacity):
        return RefCache(self.n_layers, capacity, self.n_kv_heads, self.head_dim)

    def _r(self, t, *kinds):
        """Round `t` to fp16 when the storage mode stores this tensor kind in fp16 ('fp16': the reference's fp16
        tensors; a point name: that fp16-activation storage point)."""
        hit = (self.storage == 'fp16' and 'fp16' in kinds) or any(k in self.points for k in kinds)
        return t.half().float() if hit else t

    def _norm(self, x, weight, point='x'):
        """qwen_engine.py:90-92: fp32 x * rsqrt(mean(x^2) + eps), times the weight before the cast.  `point` names the
        GEMV the output feeds ('xq' qkv, 'xg' gate_up, 'xh' the head; 'x' rounds all three)."""
        xf = x.float()
        z = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        return self._r(z * weight, 'fp16', 'x', point)

    @staticmethod
    def _rotate_half(x):
        """qwen_engine.py:94-97: non-interleaved halves, cat(-x2, x1)."""
        a, b = x.chunk(2, dim=-1)
        return torch.cat((-b, a), dim=-1)

    def _rope(self, q, k, positions):
        """qwen_engine.py:99-103: phase = outer(float(pos), inv_freq), duplicated over both halves."""
        phase = torch.outer(positions.float(), self.inv_freq)
        phase = torch.cat((phase, phase), dim=-1)[None, :, None, :]
        cos, sin = self._r(phase.cos(), 'fp16'), self._r(phase.sin(), 'fp16')
        r = lambda t: self._r(t, 'fp16')
        return (r(r(q * cos) + r(self._rotate_half(q) * sin)), r(r(k * cos) + r(self._rotate_half(k) * sin)))

    @torch.inference_mode()
    def forward_masked(self, ids, cache, positions, allowed, all_logits=True):
        """One pass over `ids` written at cache positions [start, start + q); `allowed` [q, start + q] says which
        cache positions each query attends to.  Steps follow qwen_engine.py:117-144."""
        ids = torch.as_tensor(ids, dtype=torch.long).flatten()
        start, qlen = cache.length, ids.numel()
        if start + qlen > cache.capacity:
            raise ValueError(f'KV cache capacity {cache.capacity} exceeded')
        positions = torch.as_tensor(positions, dtype=torch.long).flatten()
        H, NH, NKV, HD = self.hidden, self.n_heads, self.n_kv_heads, self.head_dim
        r16 = lambda t: self._r(t, 'fp16')          # the reference's fp16 tensors
        x = F.embedding(ids, self.embed)[None]
        for l, ly in enumerate(self.layers):
            residual = x
            h = self._norm(x, ly['in_norm'], 'xq')
            qkv = r16(F.linear(h, ly['qkv_w'], ly['qkv_b']))
            q, k, v = qkv.split((H, NKV * HD, NKV * HD), dim=-1)
            q = q.view(1, qlen, NH, HD)
            k = k.view(1, qlen, NKV, HD)
            v = v.view(1, qlen, NKV, HD)
            q, k = self._rope(q, k, positions)
            cache.keys[l][:, start:start + qlen].copy_(self._r(k, 'kv'))
            cache.values[l][:, start:start + qlen].copy_(self._r(v, 'kv'))
            kk = cache.keys[l][:, :start + qlen].repeat_interleave(NH // NKV, dim=2)
            vv = cache.values[l][:, :start + qlen].repeat_interleave(NH // NKV, dim=2)
            qt, kt, vt = (z.transpose(1, 2) for z in (q, kk, vv))
            attn = self._r(F.scaled_dot_product_attention(qt, kt, vt, attn_mask=allowed), 'fp16', 'attn')
            x = r16(residual + r16(F.linear(attn.transpose(1, 2).reshape(1, qlen, H), ly['o_w'])))
            residual = x
            h = self._norm(x, ly['post_norm'], 'xg')
            gate, up = r16(F.linear(h, ly['gate_up_w'])).chunk(2, dim=-1)
            act = self._r(r16(r16(F.silu(gate)) * up), 'act')
            x = r16(residual + r16(F.linear(act, ly['down_w'])))
        cache.length += qlen
        x = self._norm(x, self.final_norm, 'xh')
        logits = r16(F.linear(x if all_logits else x[:, -1:], self.head)).float()[0]
        return logits

    def forward(self, input_ids, cache, all_logits=False, positions=None, window=None):
        """qwen_engine.py:105-144 (slot-based causal mask), optionally restricted to a sliding window."""
        ids = torch.as_tensor(input_ids, dtype=torch.long).flatten()
        if ids.numel() == 0:
            raise ValueError('input_ids cannot be empty')
        start, qlen = cache.length, ids.numel()
        slots = torch.arange(start, start + qlen)
        positions = slots if positions is None else torch.as_tensor(positions, dtype=torch.long).flatten()
        if positions.numel() != qlen:
            raise ValueError('positions must match input_ids')
        kpos = torch.arange(start + qlen)[None, :]
        allowed = kpos <= slots[:, None]
        if window is not None:
            allowed &= kpos > slots[:, None] - window
        return self.forward_masked(ids, cache, positions, allowed, all_logits)

    @staticmethod
    def greedy(logits):
        """qwen_engine.py:148: torch argmax, first index on ties."""
        return int(torch.argmax(logits))

    def generate_greedy(self, prompt_ids, max_new_tokens, window=None, capacity=None):
        """qwen_engine.py:158-166 at temperature 0: prefill, then one forward per token.  Returns (tokens, logits
        rows that produced them)."""
        cache = self.new_cache(capacity or (len(prompt_ids) + max_new_tokens))
        logits = self.forward(prompt_ids, cache, window=window)
        out, rows = [], []
        for i in range(max_new_tokens):
            tok = self.greedy(logits[-1])
            out.append(tok)
            rows.append(logits[-1].clone())
            if i + 1 < max_new_tokens:
                logits = self.forward([tok], cache, window=window)
        return out, torch.stack(rows)

    def teacher_forced(self, prompt_ids, continuation, window=None):
        """Logits after the prompt and after each forced continuation token (greedy decoding compares against
        these rows step by step)."""
        cache = self.new_cache(len(prompt_ids) + len(continuation) + 1)
        rows = [self.forward(prompt_ids, cache, window=window)[-1]]
        for t in continuation[:-1]:
            rows.append(self.forward([t], cache, window=window)[-1])
        return torch.stack(rows)


def top2_margin(row):
    v = torch.topk(row.float(), 2).values
    return float(v[0] - v[1])


def max_rel(a, b):
    """max |a - b| / max |b| (the tolerance metric used by the parity tests)."""
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


def tree_attention_mask(prefix_len, parents, window=None, depth=None):
    """allowed [n, prefix + n] for tree nodes written at cache positions prefix + i: every node sees the prefix
    (within the window of its own position prefix + depth) and its ancestors and itself."""
    n = len(parents)
    allowed = torch.zeros((n, prefix_len + n), dtype=torch.bool)
    for i in range(n):
        d = depth[i] if depth is not None else 0
        lo = 0 if window is None else max(0, prefix_len + d - window + 1)
        allowed[i, lo:prefix_len] = True
        j = i
        while j >= 0:
            allowed[i, prefix_len + j] = True
            j = parents[j]
    return allowed


def sdpa_scale(head_dim):
    return 1.0 / math.sqrt(head_dim)
