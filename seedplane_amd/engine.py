"""Shard-window attention plan and its decode session over the HIP engine.

`ShardPlan` (reference: seedplane/engine.py:17-33) cuts a sequence into shards of S tokens; token i of the shard
[c0, c1) attends to the sink tokens [0, min(K, h0)), the halo [h0, c0) with h0 = max(0, c0 - H), and the shard's own
tokens up to i -- all at their ORIGINAL positions (RoPE ids), causally.

`ShardedSession` runs that rule one token at a time on a `Qwen2Engine`, as the reference native session does
(native/vulkan_decode/qwen_vk.cpp:505-565, `Session::step`).  Each window is a KV cache of its own whose slot j holds
the window's j-th token (sinks, then halo, then shard tokens) with its original RoPE position; attention covers the
window's slots [0, j].  What happens at a shard boundary is a host-side slot policy over the same kernels:

  'rebuild'  (exact)  a new window cache; the K/V of the sinks and the halo are recomputed inside it, K/V-only, as one
                      batched engine call (the reference's RebuildBatch);
  'shadow'   (exact)  from H tokens before the boundary, every token also goes into the NEXT window's cache (which
                      starts with the sinks), as a second column of the same engine call; at the boundary that cache
                      simply becomes the current one -- no recomputation (the reference's ShadowBatch).

  'reuse'    (approximate, as the reference calls it) the new window's sinks and halo are COPIES of the K/V the
                      earlier windows computed (sinks saved from the first window, the halo from the current one;
                      qwen_vk.cpp:537-542): no recomputation, but a halo token's K/V were computed under its own
                      shard's visible set, not the new window's.  Every position's K/V is then computed exactly once,
                      when it is processed, so the mode equals one causal pass in which token i attends to
                      plan.visible(i) -- what the tests check it against.  Needs halo <= shard and sinks <= shard
                      (the copied slots must lie in the current window), as the reference requires.
"""
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib


@dataclass
class ShardPlan:
    shard: int = 512      # S: tokens owned by each shard
    halo: int = 256       # H: tokens borrowed from the previous shard
    sinks: int = 4        # first tokens of the sequence visible to every shard (0 = off)

    def __post_init__(self):
        if self.shard <= 0:
            raise ValueError('shard must be greater than zero')
        if self.halo < 0:
            raise ValueError('halo must be non-negative')
        if self.sinks < 0:
            raise ValueError('sinks must be non-negative')

    def sinks_of(self, c0):
        """Sink tokens visible to the shard starting at c0 (qwen_vk.cpp:279, engine.py:31)."""
        return min(self.sinks, max(0, c0 - self.halo))

    def windows(self, L):
        """Yield (core_start, core_end, index_array): the token indices each window reads, in order."""
        if L < 0:
            raise ValueError('sequence length must be non-negative')
        for c0 in range(0, L, self.shard):
            c1 = min(L, c0 + self.shard)
            h0 = max(0, c0 - self.halo)
            yield c0, c1, np.array(list(range(self.sinks_of(c0))) + list(range(h0, c1)), dtype=np.int64)

    def visible(self, i):
        """Token indices that token i attends to (its window's prefix up to i)."""
        c0 = i - i % self.shard
        h0 = max(0, c0 - self.halo)
        return list(range(self.sinks_of(c0))) + list(range(h0, i + 1))


class ShardedSession:
    """Token-at-a-time processing under a ShardPlan on a Qwen2Engine (qwen_vk.cpp:505-565).  `step` returns the
    fp32 logits row of the token when asked for it (else None, and the token is only written to the K/V cache)."""

    MODES = ('rebuild', 'shadow', 'reuse')

    def __init__(self, engine, plan, mode='rebuild'):
        if mode not in self.MODES:
            raise ValueError(f'bad mode {mode!r} (expected one of {self.MODES})')
        if mode == 'reuse' and (plan.halo > plan.shard or plan.sinks > plan.shard):
            raise ValueError('reuse needs halo <= shard and sinks <= shard')
        self.e, self.plan, self.mode = engine, plan, mode
        self.capacity = plan.sinks + plan.halo + plan.shard
        if self.capacity > engine.config['max_position_embeddings']:
            raise ValueError(f'sinks + halo + shard = {self.capacity} exceeds the model\'s positions')
        # two window caches live at once (the current one and the next); the pool is grown for them here (growth
        # keeps every live cache of the engine)
        if engine._pool_slots < self.capacity or len(engine._free) < 2:
            engine.grow(engine._pool_n + max(0, 2 - len(engine._free)), self.capacity)
        self.seq = []                 # every token processed so far (index = original position)
        self.cur = engine.new_cache(self.capacity)
        self.shadow = None            # the next window's cache while the halo of the next shard is decoded
        self.boundaries = 0           # shard boundaries crossed
        self.extra = 0                # token columns recomputed at boundaries (rebuild)
        self.dual = 0                 # tokens written to two windows (shadow)
        self.reused = 0               # K/V slots copied at boundaries (reuse)
        self._sinks = None            # per layer (K, V) of the first min(sinks, shard) positions (reuse)
        self._row = torch.empty((2, engine.vocab), dtype=torch.float32, device=engine.device)

    @property
    def done(self):
        return len(self.seq)

    def _col(self, cache, token, pos):
        """Column appending `token` at the window's next slot, RoPE position `pos`, attending to slots [0, slot]."""
        j = cache.length
        cache.length += 1
        return (int(token), cache.seq, int(pos), j % self.e._pool_slots, 0, j, 0, 0, 0)

    def _kv_only(self, cache, items):
        """K/V of (token, position) items appended to `cache`, in engine calls of at most max_tokens columns."""
        T = self.e.max_tokens
        for c0 in range(0, len(items), T):
            self.e.run([self._col(cache, t, p) for t, p in items[c0:c0 + T]], 0)

    def _fresh(self, c0):
        """A new window cache for the shard starting at c0, holding its sinks."""
        cache = self.e.new_cache(self.capacity)
        ns = self.plan.sinks_of(c0)
        self._kv_only(cache, [(self.seq[j], j) for j in range(ns)])
        return cache

    def _reuse_window(self, i):
        """The window of the shard starting at i, filled by copies (qwen_vk.cpp:524,537-542): slots [0, ns) the
        sinks saved from the first window, slots [ns, ns + i - h0) the halo [h0, i) from the current window, where
        the current shard's tokens sit after its sinks and halo."""
        S, e = self.plan.shard, self.e
        ns, h0 = self.plan.sinks_of(i), max(0, i - self.plan.halo)
        pre = self.cur.length - S                # the current window's slots before its shard's tokens
        old = self.cur
        nxt = e.new_cache(self.capacity)         # (may grow the pool: the views below are taken after it)
        src = torch.arange(pre + h0 - (i - S), pre + S, device=e.device)
        for l in range(e.n_layers):
            kp, vp = e._kv_pool(l)
            for pool, which in ((kp, 0), (vp, 1)):
                if ns:
                    pool[nxt.seq][:, :ns] = self._sinks[l][which][:, :ns]
                pool[nxt.seq][:, ns:ns + i - h0] = pool[old.seq][:, src]
        nxt.length = ns + i - h0
        self.reused += nxt.length
        return nxt

    def _save_sinks(self):
        """K/V of the first min(sinks, shard) positions, from the first window (whose slot j holds position j)."""
        K = min(self.plan.sinks, self.plan.shard)
        self._sinks = []
        for l in range(self.e.n_layers):
            kp, vp = self.e._kv_pool(l)
            self._sinks.append((kp[self.cur.seq][:, :K].clone(), vp[self.cur.seq][:, :K].clone()))

    def step(self, token, need_logits=True):
        i, S, H = self.done, self.plan.shard, self.plan.halo
        if i > 0 and i % S == 0:
            self.boundaries += 1
            if self.mode == 'reuse':
                if self._sinks is None:
                    self._save_sinks()
                self.cur = self._reuse_window(i)
            elif self.mode == 'shadow' and self.shadow is not None:
                self.cur, self.shadow = self.shadow, None
            else:                      # rebuild (or a shadow that never started: halo 0)
                h0 = max(0, i - H)
                self.cur = self._fresh(i)
                halo = [(self.seq[j], j) for j in range(h0, i)]
                self._kv_only(self.cur, halo)
                self.extra += self.plan.sinks_of(i) + len(halo)
        if self.mode == 'shadow' and self.shadow is None and H > 0:
            nb = (i // S + 1) * S
            if i >= nb - H:
                self.shadow = self._fresh(nb)
                # a halo longer than the shard starts before this shard: its earlier tokens are added now
                back = [(self.seq[j], j) for j in range(max(0, nb - H), i)]
                self._kv_only(self.shadow, back)
                self.extra += len(back)
        self.seq.append(int(token))
        cols = [self._col(self.cur, token, i)]
        if self.shadow is not None:
            cols.append(self._col(self.shadow, token, i))
            self.dual += 1
        if not need_logits:
            self.e.run(cols, 0)
            return None
        out = self._row[:len(cols)]
        self.e.run(cols, _lib.SP_F_LOGITS, logits_out=out)
        return out[0].clone()

    def feed(self, tokens):
        """Process `tokens`; returns the logits row of the last one."""
        tokens = list(tokens)
        if not tokens:
            raise ValueError('tokens cannot be empty')
        for t in tokens[:-1]:
            self.step(t, need_logits=False)
        return self.step(tokens[-1], need_logits=True)

    def generate(self, prompt_ids, max_new_tokens=32, eos_token_id=None):
        """Greedy continuation of `prompt_ids` under the plan (argmax, first index on ties)."""
        row = self.feed(prompt_ids)
        for _ in range(max_new_tokens):
            token = int(torch.argmax(row))
            yield token
            if token == eos_token_id:
                return
            row = self.step(token)
