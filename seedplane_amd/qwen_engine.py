"""Qwen2 decoder on MI355X: the reference's `seedplane.qwen_engine` API over the HIP library.

Drop-in for seedplane/qwen_engine.py: `KVCache`, `Qwen2Engine(bundle, device, dtype)`, `.new_cache`, `.forward`,
`.sample`, `.generate`, `chat_prompt` keep their names, argument meaning and exceptions (ValueError for a non-qwen2
model, bad head configuration, empty ids, capacity overflow, position/ids length mismatch; FileNotFoundError when the
bundle has no safetensors).  Every forward pass runs in libseedplane_hip (hand-written gfx950 kernels); torch is used
for device memory and streams only.  There is no CPU path: constructing an engine without the library or without a
GPU raises.

Additions over the reference API (batch and window support the reference does not have):
  * `new_cache(capacity, window=None)`: with `window=W` the cache is a ring; a token at cache position p attends to
    positions (p - W, p] (the Hugging Face sliding-window rule) and positions may grow without bound.
  * `decode(tokens, caches)`: one batched decode step over independent sequences (ragged lengths).
  * `generate_batch(prompts, max_new_tokens)`: greedy decode of many requests as one batch.
  * `QwenEngine` is an alias of `Qwen2Engine`.
Quantized bundles (`quantization_config.quant_method == 'seedplane'`) carry int8 block-32 or int4 group-32 weights
(`<name>.qweight/.scales/.qzeros`); float bundles are run with fp16 weights.
"""
import ctypes
import json
import weakref
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np
import torch

from . import _lib
from . import native_bundle

GROUP = 32


class _KVLayers:
    """`KVCache.keys` / `KVCache.values` of a cache bound to an engine: item `l` is a copy of layer l's cached keys
    (values) in the reference's layout, fp16 [1, max(capacity, length), kv_heads, head_dim] on the GPU (reference:
    qwen_engine.py:18-29), gathered from the engine's HBM ring (position p at slot p mod n_slots).  Positions the ring
    no longer holds (older than length - n_slots, windowed caches only) and positions not yet written are zero.
    A copy, not the storage: writing it does not change the cache."""

    def __init__(self, engine, cache, which):
        self._eng, self._cache, self._which = weakref.ref(engine), weakref.ref(cache), which

    def __len__(self):
        eng = self._eng()
        return 0 if eng is None else eng.n_layers

    def __iter__(self):
        return (self[i] for i in range(len(self)))

    def __getitem__(self, layer):
        eng, cache = self._eng(), self._cache()
        if eng is None or cache is None:
            raise ValueError('the cache is no longer bound to a live engine')
        if isinstance(layer, slice):
            return [self[i] for i in range(len(self))[layer]]
        return eng._kv_copy(cache, layer, self._which)


@dataclass
class KVCache:
    """Per-sequence KV state.  The keys/values live in the engine's HBM ring ([layer][seq][kv_head][slot][head_dim],
    fp16); for a cache from `new_cache`, `keys[l]` / `values[l]` give copies of layer l's in the reference's layout
    (_KVLayers).  `length` is mutable exactly as in the reference (assigning a smaller value rolls the cache back,
    experiments/hive_scaling/benchmark_speculative.py:119,127)."""
    keys: list = field(default_factory=list)
    values: list = field(default_factory=list)
    length: int = 0
    capacity: int = 0
    window: int = None
    seq: int = -1
    epoch: int = -1

    @classmethod
    def allocate(cls, layers, capacity, kv_heads, head_dim, device, dtype):
        """Reference signature (qwen_engine.py:25-29); storage is owned by the engine, so this only records capacity."""
        return cls([], [], 0, capacity)


def _np(t):
    t = t.detach().contiguous().cpu()
    if t.dtype in (torch.float16, torch.bfloat16):
        t = t.to(torch.float16).view(torch.int16)
    return t.numpy()


def _ptr(a):
    return ctypes.c_void_p(a.ctypes.data) if a is not None else None


class Qwen2Engine:
    """Inference-only Qwen2/Qwen2.5 runtime with a persistent HBM KV cache (reference: qwen_engine.py:32-166)."""

    def __init__(self, bundle=None, device='cuda', dtype=None, max_tokens=64, config=None, tensors=None):
        if tensors is None and native_bundle.is_bundle(bundle):
            # seedplane-bundle/2 directory (seedplane.json + weights.spw, SHA-256 checked)
            self.bundle = Path(bundle)
            self.config, tensors = native_bundle.load(self.bundle)
        elif tensors is None:
            self.bundle = Path(bundle)
            self.config = json.loads((self.bundle / 'config.json').read_text())
        else:
            self.bundle = None
            self.config = dict(config)
        if self.config.get('model_type') != 'qwen2':
            raise ValueError('SeedPlane Qwen2Engine only supports model_type=qwen2')
        c = self.config
        self.n_layers = c['num_hidden_layers']
        self.n_heads = c['num_attention_heads']
        self.n_kv_heads = c['num_key_value_heads']
        self.hidden = c['hidden_size']
        self.head_dim = self.hidden // self.n_heads
        if self.hidden % self.n_heads or self.n_heads % self.n_kv_heads:
            raise ValueError('invalid Qwen2 head configuration')
        self.intermediate = c['intermediate_size']
        self.vocab = c['vocab_size']
        theta = c.get('rope_theta', c.get('rope_parameters', {}).get('rope_theta', 10000.0))
        # computed exactly as the reference (fp32 torch ops on the CPU)
        self.inv_freq = 1.0 / (theta ** (torch.arange(0, self.head_dim, 2).float() / self.head_dim))
        self.eps = c.get('rms_norm_eps', 1e-6)
        if tensors is None:
            tensors = self._read_safetensors(self.bundle)
        required = {'model.embed_tokens', 'model.norm.weight'}
        names = {k.rsplit('.', 1)[0] if not k.endswith('norm.weight') else k for k in tensors}
        if not required.issubset(names):
            raise ValueError('bundle is missing Qwen2 tensors')
        q = c.get('quantization_config') or {}
        if q.get('quant_method') == 'seedplane':
            if q.get('group_size', GROUP) != GROUP or q.get('bits') not in (8, 4):
                raise ValueError('seedplane quantization must be bits 8 or 4 with group_size 32')
            self.weight_format = _lib.SP_FMT_Q8 if q['bits'] == 8 else _lib.SP_FMT_Q4
        else:
            self.weight_format = _lib.SP_FMT_F16
        self.tied = 'lm_head.weight' not in tensors and 'lm_head.qweight' not in tensors
        self.max_tokens = int(max_tokens)

        _lib.require_gpu()
        self.device = torch.device(device if device not in ('hip', None) else 'cuda')
        if self.device.type != 'cuda':
            raise ValueError('seedplane_amd runs on a ROCm GPU device ("cuda"/"hip")')
        self.dtype = torch.float16 if dtype is None else dtype
        self.lib = _lib.load()
        self._inv = np.ascontiguousarray(self.inv_freq.numpy(), dtype=np.float32)
        desc = _lib.ModelDesc(self.n_layers, self.hidden, self.n_heads, self.n_kv_heads, self.head_dim,
                              self.intermediate, self.vocab, self.weight_format, int(self.tied), self.max_tokens,
                              float(self.eps), 0.0, self._inv.ctypes.data_as(ctypes.POINTER(ctypes.c_float)))
        h = ctypes.c_void_p()
        with torch.cuda.device(self.device):
            _lib.check(self.lib.sp_engine_create(ctypes.byref(desc), ctypes.byref(h)))
        self.h = h
        self._finalizer = weakref.finalize(self, self.lib.sp_engine_destroy, h)
        self.stream = torch.cuda.current_stream(self.device)
        _lib.check(self.lib.sp_engine_set_stream(self.h, ctypes.c_void_p(self.stream.cuda_stream)), self.h)
        self._load(tensors)
        self._pool_n = 0
        self._pool_slots = 0
        self._epoch = 0
        self._free = []
        self._live = weakref.WeakValueDictionary()     # sequence index -> its live cache
        self._logits_buf = None

    # ------------------------------------------------------------------------------------------ loading
    @staticmethod
    def _read_safetensors(bundle):
        from safetensors import safe_open
        files = sorted(Path(bundle).glob('*.safetensors'))
        if not files:
            raise FileNotFoundError(f'no safetensors in {bundle}')
        w = {}
        for filename in files:
            with safe_open(filename, framework='pt', device='cpu') as f:
                for name in f.keys():
                    if name in w:
                        raise ValueError(f'duplicate tensor {name}')
                    w[name] = f.get_tensor(name)
        return w

    def _matrix(self, w, names):
        """Concatenate the rows of `names` (reference fused packing, qwen_engine.py:71-76) in the model's format."""
        if self.weight_format == _lib.SP_FMT_F16:
            mats = [w[n + '.weight'].to(torch.float16) for n in names]
            return (_np(torch.cat(mats)), None, None)
        codes = _np(torch.cat([w[n + '.qweight'] for n in names]))
        scales = _np(torch.cat([w[n + '.scales'].to(torch.float16) for n in names]))
        zeros = None
        if self.weight_format == _lib.SP_FMT_Q4:
            zeros = _np(torch.cat([w[n + '.qzeros'].to(torch.float16) for n in names]))
        return codes, scales, zeros

    def _put_matrix(self, kind, layer, rows, cols, arrays):
        data, scales, zeros = arrays
        _lib.check(self.lib.sp_engine_load(self.h, kind, layer, self.weight_format, rows, cols, _ptr(data),
                                           _ptr(scales), _ptr(zeros)), self.h)

    def _put_vector(self, kind, layer, t):
        a = np.ascontiguousarray(t.detach().float().cpu().numpy(), dtype=np.float32)
        _lib.check(self.lib.sp_engine_load(self.h, kind, layer, _lib.SP_FMT_F32, 1, a.size, _ptr(a), None, None),
                   self.h)

    def _load(self, w):
        H, I, NH, NKV, HD = self.hidden, self.intermediate, self.n_heads, self.n_kv_heads, self.head_dim
        Nqkv = (NH + 2 * NKV) * HD
        self._put_matrix(_lib.SP_T_EMBED, 0, self.vocab, H, self._matrix(w, ['model.embed_tokens']))
        if not self.tied:
            self._put_matrix(_lib.SP_T_HEAD, 0, self.vocab, H, self._matrix(w, ['lm_head']))
        self._put_vector(_lib.SP_T_FINAL_NORM, 0, w['model.norm.weight'])
        for l in range(self.n_layers):
            p = f'model.layers.{l}.'
            self._put_vector(_lib.SP_T_IN_NORM, l, w[p + 'input_layernorm.weight'])
            self._put_vector(_lib.SP_T_POST_NORM, l, w[p + 'post_attention_layernorm.weight'])
            att = [p + 'self_attn.q_proj', p + 'self_attn.k_proj', p + 'self_attn.v_proj']
            self._put_matrix(_lib.SP_T_QKV, l, Nqkv, H, self._matrix(w, att))
            self._put_vector(_lib.SP_T_QKV_BIAS, l, torch.cat([w[n + '.bias'].float() for n in att]))
            self._put_matrix(_lib.SP_T_O, l, H, NH * HD, self._matrix(w, [p + 'self_attn.o_proj']))
            self._put_matrix(_lib.SP_T_GATE_UP, l, 2 * I, H, self._matrix(w, [p + 'mlp.gate_proj', p + 'mlp.up_proj']))
            self._put_matrix(_lib.SP_T_DOWN, l, H, I, self._matrix(w, [p + 'mlp.down_proj']))

    def weight_bytes(self):
        wb, kb = ctypes.c_uint64(), ctypes.c_uint64()
        _lib.check(self.lib.sp_engine_bytes(self.h, ctypes.byref(wb), ctypes.byref(kb)), self.h)
        return wb.value, kb.value

    def time_gemv(self, kind, layer=0, n_cols=1, iters=100):
        """Average duration (us) and packed bytes of one launch of this engine's GEMV for matrix `kind`
        (an SP_T_* constant), timed with HIP events on the engine's stream.  Clobbers activation buffers."""
        us, nb = ctypes.c_float(), ctypes.c_uint64()
        _lib.check(self.lib.sp_engine_time_gemv(self.h, kind, layer, n_cols, iters, ctypes.byref(us), ctypes.byref(nb)),
                   self.h)
        return us.value, nb.value

    def time_persistent(self, cache, iters=50):
        """Average duration (us) and algorithmic bytes of one launch of the persistent one-column step's kernel for a
        decode column of `cache` at its current length (every layer; no head, no argmax), timed with HIP events on
        the engine's stream.  Clobbers activation buffers; the column's K/V slot is rewritten with the same values."""
        col = _lib.Token(*self._column(0, cache, cache.length, cache.length))
        us, nb = ctypes.c_float(), ctypes.c_uint64()
        _lib.check(self.lib.sp_engine_time_persistent(self.h, ctypes.byref(col), iters, ctypes.byref(us),
                                                      ctypes.byref(nb)), self.h)
        return us.value, nb.value

    def time_attention(self, caches, iters=100):
        """Average duration (us) and K/V bytes of one launch of the attention kernel a decode step of `caches` (one
        column each, at their current lengths) runs, timed with HIP events on the engine's stream.  Clobbers
        activation buffers."""
        cols = [self._column(0, c, c.length, c.length) for c in caches]
        arr = (_lib.Token * len(cols))(*[_lib.Token(*c) for c in cols])
        us, nb = ctypes.c_float(), ctypes.c_uint64()
        _lib.check(self.lib.sp_engine_time_attention(self.h, len(cols), arr, iters, ctypes.byref(us), ctypes.byref(nb)),
                   self.h)
        return us.value, nb.value

    @property
    def last_dispatches(self):
        """Kernels the last engine call with graph=True launched (its recorded step), -1 after a call without it."""
        return int(self.lib.sp_engine_last_dispatches(self.h))

    def fill_cache(self, cache, n_positions, seed=0, scale=1.0):
        """Benchmark stand-in for a long prefill: positions [0, n_positions) of `cache` get seeded pseudo-random K/V
        (the decode step reads the same bytes whatever the values); cache.length = n_positions."""
        self._check_cache(cache)
        S = self._pool_slots
        if cache.window is None and n_positions > cache.capacity:
            raise ValueError(f'KV cache capacity {cache.capacity} exceeded')
        n = min(n_positions, S)
        first = (n_positions - n) % S
        if first + n <= S:
            _lib.check(self.lib.sp_engine_kv_fill(self.h, cache.seq, first, n, seed, scale), self.h)
        else:
            _lib.check(self.lib.sp_engine_kv_fill(self.h, cache.seq, first, S - first, seed, scale), self.h)
            _lib.check(self.lib.sp_engine_kv_fill(self.h, cache.seq, 0, n - (S - first), seed + 1, scale), self.h)
        cache.length = n_positions

    # ------------------------------------------------------------------------------------------ KV pool
    def reserve(self, n_seq, n_slots):
        """(Re)allocate the HBM KV pool for n_seq sequences x n_slots ring slots; invalidates existing caches."""
        _lib.check(self.lib.sp_engine_kv_reserve(self.h, int(n_seq), int(n_slots)), self.h)
        self._pool_n, self._pool_slots = int(n_seq), int(n_slots)
        self._epoch += 1
        self._free = list(range(self._pool_n))[::-1]
        self._live = weakref.WeakValueDictionary()

    def grow(self, n_seq, n_slots):
        """Grow the HBM KV pool to at least n_seq sequences x n_slots slots, keeping every live cache: its K/V moves
        to the new pool (ring slot p mod n_slots) and it stays usable, as the reference's caches are independent of
        each other (qwen_engine.py:82-85)."""
        n_seq, n_slots = max(int(n_seq), self._pool_n), max(int(n_slots), self._pool_slots)
        if self._pool_n == 0:
            self.reserve(n_seq, n_slots)
            return
        if n_seq == self._pool_n and n_slots == self._pool_slots:
            return
        live = [(s, c) for s, c in list(self._live.items()) if c.epoch == self._epoch]
        seqs = np.array([s for s, _ in live], dtype=np.int32)
        lens = np.array([c.length for _, c in live], dtype=np.int32)
        _lib.check(self.lib.sp_engine_kv_grow(self.h, n_seq, n_slots, len(live), _ptr(seqs), _ptr(lens)), self.h)
        self._free = list(range(n_seq - 1, self._pool_n - 1, -1)) + self._free
        self._pool_n, self._pool_slots = n_seq, n_slots

    def slots_for(self, capacity, window=None):
        return capacity if window is None else int(window) + self.max_tokens

    def new_cache(self, capacity=4096, window=None):
        """A fresh, empty cache (reference: qwen_engine.py:82-85).  When the pool lacks a free sequence or enough
        slots it grows, keeping every live cache."""
        capacity = min(capacity, self.config['max_position_embeddings'])
        if capacity < 1:
            raise ValueError('cache capacity must be positive')
        if window is not None and window < 1:
            raise ValueError('window must be positive')
        need = self.slots_for(capacity, window)
        if self._pool_n == 0:
            self.reserve(1, need)
        elif need > self._pool_slots or not self._free:
            self.grow(self._pool_n if self._free else 2 * self._pool_n, need)
        cache = KVCache([], [], 0, capacity, window, self._free.pop(), self._epoch)
        cache.keys, cache.values = _KVLayers(self, cache, 'k'), _KVLayers(self, cache, 'v')
        self._live[cache.seq] = cache
        weakref.finalize(cache, self._release, cache.seq, cache.epoch)
        return cache

    def _kv_pool(self, layer):
        """Layer `layer`'s K and V pools as fp16 [n_seq, kv_heads, n_slots, head_dim] tensors sharing the engine's
        memory.  Internal: valid only until the pool is reserved or grown again, so callers drop them at once."""
        k, v = ctypes.c_void_p(), ctypes.c_void_p()
        _lib.check(self.lib.sp_engine_kv_layer(self.h, layer, ctypes.byref(k), ctypes.byref(v)), self.h)
        shape = (self._pool_n, self.n_kv_heads, self._pool_slots, self.head_dim)

        def view(ptr):
            class _Pool:
                __cuda_array_interface__ = {'shape': shape, 'typestr': '<f2', 'data': (ptr.value, False),
                                            'version': 3, 'strides': None}
            return torch.as_tensor(_Pool(), device=self.device)
        return view(k), view(v)

    def _kv_copy(self, cache, layer, which):
        """Layer `layer`'s keys ('k') or values ('v') of `cache`, copied out of the HBM ring (see _KVLayers)."""
        self._check_cache(cache)
        L = self.n_layers
        if not -L <= layer < L:
            raise IndexError('layer out of range')
        kp, vp = self._kv_pool(layer % L)
        pool = kp if which == 'k' else vp
        S, NKV, HD = self._pool_slots, self.n_kv_heads, self.head_dim
        n = cache.length
        out = torch.zeros((1, max(cache.capacity, n), NKV, HD), dtype=torch.float16, device=self.device)
        first = max(0, n - S)
        if n > first:
            slots = torch.arange(first, n, device=self.device) % S
            out[0, first:n] = pool[cache.seq][:, slots].permute(1, 0, 2)
        return out

    def _release(self, seq, epoch):
        if epoch == self._epoch and seq not in self._free:
            self._free.append(seq)

    def _check_cache(self, cache):
        if cache.epoch != self._epoch:
            raise ValueError('KV cache belongs to an older reservation of this engine')

    # ------------------------------------------------------------------------------------------ forward
    def _column(self, token, cache, cpos, rope_pos):
        lo = 0 if cache.window is None else max(0, cpos - cache.window + 1)
        return (int(token), cache.seq, int(rope_pos), cpos % self._pool_slots, lo, cpos, 0, 0, 0)

    def run(self, cols, flags, logits_out=None, want_ids=False):
        """Low-level: one engine call over column tuples (token, seq, pos, slot, ctx_lo, ctx_hi, tree_base,
        tree_count, tree_mask), or a numpy array of _lib.TOKEN_DTYPE.  Returns greedy ids (numpy int32) when
        want_ids."""
        if isinstance(cols, np.ndarray):
            if cols.dtype != _lib.TOKEN_DTYPE or not cols.flags.c_contiguous:
                raise ValueError('column array must be a contiguous TOKEN_DTYPE array')
            n = len(cols)
            arr = cols.ctypes.data_as(ctypes.POINTER(_lib.Token))
        else:
            n = len(cols)
            arr = (_lib.Token * n)(*[_lib.Token(*c) for c in cols])
        return self._forward(n, arr, flags, logits_out, want_ids)

    def run_raw(self, n, cols_addr, flags, logits_out=None, want_ids=False):
        """run() over n TOKEN_DTYPE records at host address cols_addr (an int), for callers that fill the records
        in place (TreeVerifier.forward)."""
        return self._forward(n, cols_addr, flags, logits_out, want_ids)

    def _forward(self, n, arr, flags, logits_out, want_ids):
        ids = np.zeros(n, dtype=np.int32) if want_ids else None
        if want_ids:
            flags |= _lib.SP_F_ARGMAX | _lib.SP_F_LOGITS
        out = ctypes.c_void_p(logits_out.data_ptr()) if logits_out is not None else None
        _lib.check(self.lib.sp_engine_forward(self.h, n, arr, flags, out,
                                              ids.ctypes.data_as(ctypes.c_void_p) if want_ids else None), self.h)
        return ids

    @torch.inference_mode()
    def forward(self, input_ids, cache=None, all_logits=False, positions=None):
        """Run tokens through the graph (reference: qwen_engine.py:105-144).  `positions` (default: cache slots) are
        the RoPE position ids.  Returns (fp32 logits [q or 1, vocab] on the GPU, cache)."""
        ids = torch.as_tensor(input_ids, dtype=torch.long).flatten().tolist()
        if len(ids) == 0:
            raise ValueError('input_ids cannot be empty')
        if cache is None:
            cache = self.new_cache()
        self._check_cache(cache)
        start, qlen = cache.length, len(ids)
        if cache.window is None and start + qlen > cache.capacity:
            raise ValueError(f'KV cache capacity {cache.capacity} exceeded')
        slots = list(range(start, start + qlen))
        positions = slots if positions is None else torch.as_tensor(positions, dtype=torch.long).flatten().tolist()
        if len(positions) != qlen:
            raise ValueError('positions must match input_ids')
        logits = torch.empty((qlen if all_logits else 1, self.vocab), dtype=torch.float32, device=self.device)
        T = self.max_tokens
        for c0 in range(0, qlen, T):
            c1 = min(qlen, c0 + T)
            cols = [self._column(ids[i], cache, slots[i], positions[i]) for i in range(c0, c1)]
            last = c1 == qlen
            if all_logits:
                self.run(cols, _lib.SP_F_LOGITS, logits_out=logits[c0:c1])
            elif last:
                buf = self._scratch_logits(c1 - c0)
                self.run(cols, _lib.SP_F_LOGITS, logits_out=buf)
                logits[0].copy_(buf[c1 - c0 - 1])
            else:
                self.run(cols, 0)
        cache.length += qlen
        return logits, cache

    @property
    def last_path(self):
        """Which implementation ran the last engine call: 0 the kernel chain, 1 the persistent one-column step, -1
        none yet."""
        return int(self.lib.sp_engine_last_path(self.h))

    def persistent_status(self):
        """(True, '') when a plain one-column decode step on this engine's weights and KV pool runs the persistent
        kernel, else (False, the reason); the pool must be reserved."""
        buf = ctypes.create_string_buffer(256)
        rc = int(self.lib.sp_engine_persistent_status(self.h, buf, 256))
        if rc < 0:
            _lib.check(_lib.SP_EHIP, self.h)
        return rc == 1, buf.value.decode()

    def logits_view(self, n):
        """The engine's own fp32 logits of the first n columns of the last SP_F_LOGITS call, as a [n, vocab] CUDA tensor
        that shares the engine's memory (no copy; overwritten by the next forward call)."""
        if not 1 <= n <= self.max_tokens:
            raise ValueError('n must be in [1, max_tokens]')
        ptr = ctypes.c_void_p()
        _lib.check(self.lib.sp_engine_logits(self.h, ctypes.byref(ptr)), self.h)

        class _Rows:
            __cuda_array_interface__ = {'shape': (n, self.vocab), 'typestr': '<f4', 'data': (ptr.value, False),
                                        'version': 3, 'strides': None}
        return torch.as_tensor(_Rows(), device=self.device)

    def _scratch_logits(self, n):
        if self._logits_buf is None or self._logits_buf.shape[0] < n:
            self._logits_buf = torch.empty((self.max_tokens, self.vocab), dtype=torch.float32, device=self.device)
        return self._logits_buf[:n]

    @torch.inference_mode()
    def decode(self, tokens, caches, logits_out=None, graph=True):
        """One batched decode step: token i appended to caches[i] (all distinct sequences).  Returns greedy ids.
        One sequence runs the persistent one-column step where it applies (persistent_status()); otherwise the step
        runs as the kernel chain, captured as a graph when `graph`."""
        if len(tokens) != len(caches) or not tokens:
            raise ValueError('one token per cache')
        cols = []
        for t, c in zip(tokens, caches):
            self._check_cache(c)
            if c.window is None and c.length + 1 > c.capacity:
                raise ValueError(f'KV cache capacity {c.capacity} exceeded')
            cols.append(self._column(t, c, c.length, c.length))
        flags = _lib.SP_F_GRAPH if graph else 0
        ids = self.run(cols, flags, logits_out=logits_out, want_ids=True)
        for c in caches:
            c.length += 1
        return ids

    @torch.inference_mode()
    def decode_greedy(self, tokens, caches, steps, eos_token_id=None, burst=32, graph=True):
        """Greedy decode of up to `steps` tokens per cache, step i + 1 taking step i's argmax on the device
        (SP_F_FEED): no host round trip per step; the ids come back through a pinned buffer every `burst` steps.
        tokens: the next input token of each cache.  Returns one id list per cache (the ids decode() would return
        step by step).  With eos_token_id a sequence's list ends at its first eos, decoding stops once every
        sequence has one, and each cache is rolled back to just after its eos (positions decoded past it are
        dropped, as the reference rolls back by assigning `length`)."""
        n = len(tokens)
        if n != len(caches) or n == 0:
            raise ValueError('one token per cache')
        if steps <= 0:
            return [[] for _ in range(n)]
        for c in caches:
            self._check_cache(c)
            if c.window is None and c.length + steps > c.capacity:
                raise ValueError(f'KV cache capacity {c.capacity} exceeded')
        burst = max(1, min(int(burst), steps))
        ring = torch.empty((burst, n), dtype=torch.int32, pin_memory=True)
        base = ring.data_ptr()
        start = [c.length for c in caches]
        out = [[] for _ in range(n)]
        done = [False] * n
        flags = _lib.SP_F_LOGITS | _lib.SP_F_ARGMAX | (_lib.SP_F_GRAPH if graph else 0)
        step = 0
        while step < steps and not all(done):
            k = min(burst, steps - step)
            for j in range(k):
                feed = step + j > 0
                cols = [self._column(-1 if feed else int(t), c, c.length, c.length) for t, c in zip(tokens, caches)]
                self.run(cols, flags | (_lib.SP_F_FEED if feed else 0))
                _lib.check(self.lib.sp_engine_copy_ids(self.h, n, ctypes.c_void_p(base + 4 * n * j)), self.h)
                for c in caches:
                    c.length += 1
            _lib.check(self.lib.sp_engine_sync(self.h), self.h)
            ids = ring[:k].numpy()
            for j in range(k):
                for b in range(n):
                    if not done[b]:
                        t = int(ids[j, b])
                        out[b].append(t)
                        done[b] = eos_token_id is not None and t == eos_token_id
            step += k
        if eos_token_id is not None:
            for b, c in enumerate(caches):
                c.length = start[b] + len(out[b])
        return out

    # ------------------------------------------------------------------------------------------ sampling / loops
    @staticmethod
    def sample(logits, temperature=0.0, top_k=0, top_p=1.0, generator=None):
        """Reference sampling semantics (qwen_engine.py:146-156) on a logits tensor."""
        if temperature <= 0:
            return int(logits.argmax())
        z = logits / temperature
        if top_k > 0:
            cutoff = torch.topk(z, min(top_k, z.numel())).values[-1]
            z = z.masked_fill(z < cutoff, -torch.inf)
        if top_p < 1:
            values, indices = torch.sort(z, descending=True)
            probs = values.softmax(-1)
            drop = probs.cumsum(-1) - probs > top_p
            values = values.masked_fill(drop, -torch.inf)
            z = torch.full_like(z, -torch.inf).scatter(0, indices, values)
        return int(torch.multinomial(z.softmax(-1), 1, generator=generator))

    @torch.inference_mode()
    def generate(self, prompt_ids, max_new_tokens=128, temperature=0.0, top_k=0, top_p=1.0, eos_token_id=None,
                 seed=1, window=None):
        """Reference generation loop (qwen_engine.py:158-166).  Greedy decoding takes the ids from the GPU argmax."""
        cache = self.new_cache(len(prompt_ids) + max_new_tokens, window=window)
        if temperature <= 0:
            token = self._prefill_greedy(prompt_ids, cache)
            yield token
            left = max_new_tokens - 1
            # later tokens in bursts, the ids fed back on the GPU (decode_greedy); the first burst is short so the
            # first tokens arrive early
            burst = 8
            while left > 0 and token != eos_token_id:
                ids = self.decode_greedy([token], [cache], min(burst, left), eos_token_id=eos_token_id, burst=burst)[0]
                for token in ids:
                    yield token
                left -= len(ids)
                burst = min(64, burst * 2)
            return
        # T > 0: each token is drawn on the GPU (sp_op_sample_filtered: temperature, top-k, top-p, inverse CDF) with
        # the counter-based uniform u(seed, step); the reference draws from the same distribution with
        # torch.multinomial and a torch.Generator(seed), so the random streams differ
        from .speculative import uniforms
        logits, cache = self.forward(prompt_ids, cache)
        row = torch.zeros(1, dtype=torch.int32, device=self.device)
        for step in range(max_new_tokens):
            token = self.sample_gpu(logits, [0], uniforms(seed, step, 1), temperature, top_k, top_p, row)[0]
            yield token
            if token == eos_token_id:
                break
            logits, cache = self.forward([token], cache)

    def sample_gpu(self, logits, rows, u, temperature, top_k=0, top_p=1.0, rows_dev=None):
        """Filtered draws on the GPU: token s from softmax(logits[rows[s]] / T) after top-k / top-p, by inverse CDF
        with uniform u[s] (sp_op_sample_filtered).  `logits` is a 2-D fp32 CUDA tensor; returns a list of ids."""
        if temperature <= 0:
            raise ValueError('temperature must be positive (T <= 0 is the greedy argmax)')
        if logits.dim() != 2 or logits.dtype != torch.float32 or logits.device.type != 'cuda':
            raise ValueError('logits must be a 2-D fp32 GPU tensor')
        if logits.stride(1) != 1:
            raise ValueError('logits rows must be contiguous (stride 1 along the vocabulary)')
        u = np.asarray(u, dtype=np.float64).ravel()
        if rows_dev is None:
            # the kernel reads row rows[s] for every draw s: check every index before the launch
            rows = [int(r) for r in rows]
            if len(rows) != len(u):
                raise ValueError('rows and u must have the same length')
            if any(r < 0 or r >= logits.shape[0] for r in rows):
                raise ValueError('a row index is outside the logits')
        elif (rows_dev.dtype != torch.int32 or rows_dev.device != logits.device or rows_dev.dim() != 1
              or rows_dev.numel() != len(u)):
            # a device row list is the caller's to keep in range (it is not read back to the host)
            raise ValueError('rows_dev must be a 1-D int32 tensor on the logits device with one entry per draw')
        dev = logits.device
        r = rows_dev if rows_dev is not None else torch.tensor(rows, dtype=torch.int32, device=dev)
        ud = torch.as_tensor(u).to(dev, non_blocking=False)
        out = torch.empty(len(ud), dtype=torch.int32, device=dev)
        stream = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
        _lib.check(self.lib.sp_op_sample_filtered(ctypes.c_void_p(logits.data_ptr()), logits.shape[1],
                                                  logits.stride(0), ctypes.c_void_p(r.data_ptr()),
                                                  ctypes.c_void_p(ud.data_ptr()), len(ud), float(temperature),
                                                  int(top_k), float(top_p), ctypes.c_void_p(out.data_ptr()), stream))
        return out.cpu().tolist()

    def _prefill_greedy(self, prompt_ids, cache):
        ids = [int(t) for t in prompt_ids]
        if not ids:
            raise ValueError('input_ids cannot be empty')
        T = self.max_tokens
        start = cache.length
        out = None
        for c0 in range(0, len(ids), T):
            c1 = min(len(ids), c0 + T)
            cols = [self._column(ids[i], cache, start + i, start + i) for i in range(c0, c1)]
            if c1 == len(ids):
                out = int(self.run(cols, _lib.SP_F_LOGITS, want_ids=True)[-1])
            else:
                self.run(cols, 0)
        cache.length += len(ids)
        return out

    @torch.inference_mode()
    def prefill(self, prompts, caches):
        """Prefill many sequences (K/V only except the last token of each), batching columns across sequences.
        Returns the greedy next token of every sequence."""
        nxt = [None] * len(prompts)
        T = self.max_tokens
        queue = [(s, i, t) for s, p in enumerate(prompts) for i, t in enumerate(p)]
        for c0 in range(0, len(queue), T):
            chunk = queue[c0:c0 + T]
            cols = [self._column(t, caches[s], caches[s].length + i, caches[s].length + i) for s, i, t in chunk]
            ids = self.run(cols, _lib.SP_F_LOGITS, want_ids=True)
            for (s, i, _), tid in zip(chunk, ids):
                if i == len(prompts[s]) - 1:
                    nxt[s] = int(tid)
        for s, p in enumerate(prompts):
            caches[s].length += len(p)
        return nxt

    @torch.inference_mode()
    def generate_batch(self, prompts, max_new_tokens=32, eos_token_id=None, window=None, graph=True):
        """Greedy decode of independent requests as one batch (ragged prompt lengths).  Returns token lists."""
        need = max(self.slots_for(len(p) + max_new_tokens, window) for p in prompts)
        if self._pool_n == 0:
            self.reserve(len(prompts), need)
        elif len(self._free) < len(prompts) or need > self._pool_slots:
            self.grow(self._pool_n + max(0, len(prompts) - len(self._free)), need)
        caches = [self.new_cache(len(p) + max_new_tokens, window=window) for p in prompts]
        tok = self.prefill(prompts, caches)
        out = [[int(t)] for t in tok]
        live = [i for i in range(len(prompts)) if tok[i] != eos_token_id]
        if live and max_new_tokens > 1:
            ids = self.decode_greedy([out[i][-1] for i in live], [caches[i] for i in live], max_new_tokens - 1,
                                     eos_token_id=eos_token_id, graph=graph)
            for i, seq in zip(live, ids):
                out[i] += seq
        return out


QwenEngine = Qwen2Engine


def chat_prompt(messages):
    """Render Qwen's ChatML without depending on Transformers (reference: qwen_engine.py:169-172)."""
    text = ''.join(f"<|im_start|>{m['role']}\n{m['content']}<|im_end|>\n" for m in messages)
    return text + '<|im_start|>assistant\n'
