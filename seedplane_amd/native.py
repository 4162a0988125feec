"""In-process front end with the interface of the reference's native runtime client (seedplane/native.py).

The reference drives a separate engine process (`qwen_vk <bundle> --serve`) over JSON lines; here the engine is the
HIP library loaded into this process (seedplane_amd._lib, ctypes), so requests are method calls.  The class, its
methods, their arguments and the errors they raise are the reference's (native.py:19-96), and `info`, `last` and
`state()` keep the engine's JSON schema (qwen_vk.cpp:811-853):

    info  = {"ready", "device", "mode", "plan": {"shard", "halo", "sinks"}, "positions", "window_slots"}
    last  = {"done", "reason", "generated", "prompt_tokens", "prefill_s", "decode_s", "decode_tok_s", "position"}
    state = {"position", "processed", "tokens"}

The session keeps its token sequence and KV cache between calls (qwen_vk.cpp:500-565): a call appends its prompt,
processes the positions not yet in the cache, then generates until a stop token ("stop"), the token budget
("length") or the end of the positions ("context").  Greedy decoding takes the ids from the GPU argmax; T > 0 draws
from the GPU logits with the reference sampler semantics (Qwen2Engine.sample, qwen_engine.py:146-156).

Text needs the bundle's tokenizer.json (the HF `tokenizers` library reads it, as the reference engine reads the same
file).  Without it, generation from token ids still works: tokens are recorded in `last_tokens` and no text is
yielded; tokenize / detokenize / chat raise RuntimeError.

The attention is full over `ctx` positions unless a shard-window mode is asked for (qwen_vk.cpp:686-690): 'rebuild' /
'rebuild-batch' and 'shadow' / 'shadow-batch' run the exact boundary policies of seedplane_amd.engine.ShardedSession,
'reuse' its approximate copy policy, with the bundle's plan (seedplane.json) or the default ShardPlan.
Sampling at temperature > 0 (top-k / top-p) draws on the GPU with counter-based uniforms u(seed, draw counter).
"""
import ctypes.util
import json
import os
import time
from pathlib import Path

from . import _lib

REPO_ENGINE = _lib.LIB_PATH
_MODES = ('rebuild', 'rebuild-batch', 'shadow', 'shadow-batch', 'reuse')


def find_engine(explicit=None):
    """Engine library: explicit path, $SEEDPLANE_NATIVE_ENGINE, the in-repo build, or libseedplane_hip on the library
    search path (reference order: native.py:18-22)."""
    found = ctypes.util.find_library('seedplane_hip')
    for cand in (explicit, os.environ.get('SEEDPLANE_NATIVE_ENGINE'), REPO_ENGINE, found):
        if cand and Path(cand).is_file():
            return str(cand)
    raise FileNotFoundError('native engine not found: build it (python -m seedplane_amd.build) or set '
                            'SEEDPLANE_NATIVE_ENGINE')


def chat_turn(seq, system, user, im_end_id=None):
    """ChatML text of one user turn appended to a session holding `seq` (qwen_vk.cpp:615-620): the first turn opens
    with the system message; a later turn closes an unterminated assistant reply first."""
    tail = '<|im_start|>user\n' + user + '<|im_end|>\n<|im_start|>assistant\n'
    if not seq:
        return '<|im_start|>system\n' + system + '<|im_end|>\n' + tail
    closed = im_end_id is not None and seq[-1] == im_end_id
    return ('' if closed else '<|im_end|>') + '\n' + tail


class _TextStream:
    """Incremental detokenizer: yields the text added by each token, holding back an incomplete UTF-8 sequence."""

    def __init__(self, tok):
        self.tok, self.ids, self.out = tok, [], ''

    def push(self, t):
        if self.tok is None:
            return ''
        self.ids.append(int(t))
        text = self.tok.decode(self.ids, skip_special_tokens=False)
        if text.endswith('�'):
            return ''
        piece, self.out = text[len(self.out):], text
        return piece

    def flush(self):
        if self.tok is None or not self.ids:
            return ''
        text = self.tok.decode(self.ids, skip_special_tokens=False)
        piece, self.out = text[len(self.out):], text
        return piece


class NativeEngine:
    DEFAULT_SYSTEM = 'You are a helpful assistant.'

    def __init__(self, bundle, engine=None, mode=None, full=False, ctx=None, temperature=None, top_k=None, top_p=None,
                 seed=None, max_new_tokens=None, system=None, extra_args=(), dump_at=None, dump_dir='.'):
        import torch
        from .qwen_engine import Qwen2Engine
        path = find_engine(engine)
        if mode is not None and mode != 'full':
            if mode not in _MODES:
                raise ValueError(f'bad mode {mode!r}')
        sharded = mode not in (None, 'full') and not full
        if extra_args:
            raise ValueError(f'unknown engine arguments {list(extra_args)}')
        if _lib._lib is None:
            os.environ.setdefault('SEEDPLANE_HIP_LIB', path)
        self.bundle = Path(bundle)
        try:
            self.engine = Qwen2Engine(self.bundle)
        except (ValueError, FileNotFoundError, OSError) as ex:
            raise RuntimeError(f'engine failed to start: {ex}') from ex
        cfg = self.engine.config
        self.positions = int(min(ctx if ctx else 4096, cfg.get('max_position_embeddings', 4096)))
        self.sampling = {'temperature': 0.0 if temperature is None else float(temperature),
                         'top_k': 0 if top_k is None else int(top_k),
                         'top_p': 1.0 if top_p is None else float(top_p),
                         'seed': 1 if seed is None else int(seed)}
        self.max_new_tokens = 128 if max_new_tokens is None else int(max_new_tokens)
        self.system = self.DEFAULT_SYSTEM if system is None else system
        tj = self.bundle / 'tokenizer.json'
        self.tok = None
        if tj.is_file():
            from tokenizers import Tokenizer
            self.tok = Tokenizer.from_file(str(tj))
        self.stop_ids = self._stop_ids(cfg)
        self.im_end_id = self.tok.token_to_id('<|im_end|>') if self.tok is not None else None
        self._seq, self._done, self._cache = [], 0, None
        self._closed = False
        self._draws = 0                  # uniforms drawn so far (the counter of u(seed, counter))
        self._shard = None
        if sharded:
            from .engine import ShardPlan, ShardedSession
            from . import native_bundle
            plan = (native_bundle.read_manifest(self.bundle)['plan'] if native_bundle.is_bundle(self.bundle)
                    else {'shard': 512, 'halo': 256, 'sinks': 4})
            self._plan = ShardPlan(int(plan['shard']), int(plan['halo']), int(plan['sinks']))
            self._shard_mode = ('rebuild' if mode.startswith('rebuild') else 'reuse' if mode == 'reuse'
                                else 'shadow')
            self._shard = ShardedSession(self.engine, self._plan, self._shard_mode)
            window = self._shard.capacity
            plan_info = {'shard': self._plan.shard, 'halo': self._plan.halo, 'sinks': self._plan.sinks}
        else:
            self.engine.reserve(1, self.positions)
            window = self.positions
            plan_info = {'shard': self.positions, 'halo': 0, 'sinks': 0}
        self.info = {'ready': True, 'device': torch.cuda.get_device_name(self.engine.device),
                     'mode': mode if sharded else 'full', 'plan': plan_info, 'positions': self.positions,
                     'window_slots': window}
        self.last = None
        self.last_tokens = []
        # logits dumps (qwen_vk.cpp:891-894, --dump-at / --dump-dir): after the token at session position i is
        # processed, its fp32 logits row goes to <dump_dir>/logits_<i>.f32 (raw little-endian floats, vocab of them)
        self.dump_at = frozenset(int(i) for i in (dump_at or ()))
        self.dump_dir = Path(dump_dir)
        if self.dump_at and self._shard is not None:
            raise ValueError('--dump-at is available with full attention only')

    # ---------------------------------------------------------------------------------------------- helpers
    def _stop_ids(self, cfg):
        ids = []
        for src in (cfg.get('eos_token_id'), self._gen_cfg().get('eos_token_id')):
            if src is None:
                continue
            ids += [int(x) for x in (src if isinstance(src, list) else [src])]
        if self.tok is not None:
            for name in ('<|im_end|>', '<|endoftext|>'):
                i = self.tok.token_to_id(name)
                if i is not None:
                    ids.append(int(i))
        return sorted(set(ids))

    def _gen_cfg(self):
        p = self.bundle / 'generation_config.json'
        return json.loads(p.read_text()) if p.is_file() else {}

    def _need_tok(self):
        if self.tok is None:
            raise RuntimeError(f'{self.bundle} has no tokenizer.json')
        return self.tok

    def _live(self):
        if self._closed:
            raise RuntimeError('engine exited: closed')

    def _session_cache(self):
        if self._shard is not None:
            return None
        if self._cache is None:
            self._cache = self.engine.new_cache(self.positions)
            self._done = 0
        return self._cache

    def _stream(self, ids, reset, sampling):
        """The text pieces of _events (non-empty ones only)."""
        for _, piece in self._events(ids, reset, sampling):
            if piece:
                yield piece

    def _events(self, ids, reset, sampling):
        """Append `ids` to the session and generate (qwen_vk.cpp:589-613), yielding (token, text piece) per generated
        token (a stop token's piece is empty) and finally (-1, rest) when the incremental detokenizer held text back."""
        import torch
        self._live()
        if reset:
            self.reset()
        sp = dict(self.sampling)
        sp.update({k: v for k, v in sampling.items() if k in sp and v is not None})
        max_new = int(sampling.get('max_new_tokens') or self.max_new_tokens)
        stop = sampling.get('stop')
        stop = self.stop_ids if stop is None else [int(s) for s in stop]
        eng, cache = self.engine, self._session_cache()
        self.last_tokens, self.last = [], None
        ids = [int(i) for i in ids]
        for i in ids:
            if not 0 <= i < eng.vocab:
                raise RuntimeError(f'token id {i} out of range')
        self._seq += ids
        res = {'done': True, 'reason': 'length', 'generated': 0, 'prompt_tokens': len(ids), 'prefill_s': 0.0,
               'decode_s': 0.0, 'decode_tok_s': 0.0, 'position': 0}
        dec = _TextStream(self.tok)
        greedy = sp['temperature'] <= 0
        sh = self._shard
        t0 = time.perf_counter()
        try:
            pending = self._seq[self._done:]
            if not pending:
                raise RuntimeError('nothing to continue from: the session is empty')
            if len(self._seq) > self.positions:
                raise _ContextFull()
            start = len(self._seq) - len(pending)
            dumps = [i for i in range(start, len(self._seq)) if i in self.dump_at]
            if sh is not None:
                logits = sh.feed(pending)[None]
                nxt = int(torch.argmax(logits[0])) if greedy else None
            elif dumps:
                # every row of the call, for the rows to dump (the K/V-only prefill computes no logits)
                rows, _ = eng.forward(pending, cache, all_logits=True)
                for i in dumps:
                    self._dump(i, rows[i - start])
                logits = rows[-1:]
                nxt = int(torch.argmax(logits[0])) if greedy else None
            elif greedy:
                nxt = int(eng.prefill([pending], [cache])[0])
                logits = None
            else:
                logits, _ = eng.forward(pending, cache)
            self._done = len(self._seq)
            torch.cuda.synchronize(eng.device)
            res['prefill_s'] = time.perf_counter() - t0
            t0 = time.perf_counter()
            while True:
                t = nxt if greedy else self._draw(logits, sp)
                self._seq.append(int(t))
                res['generated'] += 1
                self.last_tokens.append(int(t))
                is_stop = int(t) in stop
                piece = '' if is_stop else dec.push(t)
                yield int(t), piece
                if is_stop:
                    res['reason'] = 'stop'
                    break
                if res['generated'] >= max_new:
                    break
                if len(self._seq) > self.positions:
                    raise _ContextFull()
                pos = len(self._seq) - 1
                if sh is not None:
                    logits = sh.step(int(t))[None]
                    nxt = int(torch.argmax(logits[0])) if greedy else None
                elif greedy and pos not in self.dump_at:
                    nxt = int(eng.decode([int(t)], [cache])[0])
                else:
                    logits, _ = eng.forward([int(t)], cache)
                    nxt = int(torch.argmax(logits[0])) if greedy else None
                    if pos in self.dump_at:
                        self._dump(pos, logits[0])
                self._done = len(self._seq)
        except _ContextFull:
            res['reason'] = 'context'
        rest = dec.flush()
        if rest:
            yield -1, rest
        torch.cuda.synchronize(eng.device)
        res['decode_s'] = time.perf_counter() - t0
        res['decode_tok_s'] = res['generated'] / max(res['decode_s'], 1e-9)
        res['position'] = len(self._seq)
        self.last = res

    # ---------------------------------------------------------------------------------------------- interface
    def chat(self, content, system=None, reset=False, **sampling):
        """One user turn; yields the assistant's text as it is generated.  The conversation stays in the engine."""
        tok = self._need_tok()
        if reset:
            self.reset()
        text = chat_turn(self._seq, self.system if system is None else system, content, self.im_end_id)
        yield from self._stream(tok.encode(text, add_special_tokens=False).ids, False, sampling)

    def generate(self, text=None, ids=None, reset=True, **sampling):
        """Raw continuation of `text` (special tokens allowed) or of token `ids`."""
        if ids is None:
            ids = self._need_tok().encode(text or '', add_special_tokens=False).ids
        yield from self._stream(list(ids), reset, sampling)

    def chat_events(self, content, system=None, reset=False, **sampling):
        """chat() as (token, text piece) events (the wire records of the --serve protocol)."""
        tok = self._need_tok()
        if reset:
            self.reset()
        text = chat_turn(self._seq, self.system if system is None else system, content, self.im_end_id)
        yield from self._events(tok.encode(text, add_special_tokens=False).ids, False, sampling)

    def generate_events(self, text=None, ids=None, reset=True, **sampling):
        """generate() as (token, text piece) events."""
        if ids is None:
            ids = self._need_tok().encode(text or '', add_special_tokens=False).ids
        yield from self._events(list(ids), reset, sampling)

    def tokenize(self, text, special=True):
        self._live()
        return self._need_tok().encode(text, add_special_tokens=bool(special)).ids

    def detokenize(self, ids, skip_special=False):
        self._live()
        return self._need_tok().decode([int(i) for i in ids], skip_special_tokens=bool(skip_special))

    def state(self):
        self._live()
        return {'position': len(self._seq), 'processed': self._done, 'tokens': list(self._seq)}

    def _dump(self, pos, row):
        self.dump_dir.mkdir(parents=True, exist_ok=True)
        row.detach().float().cpu().numpy().astype('<f4').tofile(self.dump_dir / f'logits_{pos}.f32')

    def _draw(self, logits, sp):
        """One GPU draw from the last logits row (temperature, top-k, top-p) with the next seeded uniform."""
        from .speculative import uniforms
        u = uniforms(int(sp['seed']), self._draws, 1)
        self._draws += 1
        return self.engine.sample_gpu(logits[-1:], [0], u, sp['temperature'], sp['top_k'], sp['top_p'])[0]

    def reset(self):
        self._live()
        self._seq, self._done = [], 0
        if self._shard is not None:
            from .engine import ShardedSession
            self._shard = None                     # release the old windows before the new session takes slots
            self._shard = ShardedSession(self.engine, self._plan, self._shard_mode)
        if self._cache is not None:
            self._cache.length = 0

    def close(self):
        self._closed = True
        self._cache = None

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()


class _ContextFull(Exception):
    pass
