#!/usr/bin/env python3
"""JSON-lines engine server with the protocol of the reference's native engine (`qwen_vk <bundle> --serve`,
native/vulkan_decode/qwen_vk.cpp:810-853), over the HIP engine of this package.

    python -m seedplane_amd.serve <bundle> --serve [--mode M] [--full] [--ctx N] [--temperature T] [--top-k K]
                                             [--top-p P] [--seed S] [-n N] [--system TEXT]

The file is also an executable engine for the reference's own client (seedplane/native.py:25-96): that client runs
`<engine> <bundle> --serve <flags>`, so pointing it at this file (SEEDPLANE_NATIVE_ENGINE=<path of this file>) makes
it drive the HIP engine unchanged.

Wire format (one JSON object per line; compact separators):
  startup   {"ready":true,"device":...,"mode":...,"plan":{"shard","halo","sinks"},"positions":...,"window_slots":...}
  requests  {"op":"reset"} -> {"ok":true}
            {"op":"tokenize","text":...,"special":1} -> {"ids":[...]}
            {"op":"detokenize","ids":[...],"skip_special":0} -> {"text":...}
            {"op":"state"} -> {"position":...,"processed":...,"tokens":[...]}
            {"op":"chat","content":...,"system":...,...} / {"op":"generate","ids":[...] | "text":...,...}
                with "reset", "temperature", "top_k", "top_p", "seed", "stop":[ids], "max_new_tokens"
                -> {"token":t,"text":piece} per generated token ({"token":-1,"text":rest} for held-back text),
                   then {"done":true,"reason":"stop"|"length"|"context","generated","prompt_tokens","prefill_s",
                         "decode_s","decode_tok_s","position"}
  failures  {"error":message} (the request is dropped; the session stays usable)
The process exits when its input ends.
"""
import json
import os
import sys

if __package__ in (None, ''):                   # run as a file (the reference client's engine path)
    from pathlib import Path
    sys.path[0] = str(Path(__file__).resolve().parents[1])     # the package's parent, not the package directory
    from seedplane_amd.native import NativeEngine
else:
    from .native import NativeEngine

_FLAGS = {'--mode': 'mode', '--ctx': 'ctx', '--temperature': 'temperature', '--top-k': 'top_k', '--top-p': 'top_p',
          '--seed': 'seed', '-n': 'max_new_tokens', '--system': 'system', '--dump-at': 'dump_at',
          '--dump-dir': 'dump_dir'}
_CONVERT = {'ctx': int, 'temperature': float, 'top_k': int, 'top_p': float, 'seed': int, 'max_new_tokens': int,
            'dump_at': lambda v: [int(x) for x in v.split(',') if x]}
_SAMPLING = ('temperature', 'top_k', 'top_p', 'seed')


def parse_args(argv):
    """(bundle, NativeEngine keyword arguments) from the reference engine's command line (qwen_vk.cpp:665-688)."""
    if not argv:
        raise ValueError('usage: serve <bundle> --serve [--mode M] [--full] [--ctx N] [--temperature T] [--top-k K] '
                         '[--top-p P] [--seed S] [-n N] [--system TEXT] [--dump-at p1,p2 --dump-dir d]')
    bundle, kw, serve, i = argv[0], {}, False, 1
    while i < len(argv):
        a = argv[i]
        if a == '--serve':
            serve = True
        elif a == '--full':
            kw['full'] = True
        elif a in _FLAGS:
            if i + 1 >= len(argv):
                raise ValueError(f'missing value for {a}')
            key = _FLAGS[a]
            i += 1
            kw[key] = _CONVERT.get(key, str)(argv[i])
        else:
            raise ValueError(f'unknown argument {a}')
        i += 1
    if not serve:
        raise ValueError('this engine speaks the --serve protocol only')
    return bundle, kw


def _line(obj, out):
    out.write(json.dumps(obj, separators=(',', ':'), ensure_ascii=False) + '\n')
    out.flush()


def handle(eng, q, out):
    """One request: its records go to `out`; an exception becomes the caller's error record."""
    op = q.get('op', '')
    if op == 'reset':
        eng.reset()
        _line({'ok': True}, out)
    elif op == 'tokenize':
        _line({'ids': eng.tokenize(q.get('text', ''), bool(q.get('special', 1)))}, out)
    elif op == 'detokenize':
        _line({'text': eng.detokenize(q.get('ids', []), bool(q.get('skip_special', 0)))}, out)
    elif op == 'state':
        _line(eng.state(), out)
    elif op in ('chat', 'generate'):
        sampling = {k: q[k] for k in _SAMPLING if q.get(k) is not None}
        if q.get('stop') is not None:
            sampling['stop'] = [int(t) for t in q['stop']]
        if q.get('max_new_tokens') is not None:
            sampling['max_new_tokens'] = int(q['max_new_tokens'])
        reset = bool(q.get('reset', 0))
        if op == 'chat':
            events = eng.chat_events(q.get('content', ''), system=q.get('system'), reset=reset, **sampling)
        elif 'ids' in q:
            events = eng.generate_events(ids=[int(t) for t in q['ids']], reset=reset, **sampling)
        else:
            events = eng.generate_events(text=q.get('text', ''), reset=reset, **sampling)
        for t, piece in events:
            _line({'token': t, 'text': piece}, out)
        _line(eng.last, out)
    else:
        raise ValueError(f'unknown op {op}')


def serve(eng, inp, out):
    """The request loop: startup record, then one request per input line until the input ends."""
    _line(eng.info, out)
    for line in inp:
        line = line.rstrip('\r\n')
        if not line:
            continue
        try:
            handle(eng, json.loads(line), out)
        except Exception as ex:                  # every failure is reported on the wire, as the reference engine does
            _line({'error': str(ex)}, out)


def main(argv=None):
    argv = sys.argv[1:] if argv is None else argv
    env = os.environ.get('SEEDPLANE_NATIVE_ENGINE')
    if env and os.path.realpath(env) == os.path.realpath(__file__):
        # the reference client names its engine executable here; this server's library is found without it
        del os.environ['SEEDPLANE_NATIVE_ENGINE']
    try:
        bundle, kw = parse_args(argv)
        eng = NativeEngine(bundle, **kw)
    except Exception as ex:
        print(f'error: {ex}', file=sys.stderr, flush=True)
        return 1
    try:
        serve(eng, sys.stdin, sys.stdout)
    finally:
        eng.close()
    return 0


if __name__ == '__main__':
    sys.exit(main())
