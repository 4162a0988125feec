"""Host logic of the --serve JSON-lines server (qwen_vk.cpp:810-853) over a stub engine: argument parsing, request
dispatch, the record shapes, and errors reported per request with the loop still running."""
import io
import json
import os
from pathlib import Path

import pytest

from seedplane_amd import serve


class StubEngine:
    info = {'ready': True, 'device': 'stub', 'mode': 'full', 'plan': {'shard': 64, 'halo': 0, 'sinks': 0},
            'positions': 64, 'window_slots': 64}

    def __init__(self):
        self.calls, self.last, self.seq = [], None, []

    def reset(self):
        self.calls.append(('reset',))
        self.seq = []

    def tokenize(self, text, special=True):
        return [len(w) for w in text.split()] + ([99] if special else [])

    def detokenize(self, ids, skip_special=False):
        return ' '.join(f't{i}' for i in ids if not (skip_special and i == 99))

    def state(self):
        return {'position': len(self.seq), 'processed': len(self.seq), 'tokens': list(self.seq)}

    def _events(self, kind, src, reset, sampling):
        self.calls.append((kind, src, reset, sampling))
        if src == 'boom':
            raise RuntimeError('token id 5000 out of range')
        self.seq += [7, 8]
        yield 7, 'a'
        yield 8, ''
        yield -1, 'rest'
        self.last = {'done': True, 'reason': 'stop', 'generated': 2, 'prompt_tokens': 1, 'prefill_s': 0.0,
                     'decode_s': 0.0, 'decode_tok_s': 0.0, 'position': len(self.seq)}

    def chat_events(self, content, system=None, reset=False, **sampling):
        return self._events('chat', (content, system), reset, sampling)

    def generate_events(self, text=None, ids=None, reset=True, **sampling):
        return self._events('generate', text if ids is None else tuple(ids), reset, sampling)


def _run(eng, requests):
    inp = io.StringIO(''.join((r if isinstance(r, str) else json.dumps(r, ensure_ascii=False)) + '\n'
                              for r in requests))
    out = io.StringIO()
    serve.serve(eng, inp, out)
    lines = out.getvalue().splitlines()
    assert all('": ' not in ln and ', "' not in ln for ln in lines)     # compact separators, as the C++ writer
    return [json.loads(ln) for ln in lines]


def test_ready_then_requests():
    eng = StubEngine()
    recs = _run(eng, [{'op': 'tokenize', 'text': 'ab c', 'special': True},
                      {'op': 'detokenize', 'ids': [1, 99], 'skip_special': True},
                      '', '  ',
                      {'op': 'generate', 'ids': [3], 'reset': True, 'temperature': 0.5, 'seed': 9, 'stop': [8],
                       'max_new_tokens': 4, 'top_k': None},
                      {'op': 'state'},
                      {'op': 'reset'}])
    assert recs[0] == StubEngine.info
    assert recs[1] == {'ids': [2, 1, 99]}
    assert recs[2] == {'text': 't1'}
    # the blank line is skipped; '  ' is not valid JSON and reports an error
    assert 'error' in recs[3]
    assert recs[4:7] == [{'token': 7, 'text': 'a'}, {'token': 8, 'text': ''}, {'token': -1, 'text': 'rest'}]
    assert recs[7]['done'] is True and recs[7]['reason'] == 'stop'
    assert eng.calls[0] == ('generate', (3,), True, {'temperature': 0.5, 'seed': 9, 'stop': [8], 'max_new_tokens': 4})
    assert recs[8] == {'position': 2, 'processed': 2, 'tokens': [7, 8]}
    assert recs[9] == {'ok': True}
    assert len(recs) == 10


def test_chat_defaults_and_text_generate():
    eng = StubEngine()
    _run(eng, [{'op': 'chat', 'content': 'Olá', 'reset': False},
               {'op': 'generate', 'text': 'x y'}])
    # chat: reset defaults to 0 and the server's system prompt is used when the request names none
    assert eng.calls[0] == ('chat', ('Olá', None), False, {})
    assert eng.calls[1] == ('generate', 'x y', False, {})


def test_errors_are_per_request():
    eng = StubEngine()
    recs = _run(eng, [{'op': 'bogus'}, {'op': 'generate', 'text': 'boom'}, {}, {'op': 'state'}])
    assert recs[1] == {'error': 'unknown op bogus'}
    assert recs[2] == {'error': 'token id 5000 out of range'}
    assert recs[3] == {'error': 'unknown op '}
    assert recs[4]['position'] == 0


def test_parse_args():
    b, kw = serve.parse_args(['m.sp', '--serve', '--mode', 'shadow', '--ctx', '512', '--temperature', '0.7',
                              '--top-k', '20', '--top-p', '0.9', '--seed', '3', '-n', '16', '--system', 'Be brief.'])
    assert b == 'm.sp'
    assert kw == {'mode': 'shadow', 'ctx': 512, 'temperature': 0.7, 'top_k': 20, 'top_p': 0.9, 'seed': 3,
                  'max_new_tokens': 16, 'system': 'Be brief.'}
    assert serve.parse_args(['m.sp', '--full', '--serve'])[1] == {'full': True}
    # the reference engine's logits dumps (qwen_vk.cpp:21,674): positions as a comma list, and their directory
    assert serve.parse_args(['m.sp', '--serve', '--dump-at', '3,17', '--dump-dir', '/tmp/d'])[1] == {
        'dump_at': [3, 17], 'dump_dir': '/tmp/d'}
    for bad in ([], ['m.sp'], ['m.sp', '--serve', '--bogus'], ['m.sp', '--serve', '--ctx']):
        with pytest.raises(ValueError):
            serve.parse_args(bad)


def test_main_reports_startup_failure(capsys, monkeypatch):
    monkeypatch.setenv('SEEDPLANE_NATIVE_ENGINE', serve.__file__)
    assert serve.main(['m.sp']) == 1                      # no --serve
    assert 'error:' in capsys.readouterr().err
    assert 'SEEDPLANE_NATIVE_ENGINE' not in os.environ     # it named this server, not the library


def test_server_file_is_executable():
    # the reference client starts its engine as `<path> <bundle> --serve`
    p = Path(serve.__file__)
    assert os.access(p, os.X_OK) and p.read_text().startswith('#!/usr/bin/env python3\n')
