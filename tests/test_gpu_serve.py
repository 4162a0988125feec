"""The --serve JSON-lines server (seedplane_amd/serve.py) over a pipe, driven with the reference client's request
and response shapes (seedplane/native.py:25-96; protocol qwen_vk.cpp:810-853): the server file is started as the
client starts its engine (`<engine> <bundle> --serve <flags>`, with SEEDPLANE_NATIVE_ENGINE naming it), greedy
tokens equal Qwen2Engine.generate's on the same bundle (same kernels: bit-exact), and every request kind answers
with the reference's records."""
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

from seedplane_amd import serve as serve_mod
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import random_prompt
from tests.test_gpu_native import SPECIAL, _bundle

pytestmark = pytest.mark.gpu
SERVER = Path(serve_mod.__file__).resolve()


class PipeClient:
    """The reference client's wire behaviour: one JSON request per line, records read until `done` or `error`."""

    def __init__(self, args, env, err):
        self.proc = subprocess.Popen(args, stdin=subprocess.PIPE, stdout=subprocess.PIPE, stderr=err, env=env)
        self.info = self.read()

    def read(self):
        line = self.proc.stdout.readline()
        if not line:
            raise RuntimeError(f'engine exited with {self.proc.wait()}')
        return json.loads(line.decode('utf-8'))

    def send(self, req):
        self.proc.stdin.write((json.dumps(req, ensure_ascii=False) + '\n').encode('utf-8'))
        self.proc.stdin.flush()

    def call(self, req):
        self.send(req)
        return self.read()

    def stream(self, req):
        """(token records, final record): the final record is `done` or `error`."""
        self.send(req)
        recs = []
        while True:
            r = self.read()
            if 'error' in r or r.get('done'):
                return recs, r
            recs.append(r)

    def close(self):
        self.proc.stdin.close()
        return self.proc.wait(timeout=60)


@pytest.fixture(scope='module')
def served(gpu_device, tmp_path_factory):
    tmp = tmp_path_factory.mktemp('serve')
    d, cfg, _ = _bundle(tmp, seed=21)
    env = dict(os.environ, SEEDPLANE_NATIVE_ENGINE=str(SERVER))
    args = [str(SERVER), str(d), '--serve', '--ctx', '256', '-n', '12']
    if not os.access(SERVER, os.X_OK):             # a checkout that lost the mode bit: same program, same protocol
        args = [sys.executable] + args
    print(f'serve: starting {args}', flush=True)
    with open(tmp / 'stderr.txt', 'wb') as err:
        c = PipeClient(args, env, err)
        try:
            yield c, d, cfg
        finally:
            rc = c.close()
    assert rc == 0, (tmp / 'stderr.txt').read_text()


def test_ready_record(served):
    c, _, _ = served
    assert c.info['ready'] is True and c.info['mode'] == 'full'
    assert set(c.info) == {'ready', 'device', 'mode', 'plan', 'positions', 'window_slots'}
    assert c.info['plan'] == {'shard': 256, 'halo': 0, 'sinks': 0}
    assert c.info['positions'] == 256 and c.info['window_slots'] == 256


def test_generate_records_match_engine(served):
    c, d, cfg = served
    prompt = random_prompt(9, cfg['vocab_size'] - len(SPECIAL), seed=5)
    ref = list(Qwen2Engine(d).generate(prompt, max_new_tokens=12))
    recs, done = c.stream({'op': 'generate', 'reset': True, 'ids': prompt, 'stop': []})
    assert [r['token'] for r in recs if r['token'] >= 0] == ref
    assert all(set(r) == {'token', 'text'} for r in recs)
    text = ''.join(r['text'] for r in recs)
    assert text.split() == c.call({'op': 'detokenize', 'ids': ref, 'skip_special': False})['text'].split()
    assert set(done) == {'done', 'reason', 'generated', 'prompt_tokens', 'prefill_s', 'decode_s', 'decode_tok_s',
                         'position'}
    assert done['reason'] == 'length' and done['generated'] == 12 and done['prompt_tokens'] == 9
    assert done['position'] == 21
    st = c.call({'op': 'state'})
    assert st == {'position': 21, 'processed': 20, 'tokens': prompt + ref}
    # a continuation without reset extends the session
    more = random_prompt(3, cfg['vocab_size'] - len(SPECIAL), seed=6)
    recs2, done2 = c.stream({'op': 'generate', 'reset': False, 'ids': more, 'stop': [], 'max_new_tokens': 4})
    assert done2['generated'] == 4 and done2['position'] == 21 + 3 + 4
    ref2 = list(Qwen2Engine(d).generate(prompt + ref + more, max_new_tokens=4))
    assert [r['token'] for r in recs2 if r['token'] >= 0] == ref2


def test_stop_token_record(served):
    c, d, cfg = served
    prompt = random_prompt(7, cfg['vocab_size'] - len(SPECIAL), seed=8)
    ref = list(Qwen2Engine(d).generate(prompt, max_new_tokens=12))
    stop = ref[4]
    first = ref.index(stop)
    recs, done = c.stream({'op': 'generate', 'reset': True, 'ids': prompt, 'stop': [stop]})
    toks = [r for r in recs if r['token'] >= 0]
    assert [r['token'] for r in toks] == ref[:first + 1]
    assert toks[-1]['text'] == ''                                  # a stop token's piece is empty
    assert done['reason'] == 'stop' and done['generated'] == first + 1


def test_tokenize_detokenize_chat_and_reset(served):
    c, d, cfg = served
    V = cfg['vocab_size']
    assert c.call({'op': 'tokenize', 'text': 't1 t2 <|im_end|>', 'special': True}) == {'ids': [1, 2, V - 2]}
    assert c.call({'op': 'detokenize', 'ids': [3, V - 1], 'skip_special': True}) == {'text': 't3'}
    assert c.call({'op': 'reset'}) == {'ok': True}
    assert c.call({'op': 'state'})['position'] == 0
    recs, done = c.stream({'op': 'chat', 'content': 't5 t6 t7', 'reset': False, 'max_new_tokens': 6, 'stop': []})
    assert 'error' not in done and done['generated'] == 6
    st = c.call({'op': 'state'})
    n_prompt = done['prompt_tokens']
    assert st['position'] == n_prompt + 6 and st['tokens'][0] == V - 3           # <|im_start|> opens the turn
    ref = list(Qwen2Engine(d).generate(st['tokens'][:n_prompt], max_new_tokens=6))
    assert [r['token'] for r in recs if r['token'] >= 0] == ref


def test_errors_keep_the_session(served):
    c, _, cfg = served
    assert c.call({'op': 'bogus'}) == {'error': 'unknown op bogus'}
    _, r = c.stream({'op': 'generate', 'reset': True, 'ids': [cfg['vocab_size'] + 5]})
    assert 'error' in r and 'out of range' in r['error']
    _, done = c.stream({'op': 'generate', 'reset': True, 'ids': [1, 2, 3], 'max_new_tokens': 2, 'stop': []})
    assert done['generated'] == 2


def test_context_full(served):
    c, _, cfg = served
    prompt = random_prompt(250, cfg['vocab_size'] - len(SPECIAL), seed=9)
    _, done = c.stream({'op': 'generate', 'reset': True, 'ids': prompt, 'max_new_tokens': 40, 'stop': []})
    assert done['reason'] == 'context' and done['position'] <= 257
