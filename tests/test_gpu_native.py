"""In-process NativeEngine over the HIP engine: the reference client's interface (seedplane/native.py) on a
synthetic bundle with a word-level tokenizer.json.  Greedy tokens equal Qwen2Engine.generate's (same kernels, so
bit-exact); finish reasons, session continuation, state and the JSON fields of info / last follow qwen_vk.cpp."""
import pytest
import torch

from oracle.qwen_ref import RefQwen2, top2_margin
from seedplane_amd.native import NativeEngine
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt, write_bundle
from tests.conftest import small_cfg

pytestmark = pytest.mark.gpu
SPECIAL = ['<|im_start|>', '<|im_end|>', '<|endoftext|>']


TOL = 2e-2


def _greedy_under_oracle(ref, prefix, gen):
    """Each generated id is the oracle's argmax after prefix + gen[:i], unless the oracle's top-2 margin is within the
    fp16-class tolerance."""
    rows = ref.teacher_forced(prefix, gen)
    for i, (t, row) in enumerate(zip(gen, rows)):
        if t != int(torch.argmax(row)):
            assert top2_margin(row) <= TOL * float(row.abs().max()), f'token {i}'


def _bundle(tmp_path, fmt='q8', seed=11):
    from tokenizers import Tokenizer, models, pre_tokenizers
    cfg, w = make_weights(small_cfg(), fmt, seed=seed)
    V = cfg['vocab_size']
    vocab = {f't{i}': i for i in range(V - len(SPECIAL))}
    for j, s in enumerate(SPECIAL):
        vocab[s] = V - len(SPECIAL) + j
    cfg = dict(cfg, eos_token_id=vocab['<|endoftext|>'])
    d = write_bundle(tmp_path / 'bundle', cfg, w)
    tok = Tokenizer(models.WordLevel(vocab, unk_token='t0'))
    tok.pre_tokenizer = pre_tokenizers.WhitespaceSplit()
    tok.add_special_tokens(SPECIAL)
    tok.save(str(d / 'tokenizer.json'))
    return d, cfg, w


def test_info_and_greedy_matches_engine(gpu_device, tmp_path):
    d, cfg, _ = _bundle(tmp_path)
    prompt = random_prompt(9, cfg['vocab_size'] - len(SPECIAL), seed=2)
    ref = list(Qwen2Engine(d).generate(prompt, max_new_tokens=12))
    with NativeEngine(d, max_new_tokens=12, ctx=256) as eng:
        assert eng.info['ready'] is True and eng.info['mode'] == 'full'
        assert set(eng.info) == {'ready', 'device', 'mode', 'plan', 'positions', 'window_slots'}
        assert set(eng.info['plan']) == {'shard', 'halo', 'sinks'} and eng.info['positions'] == 256
        text = ''.join(eng.generate(ids=prompt, stop=[]))
        assert eng.last_tokens == ref
        assert text.split() == eng.tok.decode(ref, skip_special_tokens=False).split()
        last = eng.last
        assert set(last) == {'done', 'reason', 'generated', 'prompt_tokens', 'prefill_s', 'decode_s', 'decode_tok_s',
                             'position'}
        assert last['reason'] == 'length' and last['generated'] == 12 and last['prompt_tokens'] == 9
        assert last['position'] == 21
        st = eng.state()
        assert st['tokens'] == prompt + ref and st['position'] == 21 and st['processed'] == 20


def test_continuation_follows_the_oracle(gpu_device, tmp_path):
    # a second call continues the session's KV state: its tokens are the oracle's greedy continuation of the whole
    # sequence (prompt, first reply, second prompt), as a fresh prefill would give (v21/RESULTS.md:16)
    d, cfg, w = _bundle(tmp_path, seed=12)
    ref = RefQwen2(cfg, w)
    a = random_prompt(6, cfg['vocab_size'] - len(SPECIAL), seed=3)
    b = random_prompt(4, cfg['vocab_size'] - len(SPECIAL), seed=4)
    with NativeEngine(d, ctx=256) as eng:
        list(eng.generate(ids=a, max_new_tokens=5, stop=[]))
        first = list(eng.last_tokens)
        list(eng.generate(ids=b, reset=False, max_new_tokens=5, stop=[]))
        cont = list(eng.last_tokens)
        assert eng.state()['tokens'] == a + first + b + cont
    _greedy_under_oracle(ref, a, first)
    _greedy_under_oracle(ref, a + first + b, cont)


def test_stop_and_context_reasons(gpu_device, tmp_path):
    d, cfg, _ = _bundle(tmp_path, seed=13)
    prompt = random_prompt(5, cfg['vocab_size'] - len(SPECIAL), seed=5)
    with NativeEngine(d, ctx=12) as eng:
        list(eng.generate(ids=prompt, max_new_tokens=3, stop=[]))
        t0 = eng.last_tokens[0]
        list(eng.generate(ids=prompt, max_new_tokens=3, stop=[t0]))
        assert eng.last['reason'] == 'stop' and eng.last['generated'] == 1 and eng.last_tokens == [t0]
        list(eng.generate(ids=prompt, max_new_tokens=50, stop=[]))
        assert eng.last['reason'] == 'context' and eng.last['position'] <= 13
        assert eng.last['generated'] == 12 - 5 + 1


def test_tokenizer_chat_and_errors(gpu_device, tmp_path):
    d, cfg, _ = _bundle(tmp_path, seed=14)
    with NativeEngine(d, ctx=256, max_new_tokens=4) as eng:
        ids = eng.tokenize('t5 t9 <|im_end|>')
        assert ids == [5, 9, cfg['vocab_size'] - 2]
        assert eng.detokenize([5, 9]).split() == ['t5', 't9']
        list(eng.chat('t1 t2'))
        assert eng.last['generated'] >= 1 and eng.last['prompt_tokens'] > 2
        n1 = eng.state()['position']
        list(eng.chat('t3'))                                # the conversation stays in the engine
        assert eng.state()['position'] > n1
        eng.reset()
        assert eng.state() == {'position': 0, 'processed': 0, 'tokens': []}
        with pytest.raises(RuntimeError):
            list(eng.generate(ids=[cfg['vocab_size'] + 5]))
    with pytest.raises(RuntimeError):
        eng.state()                                         # closed


@pytest.mark.parametrize('mode', ['shadow-batch', 'rebuild', 'reuse'])
def test_sharded_modes_follow_the_bundle_plan(gpu_device, tmp_path, mode):
    from seedplane_amd import native_bundle
    from seedplane_amd.engine import ShardPlan, ShardedSession
    d, cfg, _ = _bundle(tmp_path)
    sp = native_bundle.convert(d, tmp_path / 'b.sp', shard=8, halo=4, sinks=2)
    prompt = random_prompt(13, cfg['vocab_size'] - len(SPECIAL), seed=4)
    plain = Qwen2Engine(tmp_path / 'b.sp', max_tokens=16)
    ref = list(ShardedSession(plain, ShardPlan(8, 4, 2), mode.split('-')[0]).generate(prompt, max_new_tokens=10))
    with NativeEngine(tmp_path / 'b.sp', mode=mode, max_new_tokens=10, ctx=256) as eng:
        assert eng.info['mode'] == mode and eng.info['plan'] == sp['plan'] and eng.info['window_slots'] == 14
        list(eng.generate(ids=prompt, stop=[]))
        assert eng.last_tokens == ref
        eng.reset()
        list(eng.generate(ids=prompt, stop=[]))
        assert eng.last_tokens == ref


def test_dump_at_writes_the_logits_rows(gpu_device, tmp_path):
    """--dump-at / --dump-dir (qwen_vk.cpp:891-894): after the token at position i is processed, logits_<i>.f32
    holds that step's fp32 logits row; positions inside the prompt and generated ones, greedy ids unchanged."""
    d, cfg, _ = _bundle(tmp_path)
    V = cfg['vocab_size']
    prompt = random_prompt(9, V - len(SPECIAL), seed=4)
    out = tmp_path / 'dumps'
    with NativeEngine(d, max_new_tokens=6, ctx=256, dump_at=[3, 8, 11], dump_dir=str(out)) as eng:
        ''.join(eng.generate(ids=prompt, stop=[]))
        gen = list(eng.last_tokens)
    seq = prompt + gen
    rows, _ = Qwen2Engine(d).forward(seq, all_logits=True)
    for j, t in enumerate(gen):                      # greedy: each id is its row's argmax up to a near-tie
        row = rows[len(prompt) - 1 + j].cpu()
        if t != int(torch.argmax(row)):
            assert top2_margin(row) <= TOL * float(row.abs().max()), j
    for i in (3, 8, 11):
        got = torch.from_numpy(__import__('numpy').fromfile(out / f'logits_{i}.f32', dtype='<f4'))
        assert got.shape == (V,)
        assert float((got - rows[i].cpu()).abs().max()) <= TOL * float(rows[i].abs().max()), i
    assert sorted(p.name for p in out.iterdir()) == ['logits_11.f32', 'logits_3.f32', 'logits_8.f32']
