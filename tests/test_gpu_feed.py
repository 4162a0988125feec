"""Greedy loops with the ids fed back on the device (SP_F_FEED, decode_greedy): the same ids as decode() step by step
(bit-exact argmax ids), eos truncation with the cache rolled back to just after the eos, batches of independent
caches, and the state errors of the flag."""
import pytest
import torch

from seedplane_amd import _lib
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt
from tests.conftest import small_cfg

pytestmark = pytest.mark.gpu


def _engine(seed, fmt='q8'):
    cfg, w = make_weights(small_cfg(), fmt, seed=seed)
    return cfg, Qwen2Engine(config=cfg, tensors=w, max_tokens=8)


@pytest.mark.parametrize('graph', [False, True])
@pytest.mark.parametrize('window', [None, 16])
def test_decode_greedy_equals_stepwise(gpu_device, graph, window):
    print(f'feed graph={graph} window={window}', flush=True)
    cfg, eng = _engine(61)
    eng.reserve(2, eng.slots_for(128, window))
    ca, cb = eng.new_cache(128, window=window), eng.new_cache(128, window=window)
    prompt = random_prompt(9, cfg['vocab_size'], seed=1)
    first = eng.prefill([prompt], [ca])[0]
    assert eng.prefill([prompt], [cb])[0] == first
    steps = 37                                              # bursts of 8 and a partial one; the window wraps
    fed = eng.decode_greedy([first], [ca], steps, burst=8, graph=graph)[0]
    ref, t = [], first
    for _ in range(steps):
        t = int(eng.decode([t], [cb], graph=graph)[0])
        ref.append(t)
    assert fed == ref
    assert ca.length == cb.length


def test_decode_greedy_batch_and_eos(gpu_device):
    cfg, eng = _engine(62)
    eng.reserve(3, 96)
    prompts = [random_prompt(5 + i, cfg['vocab_size'], seed=10 + i) for i in range(3)]
    caches = [eng.new_cache(96) for _ in prompts]
    first = [int(x) for x in eng.prefill(prompts, caches)]
    lens = [c.length for c in caches]
    full = eng.decode_greedy(first, caches, 20, burst=6)
    # rerun from the same state with an eos that occurs in one of the sequences
    for c, L in zip(caches, lens):
        c.length = L
    eos = full[1][7]
    cut = eng.decode_greedy(first, caches, 20, eos_token_id=eos, burst=6)
    for seq, got, c, L in zip(full, cut, caches, lens):
        k = seq.index(eos) + 1 if eos in seq else len(seq)
        assert got == seq[:k]
        assert c.length == L + len(got)


def test_generate_greedy_matches_stepwise_decode(gpu_device):
    cfg, eng = _engine(63)
    eng.reserve(1, 128)
    prompt = random_prompt(6, cfg['vocab_size'], seed=3)
    gen = list(eng.generate(prompt, max_new_tokens=40))
    cache = eng.new_cache(128)
    t = eng.prefill([prompt], [cache])[0]
    ref = [t]
    for _ in range(39):
        t = int(eng.decode([t], [cache])[0])
        ref.append(t)
    assert gen == ref
    eos = ref[12]
    assert list(eng.generate(prompt, max_new_tokens=40, eos_token_id=eos)) == ref[:ref.index(eos) + 1]


def test_feed_needs_a_previous_argmax(gpu_device):
    cfg, eng = _engine(64)
    eng.reserve(2, 32)
    ca = eng.new_cache(32)
    col = eng._column(-1, ca, 0, 0)
    with pytest.raises(_lib.SeedPlaneError):
        eng.run([col], _lib.SP_F_LOGITS | _lib.SP_F_ARGMAX | _lib.SP_F_FEED)
    eng.run([eng._column(3, ca, 0, 0)], _lib.SP_F_LOGITS | _lib.SP_F_ARGMAX)
    cb = eng.new_cache(32)
    with pytest.raises(_lib.SeedPlaneError):                 # 2 columns fed from a 1-column argmax
        eng.run([eng._column(-1, ca, 1, 1), eng._column(-1, cb, 0, 0)], _lib.SP_F_LOGITS | _lib.SP_F_FEED)
    host = torch.empty(2, dtype=torch.int32, pin_memory=True)
    with pytest.raises(ValueError):                           # more ids than the last argmax call produced
        _lib.check(eng.lib.sp_engine_copy_ids(eng.h, 2, host.data_ptr()), eng.h)
