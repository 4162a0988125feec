"""The persistent one-column decode step (one cooperative kernel for every layer, then the head GEMV and the argmax)
against the CPU oracle and against the kernel chain on the same cache state:
  * small models in fp16, int8 and int4 whose 16-slot window ring wraps during the run (30 steps), each step run
    through the chain (SP_F_CHAIN), rolled back, and run again through the persistent step;
  * the Qwen2-1.5B layer shapes (2 layers, 4096-entry vocabulary) in int8 and int4 at 1100 cached positions past the
    1024 window (17 attention chunks per kv head, the ring wrapped), logits vs the oracle's windowed forward;
  * the device-side greedy feed (generate) through the persistent step equals step-by-step decoding;
  * where it does not apply (a 7B-shaped hidden size, an explicit SP_F_CHAIN) the chain runs, and the engine says why.
Bars: logits max-rel 2e-2 against the oracle (the fp16 bar); against the chain 5e-3 (both carry fp32-class GEMV inputs;
they differ in reduction orders and in the chain's fp16 attention output); greedy ids equal wherever the top-2 margin
exceeds the bar."""
import pytest
import torch

from oracle.qwen_ref import RefQwen2, max_rel
from seedplane_amd import _lib
from seedplane_amd.presets import preset
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt
from tests.conftest import small_cfg
from tests.parity import TOL, check_greedy, check_rows

pytestmark = pytest.mark.gpu


def _step(eng, cache, tok, flags, buf):
    col = eng._column(tok, cache, cache.length, cache.length)
    tid = int(eng.run([col], flags, logits_out=buf, want_ids=True)[0])
    cache.length += 1
    return tid


@pytest.mark.parametrize('fmt', ['f16', 'q8', 'q4'])
def test_small_models_persistent_vs_chain_and_oracle(gpu_device, fmt):
    print(f'persistent step: small {fmt}', flush=True)
    cfg, w = make_weights(small_cfg(), fmt, seed=41)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=4)
    window = 16
    eng.reserve(1, eng.slots_for(64, window))
    ok, why = eng.persistent_status()
    assert ok, why
    cache = eng.new_cache(64, window=window)
    prompt = random_prompt(7, cfg['vocab_size'], seed=1)
    eng.prefill([prompt], [cache])
    toks = random_prompt(30, cfg['vocab_size'], seed=2)
    V = cfg['vocab_size']
    pa = torch.empty((len(toks), V), dtype=torch.float32, device=eng.device)
    pc = torch.empty_like(pa)
    for i, t in enumerate(toks):
        _step(eng, cache, t, _lib.SP_F_CHAIN, pc[i:i + 1])
        assert eng.last_path == 0
        cache.length -= 1
        _step(eng, cache, t, 0, pa[i:i + 1])
        assert eng.last_path == 1, f'step {i} did not run the persistent kernel'
    worst_chain = max(max_rel(pa[i], pc[i]) for i in range(len(toks)))
    ref = RefQwen2(cfg, w)
    rc = ref.new_cache(len(prompt) + len(toks))
    ref.forward(prompt, rc, window=window)
    ref_rows = ref.forward(toks, rc, all_logits=True, window=window)
    worst = check_rows(pa.cpu(), ref_rows, what=f'persistent {fmt}')
    print(f'persistent {fmt}: max-rel vs oracle {worst:.2e}, vs chain {worst_chain:.2e}', flush=True)
    assert worst_chain < 5e-3


@pytest.mark.parametrize('fmt', ['q8', 'q4'])
def test_15b_layer_shapes_past_the_window(gpu_device, fmt):
    print(f'persistent step: 1.5B layer shapes {fmt}, 1100 positions', flush=True)
    cfg, w = make_weights(preset('qwen2-1.5b', num_hidden_layers=2, vocab_size=4096), fmt, seed=42)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    W, steps = 1024, 12
    V = cfg['vocab_size']
    prompt = random_prompt(1100, V, seed=3)
    cache = eng.new_cache(4096, window=W)
    assert eng.persistent_status()[0], eng.persistent_status()[1]
    lg, cache = eng.forward(prompt, cache)
    rows = torch.empty((steps, V), dtype=torch.float32, device=eng.device)
    rows[0].copy_(lg[0])
    ids = [int(lg[0].argmax())]
    for s in range(1, steps):
        ids.append(int(eng.decode([ids[-1]], [cache], logits_out=rows[s:s + 1])[0]))
        assert eng.last_path == 1
    ref = RefQwen2(cfg, w)
    rc = ref.new_cache(len(prompt) + steps)
    ref_rows = torch.cat([ref.forward(prompt, rc, window=W)[-1:], ref.forward(ids[:-1], rc, all_logits=True, window=W)])
    worst = check_rows(rows.cpu(), ref_rows, what=f'1.5b layers {fmt}')
    same = check_greedy(ids, ref_rows, what=f'1.5b layers {fmt}')
    print(f'persistent 1.5b layers {fmt}: max-rel {worst:.2e}, {same}/{steps} ids', flush=True)


def test_feed_loop_equals_stepwise(gpu_device):
    print('persistent step: device-side feed', flush=True)
    cfg, w = make_weights(small_cfg(), 'q8', seed=5)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=4)
    prompt = random_prompt(9, cfg['vocab_size'], seed=6)
    fed = list(eng.generate(prompt, 24))
    assert eng.last_path == 1
    cache = eng.new_cache(64)
    lg, cache = eng.forward(prompt, cache)
    ids = [int(lg[0].argmax())]
    for _ in range(23):
        ids.append(int(eng.decode([ids[-1]], [cache])[0]))
    assert fed == ids


def test_chain_where_the_step_does_not_apply(gpu_device):
    cfg, w = make_weights(small_cfg(hidden_size=2304, num_attention_heads=18, num_key_value_heads=3,
                                    intermediate_size=512), 'q8', seed=7)      # hidden 2304 > the step's 2048
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=4)
    eng.reserve(1, 64)
    ok, why = eng.persistent_status()
    assert not ok and why
    cache = eng.new_cache(32)
    lg, cache = eng.forward(random_prompt(5, cfg['vocab_size'], seed=8), cache)
    eng.decode([1], [cache])
    assert eng.last_path == 0


def test_step_argmax_takes_the_first_of_equal_logits(gpu_device):
    """The full 151936-entry vocabulary through the persistent step, its head GEMV and the two-pass argmax: the id
    equals torch's first-index argmax of the step's logits, and with the winning head row copied to a row of another
    16-row unit (another head block) the two logits are bit-equal and the lower row wins (torch.argmax and
    sampler.hpp:98-99 keep the first maximal index)."""
    print('persistent step: argmax ties, full vocabulary', flush=True)
    cfg, w = make_weights(preset('qwen2-1.5b', num_hidden_layers=2), 'q8', seed=45)
    V = cfg['vocab_size']
    prompt = random_prompt(5, V, seed=3)

    def one_step(tensors):
        eng = Qwen2Engine(config=cfg, tensors=tensors, max_tokens=4)
        eng.reserve(1, eng.slots_for(64, None))
        cache = eng.new_cache(64)
        eng.prefill([prompt], [cache])
        buf = torch.empty((1, V), dtype=torch.float32, device=eng.device)
        tid = _step(eng, cache, 7, 0, buf)
        assert eng.last_path == 1
        return tid, buf[0].cpu()

    tid, row = one_step(w)
    assert tid == int(torch.argmax(row))
    head = 'lm_head' if 'lm_head.qweight' in w else 'model.embed_tokens'
    # a row of another 16-row unit, below the winner when there is room (it must then win), else above (it must lose)
    k = tid // 2 if tid >= 32 else tid + 1000
    w2 = dict(w)
    for part in ('qweight', 'scales'):
        t = w[f'{head}.{part}'].clone()
        t[k] = t[tid]
        w2[f'{head}.{part}'] = t
    tid2, row2 = one_step(w2)
    assert float(row2[k]) == float(row2[tid])
    assert tid2 == min(k, tid) == int(torch.argmax(row2))
