"""The persistent single-column decode kernel against the CPU oracle and against the kernel chain: logits within the
fp16-class tolerance, greedy ids identical where the oracle's top-2 margin exceeds it, the KV ring shared with the
chain (either path continues the other's cache), window rule, and the real Qwen2-1.5B layer shapes (k-split
partials, 6-head groups, head_dim 128, 17 attention chunks)."""
import pytest
import torch

from oracle.qwen_ref import RefQwen2, max_rel, top2_margin
from seedplane_amd.presets import preset
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt
from tests.conftest import small_cfg

pytestmark = [pytest.mark.gpu, pytest.mark.skip(reason='the persistent decode kernel was removed: it was slower than the '
                                                 'kernel chain, and one launch of it faulted the GPU with the cause '
                                                 'not found; SP_F_PERSISTENT now runs the chain')]
TOL = 2e-2


def _decode_rows(eng, cache, tokens, persistent):
    buf = torch.empty((1, eng.vocab), dtype=torch.float32, device=eng.device)
    rows, ids = [], []
    for t in tokens:
        ids.append(int(eng.decode([t], [cache], logits_out=buf, persistent=persistent)[0]))
        assert eng.last_path == (1 if persistent else 0)
        rows.append(buf[0].clone())
    return torch.stack(rows), ids


def _check_ids(ids, ref_rows):
    for i, (t, row) in enumerate(zip(ids, ref_rows)):
        r = int(torch.argmax(row))
        if t != r:
            assert top2_margin(row) <= TOL * float(row.abs().max()), f'step {i}: {t} vs {r}'


@pytest.mark.parametrize('fmt', ['f16', 'q8', 'q4'])
@pytest.mark.parametrize('window', [None, 16])
def test_persistent_matches_oracle_and_chain(gpu_device, fmt, window):
    print(f'persistent small {fmt} window={window}', flush=True)
    cfg, w = make_weights(small_cfg(), fmt, seed=5)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=16)
    ref = RefQwen2(cfg, w)
    prompt = random_prompt(9, cfg['vocab_size'], seed=3)
    forced = random_prompt(40, cfg['vocab_size'], seed=4)     # long enough for the 16-slot window ring to wrap
    eng.reserve(2, eng.slots_for(128, window))
    ca, cb = eng.new_cache(128, window=window), eng.new_cache(128, window=window)
    eng.prefill([prompt], [ca])
    eng.prefill([prompt], [cb])
    rp, ip = _decode_rows(eng, ca, forced, persistent=True)
    rc, ic = _decode_rows(eng, cb, forced, persistent=False)
    ref_rows = ref.teacher_forced(prompt, forced + [0], window=window)[1:]
    for i in range(len(forced)):
        assert max_rel(rp[i], ref_rows[i]) < TOL, i
        assert max_rel(rp[i], rc[i]) < TOL, i
    _check_ids(ip, ref_rows)


def test_paths_share_the_cache(gpu_device):
    # alternate the two implementations on one cache: each continues what the other wrote
    cfg, w = make_weights(small_cfg(), 'q8', seed=6)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=16)
    ref = RefQwen2(cfg, w)
    prompt = random_prompt(7, cfg['vocab_size'], seed=8)
    forced = random_prompt(12, cfg['vocab_size'], seed=9)
    cache = eng.new_cache(64)
    eng.prefill([prompt], [cache])
    buf = torch.empty((1, eng.vocab), dtype=torch.float32, device=eng.device)
    ref_rows = ref.teacher_forced(prompt, forced + [0])[1:]
    for i, t in enumerate(forced):
        eng.decode([t], [cache], logits_out=buf, persistent=bool(i % 2))
        assert eng.last_path == i % 2
        assert max_rel(buf[0], ref_rows[i]) < TOL, i


def test_persistent_qwen2_1p5b_layer_shapes(gpu_device):
    # real layer shapes (2 of the 28 layers, small vocabulary): qkv / o / down split over 2 blocks each, G = 6
    cfg, w = make_weights(preset('qwen2-1.5b', num_hidden_layers=2, vocab_size=4096), 'q8', seed=2)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=16)
    ref = RefQwen2(cfg, w)
    prompt = random_prompt(12, cfg['vocab_size'], seed=5)
    forced = random_prompt(6, cfg['vocab_size'], seed=6)
    print('persistent 1.5B shapes vs oracle', flush=True)
    eng.reserve(2, 64)
    ca, cb = eng.new_cache(64), eng.new_cache(64)
    eng.prefill([prompt], [ca])
    eng.prefill([prompt], [cb])
    rp, ip = _decode_rows(eng, ca, forced, persistent=True)
    rc, _ = _decode_rows(eng, cb, forced, persistent=False)
    ref_rows = ref.teacher_forced(prompt, forced + [0])[1:]
    for i in range(len(forced)):
        assert max_rel(rp[i], ref_rows[i]) < TOL, i
        assert max_rel(rp[i], rc[i]) < TOL, i
    _check_ids(ip, ref_rows)


def test_persistent_long_window_matches_chain(gpu_device):
    # window 1024 over a 1090-position context filled with seeded K/V: 17 chunks per kv head, ring wrapped.  Each
    # step runs the persistent kernel, rolls the cache back by one and runs the chain on the same state.
    cfg, w = make_weights(preset('qwen2-1.5b', num_hidden_layers=2, vocab_size=4096), 'q8', seed=3)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=16)
    print('persistent window 1024 vs chain', flush=True)
    eng.reserve(1, eng.slots_for(1200, 1024))
    cache = eng.new_cache(1200, window=1024)
    eng.fill_cache(cache, 1090, seed=11, scale=0.5)
    bp = torch.empty((1, eng.vocab), dtype=torch.float32, device=eng.device)
    bc = torch.empty_like(bp)
    for i, t in enumerate(random_prompt(5, cfg['vocab_size'], seed=7)):
        length = cache.length
        ip = int(eng.decode([t], [cache], logits_out=bp, persistent=True)[0])
        assert eng.last_path == 1
        cache.length = length
        ic = int(eng.decode([t], [cache], logits_out=bc, persistent=False)[0])
        assert eng.last_path == 0 and cache.length == length + 1
        assert max_rel(bp[0], bc[0]) < TOL, i
        if ip != ic:
            assert top2_margin(bc[0]) <= TOL * float(bc[0].abs().max())
