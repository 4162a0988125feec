"""Single-column steps with the RMSNorms run as prologues of the qkv / gate_up GEMVs and the attention combine as the
prologue of o_proj, against the same steps with every norm and combine as a kernel of its own (SP_F_UNFUSED).  The
prologues repeat the standalone kernels' arithmetic operation by operation, so logits and greedy ids must be
bit-identical.  Covers f16 / q8 / q4 weights, head_dim 64 and 128, layer 0 (no pending residual slices) and k-split
residual slices, o_proj k-slices that cut a head in two, 1 to 18 attention chunks (two batches of chunk loads in the
combine), the window ring, and graph replay.  The unfused step is pinned to the CPU oracle by the other tests."""
import pytest
import torch

from seedplane_amd import _lib
from seedplane_amd.presets import preset
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt
from tests.conftest import small_cfg

pytestmark = pytest.mark.gpu


def _step(eng, cache, tok, flags, buf):
    col = eng._column(tok, cache, cache.length, cache.length)
    tid = int(eng.run([col], flags, logits_out=buf, want_ids=True)[0])
    cache.length += 1
    return tid


def _compare(eng, cache, tokens, graph):
    """Each token through the unfused step, then (cache rolled back: the step rewrites the same slot) the fused one,
    both as the kernel chain (a plain one-column step would otherwise take the persistent kernel)."""
    base = (_lib.SP_F_GRAPH if graph else 0) | _lib.SP_F_CHAIN
    ba = torch.empty((1, eng.vocab), dtype=torch.float32, device=eng.device)
    bb = torch.empty_like(ba)
    for i, t in enumerate(tokens):
        ib = _step(eng, cache, t, base | _lib.SP_F_UNFUSED, bb)
        cache.length -= 1
        ia = _step(eng, cache, t, base, ba)
        assert ia == ib, f'step {i}: fused id {ia}, unfused id {ib}'
        assert torch.equal(ba, bb), f'step {i}: max |diff| {float((ba - bb).abs().max())}'


@pytest.mark.parametrize('shape,fmt', [('small', 'f16'), ('small', 'q8'), ('small', 'q4'),
                                       ('qwen2-1.5b', 'q8'), ('qwen2-1.5b', 'q4')])
@pytest.mark.parametrize('graph', [False, True])
def test_fused_step_is_bit_identical(gpu_device, shape, fmt, graph):
    print(f'fusion {shape} {fmt} graph={graph}', flush=True)
    if shape == 'small':
        cfg, w = make_weights(small_cfg(), fmt, seed=41)
        window = 16
    else:
        cfg, w = make_weights(preset('qwen2-1.5b', num_hidden_layers=2, vocab_size=4096), fmt, seed=42)
        window = 1024
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=4)
    eng.reserve(1, eng.slots_for(64, window))
    cache = eng.new_cache(64, window=window)
    eng.prefill([random_prompt(7, cfg['vocab_size'], seed=1)], [cache])
    # 30 steps: the 16-slot window of the small shape wraps
    _compare(eng, cache, random_prompt(30, cfg['vocab_size'], seed=2), graph)


def test_fused_step_long_context(gpu_device):
    """1100 cached positions of the Qwen2-1.5B layer shapes: 18 attention chunks per head in the combine prologue."""
    print('fusion qwen2-1.5b q8 1100 positions', flush=True)
    cfg, w = make_weights(preset('qwen2-1.5b', num_hidden_layers=2, vocab_size=4096), 'q8', seed=43)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=4)
    eng.reserve(1, eng.slots_for(1200, None))
    cache = eng.new_cache(1200)
    eng.fill_cache(cache, 1100, seed=9, scale=0.5)
    _compare(eng, cache, random_prompt(6, cfg['vocab_size'], seed=3), graph=True)


def test_unfused_flag_only_changes_launches(gpu_device):
    """A batch step ignores SP_F_UNFUSED (it never folds): the flag must not change its results."""
    cfg, w = make_weights(small_cfg(), 'q8', seed=44)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=4)
    eng.reserve(1, 64)
    cache = eng.new_cache(64)
    cols = [eng._column(t, cache, i, i) for i, t in enumerate(random_prompt(3, cfg['vocab_size'], seed=4))]
    ba = torch.empty((3, eng.vocab), dtype=torch.float32, device=eng.device)
    bb = torch.empty_like(ba)
    eng.run(cols, _lib.SP_F_LOGITS, logits_out=ba)
    eng.run(cols, _lib.SP_F_LOGITS | _lib.SP_F_UNFUSED, logits_out=bb)
    assert torch.equal(ba, bb)
