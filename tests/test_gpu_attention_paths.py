"""The two decode attention kernels against each other on the same cache state: a batch of 32 long-context columns
(whose key splits fill the chip, so the step runs the MFMA decode kernel with split-K partials and the combine)
against the same columns decoded one at a time (64-key chunk kernel, which the oracle tests pin).  Logits within the
fp16-class tolerance, greedy ids identical where the top-2 margin exceeds it."""
import pytest
import torch

from oracle.qwen_ref import max_rel, top2_margin
from seedplane_amd.presets import preset
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt
from tests.conftest import small_cfg

pytestmark = pytest.mark.gpu
TOL = 2e-2


@pytest.mark.parametrize('shape', ['small-hd64', 'qwen2-1.5b-hd128'])
@pytest.mark.parametrize('window', [None, 1024])
def test_batch_decode_kernel_matches_chunk_kernel(gpu_device, shape, window):
    if shape == 'small-hd64':
        cfg, w = make_weights(small_cfg(), 'q8', seed=21)
    else:
        cfg, w = make_weights(preset('qwen2-1.5b', num_hidden_layers=2, vocab_size=4096), 'q8', seed=22)
    B, ctx = 32, 1100
    print(f'attention paths {shape} window={window}: {B} columns x {ctx} positions', flush=True)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=B)
    eng.reserve(B, eng.slots_for(ctx + 8, window))
    caches = [eng.new_cache(ctx + 8, window=window) for _ in range(B)]
    for i, c in enumerate(caches):
        eng.fill_cache(c, ctx, seed=300 + i, scale=0.5)
    toks = random_prompt(B, cfg['vocab_size'], seed=7)
    batch = torch.empty((B, eng.vocab), dtype=torch.float32, device=eng.device)
    ids = [int(x) for x in eng.decode(toks, caches, logits_out=batch, graph=False)]
    one = torch.empty((1, eng.vocab), dtype=torch.float32, device=eng.device)
    for i, c in enumerate(caches):
        c.length -= 1
        sid = int(eng.decode([toks[i]], [c], logits_out=one, graph=False)[0])
        assert max_rel(batch[i], one[0]) < TOL, i
        if sid != ids[i]:
            assert top2_margin(one[0]) <= TOL * float(one[0].abs().max()), i
