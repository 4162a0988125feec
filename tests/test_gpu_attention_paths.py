"""The batch decode attention kernels against the single-column one on the same cache state: a batch of 32 columns
against the same columns decoded one at a time (64-key chunk kernel with RoPE fused, which the oracle tests pin).
At 1100 positions (18 chunks, 5 decode splits per column and kv head) the batch runs the multi-query MFMA kernel,
one group per column; at 4100 positions (17 decode splits, 1088 over the batch) the MFMA decode kernel with split-K
partials and the combine.  Logits within the fp16-class tolerance, greedy ids identical where the top-2 margin
exceeds it."""
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
@pytest.mark.parametrize('window,ctx', [(None, 1100), (1024, 1100), (None, 4100)])
def test_batch_decode_kernel_matches_chunk_kernel(gpu_device, shape, window, ctx):
    if shape == 'small-hd64':
        cfg, w = make_weights(small_cfg(max_position_embeddings=8192), 'q8', seed=21)
    else:
        cfg, w = make_weights(preset('qwen2-1.5b', num_hidden_layers=2, vocab_size=4096), 'q8', seed=22)
    B = 32
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
