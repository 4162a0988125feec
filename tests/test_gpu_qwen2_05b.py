"""Oracle parity of the HIP engine at the full Qwen2-0.5B shape (24 layers, hidden 896, 14 / 2 heads, head_dim 64,
GQA group 7, SwiGLU 4864, tied 151936-row head):
  * the fp32 random-init model from seed 0 (randn * 0.05, embedding x 20, norms 1), a 16-token prompt of uniform ids and
    32 greedy tokens at batch 1: decode logits vs the oracle on the fp16-rounded weights the GPU runs, greedy ids vs the
    oracle on the original fp32 weights (reference qwen_engine.py:105-166);
  * the fp16 N(0, 0.02) model serving 16 requests with prompts of 16-128 uniform ids, 32 greedy tokens each, decoded as
    one batch with per-request caches of 512 positions: every request against its own oracle run."""
import pytest
import torch

from oracle.qwen_ref import RefQwen2
from seedplane_amd.presets import preset
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt
from tests.parity import check_greedy, check_rows, fp16_rounded

pytestmark = pytest.mark.gpu


def test_fp32_init_seed0_prompt16_greedy32(gpu_device):
    print('0.5b fp32-init: weights', flush=True)
    cfg, w = make_weights(preset('qwen2-0.5b'), 'f32', seed=0)
    V, steps = cfg['vocab_size'], 32
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    prompt = torch.randint(0, V, (16,), generator=torch.Generator().manual_seed(0)).tolist()
    cache = eng.new_cache(64)
    lg, cache = eng.forward(prompt, cache)
    rows = torch.empty((steps, V), dtype=torch.float32, device=eng.device)
    rows[0].copy_(lg[0])
    toks = [int(lg[0].argmax())]
    for s in range(1, steps):
        toks.append(int(eng.decode([toks[-1]], [cache], logits_out=rows[s:s + 1])[0]))
    assert list(eng.generate(prompt, steps)) == toks
    del eng
    print('0.5b fp32-init: oracle (fp16-rounded and fp32 weights)', flush=True)
    ref16 = RefQwen2(cfg, fp16_rounded(w))
    ref16_rows = ref16.forward(prompt + toks[:-1], ref16.new_cache(64), all_logits=True)[len(prompt) - 1:]
    del ref16
    worst = check_rows(rows.cpu(), ref16_rows, what='0.5b fp16-rounded')
    ref32 = RefQwen2(cfg, w)
    ref32_rows = ref32.forward(prompt + toks[:-1], ref32.new_cache(64), all_logits=True)[len(prompt) - 1:]
    worst32 = max(float((rows[i].cpu() - ref32_rows[i]).abs().max() / ref32_rows[i].abs().max()) for i in range(steps))
    same = check_greedy(toks, ref32_rows, what='0.5b fp32')
    print(f'0.5b fp32-init: worst max-rel {worst:.2e} (fp16-rounded oracle), {worst32:.2e} (fp32 oracle); '
          f'{same}/{steps} ids equal the fp32 oracle argmax', flush=True)
    assert same >= 0.75 * steps


def test_fp16_16_ragged_requests_batch16(gpu_device):
    print('0.5b fp16: weights', flush=True)
    cfg, w = make_weights(preset('qwen2-0.5b'), 'f16', seed=0)
    V, B, steps = cfg['vocab_size'], 16, 32
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    g = torch.Generator().manual_seed(2)
    lens = torch.randint(16, 129, (B,), generator=g).tolist()
    prompts = [torch.randint(0, V, (n,), generator=g).tolist() for n in lens]
    caches = [eng.new_cache(512) for _ in range(B)]
    first = eng.prefill(prompts, caches)
    rows = torch.empty((steps - 1, B, V), dtype=torch.float32, device=eng.device)
    toks = [list(first)]
    for s in range(steps - 1):
        toks.append([int(t) for t in eng.decode(toks[-1], caches, logits_out=rows[s])])
    per_req = [[toks[s][b] for s in range(steps)] for b in range(B)]
    assert eng.generate_batch(prompts, steps) == per_req
    rows = rows.cpu()
    del eng, caches
    ref = RefQwen2(cfg, w)
    worst, same = 0.0, 0
    for b in range(B):
        print(f'0.5b fp16: oracle request {b} (prompt {lens[b]})', flush=True)
        seq = prompts[b] + per_req[b][:-1]
        ref_rows = ref.forward(seq, ref.new_cache(len(seq)), all_logits=True)[lens[b] - 1:]
        worst = max(worst, check_rows(rows[:, b], ref_rows[1:], what=f'request {b}'))
        same += check_greedy(per_req[b], ref_rows, what=f'request {b}')
    print(f'0.5b fp16: worst max-rel {worst:.2e}, {same}/{B * steps} ids equal the oracle argmax', flush=True)
    assert same >= 0.75 * B * steps
