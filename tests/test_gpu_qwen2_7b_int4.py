"""Parity of the HIP engine at the Qwen2-7B shape (hidden 3584, 28 / 4 heads, head_dim 128, GQA group 7, SwiGLU 18944,
untied 152064-row head) with int4 group-32 weights (codes U[0, 15], fp16 scale |N(0, 0.002)| and zero per group):
  * a 2-layer model of that shape against the oracle: batch-1 decode after a 300-token prompt (the chunk kernel with
    RoPE fused), 8 sequences of about 1000 positions decoded as one batch (the multi-query MFMA kernel), and 32
    sequences of about 2000 positions (the MFMA decode kernel over 256-key splits);
  * the full 28-layer model at batch 32 with 8192 cached positions per request: the batched step's logits equal the
    single-column step's (a different attention kernel) within the fp16 tolerance, and are finite.
Sequences share a prompt prefix that the oracle runs once; its cache is cloned per sequence."""
import pytest
import torch

from oracle.qwen_ref import RefQwen2, max_rel
from seedplane_amd.presets import preset
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt
from tests.parity import TOL, check_greedy, check_rows, clone_cache

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def m7(gpu_device):
    print('qwen2-7b shape, 2 layers, int4: weights, engine, oracle prefixes', flush=True)
    cfg, w = make_weights(preset('qwen2-7b', num_hidden_layers=2), 'q4', seed=0)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    ref = RefQwen2(cfg, w)
    del w
    V = cfg['vocab_size']
    pre = random_prompt(2000, V, seed=1)
    rc1 = ref.new_cache(1000)
    ref.forward(pre[:1000], rc1)
    rc2 = clone_cache(ref, rc1, 2000)
    ref.forward(pre[1000:], rc2)
    yield cfg, eng, ref, pre, rc1, rc2


def _batch_vs_oracle(m7, base, suffix_lens, steps, tag):
    cfg, eng, ref, pre, rc1, rc2 = m7
    V, B = cfg['vocab_size'], len(suffix_lens)
    rc = rc1 if base == 1000 else rc2
    suffixes = [random_prompt(n, V, seed=1000 * base + i) for i, n in enumerate(suffix_lens)]
    prompts = [pre[:base] + s for s in suffixes]
    print(f'7b-2L {tag}: prefill + decode', flush=True)
    caches = [eng.new_cache(base + 200) for _ in range(B)]
    first = eng.prefill(prompts, caches)
    rows = torch.empty((steps, B, V), dtype=torch.float32, device=eng.device)
    toks = [list(first)]
    for s in range(steps):
        toks.append([int(t) for t in eng.decode(toks[-1], caches, logits_out=rows[s])])
    rows = rows.cpu()
    worst, same = 0.0, 0
    for b in range(B):
        seq = [toks[s][b] for s in range(steps + 1)]
        oc = clone_cache(ref, rc, len(prompts[b]) + steps + 1)
        ref_rows = torch.cat([ref.forward(suffixes[b], oc)[-1:], ref.forward(seq[:-1], oc, all_logits=True)])
        worst = max(worst, check_rows(rows[:, b], ref_rows[1:], what=f'{tag} seq {b}'))
        same += check_greedy(seq, ref_rows, what=f'{tag} seq {b}')
    print(f'7b-2L {tag}: worst max-rel {worst:.2e}, {same}/{B * (steps + 1)} ids equal the oracle argmax', flush=True)
    assert same >= 0.75 * B * (steps + 1)


def test_bs1_decode_vs_oracle(m7):
    cfg, eng, ref, pre, rc1, rc2 = m7
    V, steps = cfg['vocab_size'], 8
    prompt = random_prompt(300, V, seed=5)
    print('7b-2L bs1: prefill + decode', flush=True)
    cache = eng.new_cache(400)
    lg, cache = eng.forward(prompt, cache)
    rows = torch.empty((steps, V), dtype=torch.float32, device=eng.device)
    rows[0].copy_(lg[0])
    toks = [int(lg[0].argmax())]
    for s in range(1, steps):
        toks.append(int(eng.decode([toks[-1]], [cache], logits_out=rows[s:s + 1])[0]))
    ref_rows = ref.forward(prompt + toks[:-1], ref.new_cache(400), all_logits=True)[len(prompt) - 1:]
    worst = check_rows(rows.cpu(), ref_rows, what='bs1')
    same = check_greedy(toks, ref_rows, what='bs1')
    print(f'7b-2L bs1: worst max-rel {worst:.2e}, {same}/{steps} ids equal the oracle argmax', flush=True)
    assert same >= 0.75 * steps


def test_batch8_multiquery_attention_vs_oracle(m7):
    _batch_vs_oracle(m7, 1000, [10 + 7 * i for i in range(8)], 4, 'batch 8 x ~1030')


def test_batch32_decode_kernel_vs_oracle(m7):
    _batch_vs_oracle(m7, 2000, [8 + 2 * i for i in range(32)], 3, 'batch 32 x ~2040')


def test_full_model_batch32_at_8192_batch_equals_single_column(gpu_device):
    print('qwen2-7b int4 full: weights', flush=True)
    cfg, w = make_weights(preset('qwen2-7b'), 'q4', seed=0)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=64)
    del w
    V, B, ctx = cfg['vocab_size'], 32, 8192
    eng.reserve(B, ctx + 64)
    caches = [eng.new_cache(ctx + 64) for _ in range(B)]
    for b, c in enumerate(caches):
        eng.fill_cache(c, ctx, seed=1 + b)
    toks = random_prompt(B, V, seed=9)
    out = torch.empty((B, V), dtype=torch.float32, device=eng.device)
    print('7b full: batch-32 step at 8192 positions', flush=True)
    ids = eng.decode(toks, caches, logits_out=out)
    assert torch.isfinite(out).all()
    one = torch.empty((1, V), dtype=torch.float32, device=eng.device)
    for b in (0, 13, 31):
        caches[b].length -= 1                         # the same step again, alone
        i1 = eng.decode([toks[b]], [caches[b]], logits_out=one)
        e = max_rel(one[0], out[b])
        print(f'7b full: sequence {b} single column vs batch max-rel {e:.2e}', flush=True)
        assert e < TOL
        if int(i1[0]) != int(ids[b]):
            top = torch.topk(out[b], 2).values
            assert float(top[0] - top[1]) <= TOL * float(out[b].abs().max())
