"""GPU filtered sampling (sp_op_sample_filtered: temperature, top-k, top-p, inverse CDF) against the oracle's
sort-based restatement: bit-exact token ids for the same logits and uniforms, at the full Qwen2 vocabulary and with
heavy ties; generate(temperature > 0) draws every token through it."""
import numpy as np
import pytest
import torch

from oracle.sample_ref import sample_filtered
from seedplane_amd.presets import preset
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.speculative import uniforms
from seedplane_amd.synth import make_weights

pytestmark = pytest.mark.gpu

CASES = [(0.7, 0, 1.0), (1.3, 40, 1.0), (0.8, 0, 0.9), (0.8, 50, 0.5), (1.0, 1, 1.0), (0.6, 0, 1e-6),
         (1.1, 1999, 0.95), (0.9, 7, 0.3), (0.8, 151935, 0.99), (2.0, 100000, 1.0)]


@pytest.fixture(scope='module')
def eng(gpu_device):
    cfg, w = make_weights(preset('tiny'), 'f32', seed=0)
    return Qwen2Engine(config=cfg, tensors=w, max_tokens=16)


def _rows(V, seed):
    g = np.random.default_rng(seed)
    rows = (g.standard_normal((6, V)) * 3.0).astype(np.float32)
    rows[4] = np.round(rows[4] * 2) / 2                     # heavy ties
    rows[5] = 0.0
    rows[5, ::7] = 1.0                                      # ties at the maximum
    return rows


@pytest.mark.parametrize('V', [151936, 1000])
@pytest.mark.parametrize('case', range(len(CASES)))
def test_gpu_draws_equal_oracle(eng, V, case):
    T, k, p = CASES[case]
    print(f'sample_filtered V={V} T={T} k={k} p={p}', flush=True)
    rows = _rows(V, seed=case)
    n = rows.shape[0]
    u = uniforms(11, case, 3 * n)
    u[0], u[1] = 0.0, 1.0 - 2.0 ** -53                      # the two ends of the inverse CDF
    lg = torch.from_numpy(rows).cuda()
    got = eng.sample_gpu(lg, [i % n for i in range(3 * n)], u, T, k, p)
    want = [sample_filtered(rows[i % n], T, k, p, u[i]) for i in range(3 * n)]
    assert got == want


def test_gpu_sample_rejects_bad_arguments(eng):
    lg = torch.zeros((2, 100), dtype=torch.float32, device='cuda')
    with pytest.raises(ValueError):
        eng.sample_gpu(lg, [0], [0.5], 0.0)
    with pytest.raises(ValueError):
        eng.sample_gpu(lg, [0], [0.5], 1.0, 0, 0.0)
    # every row index is checked on the host before the launch: nothing out of bounds reaches the kernel
    with pytest.raises(ValueError):
        eng.sample_gpu(lg, [0], [0.5, 0.5], 1.0)                 # fewer rows than draws
    with pytest.raises(ValueError):
        eng.sample_gpu(lg, [2], [0.5], 1.0)                      # row past the end
    with pytest.raises(ValueError):
        eng.sample_gpu(lg, [-1], [0.5], 1.0)
    with pytest.raises(ValueError):
        eng.sample_gpu(torch.zeros((100, 2), device='cuda').t(), [0], [0.5], 1.0)   # strided rows
    with pytest.raises(ValueError):
        eng.sample_gpu(lg, None, [0.5, 0.5], 1.0, rows_dev=torch.zeros(1, dtype=torch.int32, device='cuda'))
    flat = np.zeros(100, dtype=np.float32)
    assert eng.sample_gpu(lg, [1, 0], [0.25, 0.75], 1.0) == [sample_filtered(flat, 1.0, 0, 1.0, u) for u in (0.25, 0.75)]


def test_generate_with_temperature_uses_gpu_draws(eng):
    prompt = [1, 2, 3, 4, 5]
    toks = list(eng.generate(prompt, max_new_tokens=6, temperature=0.8, top_k=20, top_p=0.9, seed=3))
    assert len(toks) == 6
    seq = prompt + toks
    lg, _ = eng.forward(seq[:-1], eng.new_cache(16), all_logits=True)
    rows = lg[len(prompt) - 1:].cpu().numpy()
    for i, t in enumerate(toks):
        assert t == sample_filtered(rows[i], 0.8, 20, 0.9, uniforms(3, i, 1)[0]), i
