"""Sharded-window decode on the HIP engine: every token's logits equal the oracle run over exactly the tokens its
shard window shows (sinks + halo + shard prefix, original positions), in both exact boundary modes."""
import pytest
import torch

from oracle.qwen_ref import RefQwen2, max_rel
from seedplane_amd.engine import ShardPlan, ShardedSession
from seedplane_amd.presets import preset
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights, random_prompt

pytestmark = pytest.mark.gpu


@pytest.fixture(scope='module')
def model(gpu_device):
    cfg, w = make_weights(preset('tiny'), 'f32', seed=2)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=16)
    ref = RefQwen2(cfg, {k: (v.half().float() if v.dim() == 2 else v) for k, v in w.items()})
    return cfg, eng, ref


def _window_row(ref, ids, plan, i):
    vis = plan.visible(i)
    lg = ref.forward([ids[j] for j in vis], ref.new_cache(len(vis)), all_logits=True, positions=vis)
    return lg[-1]


@pytest.mark.parametrize('mode', ['rebuild', 'shadow'])
@pytest.mark.parametrize('shard,halo,sinks', [(8, 4, 2), (4, 10, 3), (6, 0, 1)])
def test_session_matches_window_oracle(model, mode, shard, halo, sinks):
    cfg, eng, ref = model
    print(f'shard session {mode} S={shard} H={halo} K={sinks}', flush=True)
    plan = ShardPlan(shard, halo, sinks)
    ids = random_prompt(30, cfg['vocab_size'], seed=shard + halo)
    s = ShardedSession(eng, plan, mode)
    for i, t in enumerate(ids):
        row = s.step(t, need_logits=(i % 3 == 2 or i == len(ids) - 1))
        if row is not None:
            err = max_rel(row[None], _window_row(ref, ids, plan, i)[None])
            assert err < 2e-2, (i, err)
    assert s.boundaries == (len(ids) - 1) // shard
    if mode == 'shadow' and halo > 0:
        assert s.dual > 0


def test_one_shard_equals_plain_forward(model):
    cfg, eng, ref = model
    ids = random_prompt(20, cfg['vocab_size'], seed=9)
    s = ShardedSession(eng, ShardPlan(64, 8, 4), 'rebuild')
    row = s.feed(ids)
    lg, _ = eng.forward(ids, eng.new_cache(32))
    assert max_rel(row[None], lg) < 1e-3
    assert s.boundaries == 0 and s.extra == 0
