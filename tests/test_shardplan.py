"""ShardPlan windows (reference unit tests tests/test_core.py:20-36, restated) and the per-token visible sets the
sharded session attends to, checked against the windows by brute force."""
import numpy as np
import pytest

from seedplane_amd.engine import ShardPlan, ShardedSession


def test_windows_cover_each_core_once():
    plan = ShardPlan(shard=4, halo=2, sinks=1)
    windows = list(plan.windows(10))
    assert [(a, b) for a, b, _ in windows] == [(0, 4), (4, 8), (8, 10)]
    assert np.concatenate([np.arange(a, b) for a, b, _ in windows]).tolist() == list(range(10))
    assert windows[1][2].tolist() == [0, 2, 3, 4, 5, 6, 7]


def test_empty_sequence():
    assert list(ShardPlan().windows(0)) == []


def test_rejects_invalid_values():
    for args in ((0, 1, 0), (1, -1, 0), (1, 0, -1)):
        with pytest.raises(ValueError):
            ShardPlan(*args)
    with pytest.raises(ValueError):
        list(ShardPlan().windows(-1))


@pytest.mark.parametrize('shard,halo,sinks', [(4, 2, 1), (8, 4, 2), (4, 10, 3), (5, 0, 0), (3, 3, 5), (16, 0, 4)])
def test_visible_is_the_window_prefix(shard, halo, sinks):
    plan = ShardPlan(shard, halo, sinks)
    L = 41
    for c0, c1, idx in plan.windows(L):
        idx = idx.tolist()
        core_at = len(idx) - (c1 - c0)           # the core tokens close the window
        for i in range(c0, c1):
            assert plan.visible(i) == idx[:core_at + (i - c0) + 1]
            # the session's window slots: sinks, halo, then the shard's tokens, each at its original position
            assert len(plan.visible(i)) <= shard + halo + sinks


def test_session_rejects_unknown_modes_and_reuse_plans_it_cannot_copy():
    with pytest.raises(ValueError):
        ShardedSession(None, ShardPlan(), mode='bogus')
    # reuse copies the halo and the sinks out of one window: both must fit a shard (qwen_vk.cpp:297)
    with pytest.raises(ValueError, match='halo <= shard'):
        ShardedSession(None, ShardPlan(shard=4, halo=10, sinks=3), mode='reuse')
    with pytest.raises(ValueError, match='sinks <= shard'):
        ShardedSession(None, ShardPlan(shard=4, halo=2, sinks=6), mode='reuse')
