"""The reference's import path: `seedplane.<module>` is this build's `seedplane_amd.<module>` -- the same module
objects, so the names the reference's own tests import (tests/test_speculative.py:3, tests/test_core.py:13-17 for the
modules on this path) resolve to this build's implementations."""
import importlib

import pytest

import seedplane_amd


@pytest.mark.parametrize('name', ['qwen_engine', 'speculative', 'engine', 'native', 'native_bundle'])
def test_module_is_the_same_object(name):
    alias = importlib.import_module(f'seedplane.{name}')
    assert alias is importlib.import_module(f'seedplane_amd.{name}')


def test_reference_test_imports_resolve():
    from seedplane.speculative import CommitLedger, SpeculativeForest, verify_greedy
    from seedplane.engine import ShardPlan
    from seedplane.qwen_engine import Qwen2Engine, chat_prompt
    from seedplane import native, native_bundle
    from seedplane_amd import speculative, engine, qwen_engine
    assert (CommitLedger, SpeculativeForest, verify_greedy) == (speculative.CommitLedger, speculative.SpeculativeForest,
                                                                 speculative.verify_greedy)
    assert ShardPlan is engine.ShardPlan and Qwen2Engine is qwen_engine.Qwen2Engine
    assert chat_prompt is qwen_engine.chat_prompt
    assert native.find_engine is seedplane_amd.native.find_engine
    assert native_bundle.load is seedplane_amd.native_bundle.load


def test_forest_through_the_reference_path():
    """The reference test's own scenario shape, through the alias: two branches sharing a prefix, greedy
    verification accepts the branch the target agrees with."""
    from seedplane.speculative import SpeculativeForest, verify_greedy
    forest = SpeculativeForest.build([[1, 2, 3], [1, 4]])
    assert forest.node_count == 4
    nxt = {(7,): 1, (7, 1): 2, (7, 1, 2): 3, (7, 1, 2, 3): 9}

    def logits(prefix):
        out = [0.0] * 10
        out[nxt.get(tuple(prefix), 0)] = 1.0
        return out
    v = verify_greedy([7], forest, logits)
    assert v.emitted == (1, 2, 3)          # the whole path accepted; no correction token


def test_kvcache_keeps_the_reference_dataclass_signature():
    from seedplane.qwen_engine import KVCache
    c = KVCache([], [], 0, 16)                       # qwen_engine.py:18-23 field order
    assert (c.keys, c.values, c.length, c.capacity) == ([], [], 0, 16)
    a = KVCache.allocate(2, 32, 2, 64, 'cpu', None)
    assert a.capacity == 32 and a.length == 0
    a.length = 5                                     # rollback by assignment, as the reference does
    assert a.length == 5
