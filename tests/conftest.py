import os
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line('markers', 'gpu: needs a ROCm GPU (MI355X, gfx950) and the built HIP library')


def small_cfg(**kw):
    """A small Qwen2 shape that satisfies the kernels' constraints (hidden/intermediate multiples of 128)."""
    from seedplane_amd.presets import preset
    base = dict(num_hidden_layers=2, hidden_size=256, num_attention_heads=4, num_key_value_heads=2,
                intermediate_size=512, vocab_size=1000, max_position_embeddings=4096)
    base.update(kw)
    return preset('tiny', **base)


@pytest.fixture(scope='session')
def tiny_f32():
    from seedplane_amd.presets import preset
    from seedplane_amd.synth import make_weights
    return make_weights(preset('tiny'), 'f32', seed=0)


@pytest.fixture(scope='session')
def gpu_device():
    import torch
    from seedplane_amd import _lib
    _lib.load()
    assert torch.cuda.is_available(), 'GPU tests need a ROCm GPU'
    return torch.device('cuda:0')
