"""The C-ABI example of INTEGRATION.md, run as written: it must build, load and decode through the raw ctypes binding,
and its greedy id must equal the Python engine's on the same weights."""
import os
import re
from pathlib import Path

import pytest

from seedplane_amd.presets import preset
from seedplane_amd.qwen_engine import Qwen2Engine
from seedplane_amd.synth import make_weights

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]


def _example():
    text = (ROOT / 'INTEGRATION.md').read_text()
    m = re.search(r'<!-- capi-example -->\s*```python\n(.*?)```\s*<!-- /capi-example -->', text, flags=re.S)
    assert m, 'INTEGRATION.md lost its C-ABI example block'
    return m.group(1)


def test_integration_capi_example_runs_and_agrees_with_the_engine(gpu_device):
    code = _example()
    here = os.getcwd()
    os.chdir(ROOT)                            # the example opens the library by its repository-relative path
    try:
        ns = {}
        exec(compile(code, 'INTEGRATION.md:capi-example', 'exec'), ns)
    finally:
        os.chdir(here)
    cfg, w = make_weights(preset('tiny'), 'q8', seed=0)
    eng = Qwen2Engine(config=cfg, tensors=w, max_tokens=16)
    assert ns['next_token'] == next(eng.generate(ns['prompt'], max_new_tokens=1))
