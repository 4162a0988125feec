"""`seedplane.qwen_engine` is `seedplane_amd.qwen_engine` (the same module object)."""
import sys

from seedplane_amd import qwen_engine as _module

sys.modules[__name__] = _module
