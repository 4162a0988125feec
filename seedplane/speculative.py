"""`seedplane.speculative` is `seedplane_amd.speculative` (the same module object)."""
import sys

from seedplane_amd import speculative as _module

sys.modules[__name__] = _module
