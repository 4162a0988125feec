"""`seedplane.engine` is `seedplane_amd.engine` (the same module object)."""
import sys

from seedplane_amd import engine as _module

sys.modules[__name__] = _module
