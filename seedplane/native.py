"""`seedplane.native` is `seedplane_amd.native` (the same module object)."""
import sys

from seedplane_amd import native as _module

sys.modules[__name__] = _module
