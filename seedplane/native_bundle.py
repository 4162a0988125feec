"""`seedplane.native_bundle` is `seedplane_amd.native_bundle` (the same module object)."""
import sys

from seedplane_amd import native_bundle as _module

sys.modules[__name__] = _module
