"""``mcoplib.custom_ops`` (reference mcoplib/custom_ops.py) is ``mcoplib_amd.custom_ops``.

The module object under the reference's name is the implementation module itself, so both
names give the same functions (and registration happens once)."""

import sys

from mcoplib_amd import custom_ops as _impl

sys.modules[__name__] = _impl
