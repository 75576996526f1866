"""``mcoplib.op`` (the reference's pybind module, op/pybind.cpp:30) is ``mcoplib_amd.op``.

The module object under the reference's name is the implementation module itself, so both
names give the same functions (and registration happens once)."""

import sys

from mcoplib_amd import op as _impl

sys.modules[__name__] = _impl
