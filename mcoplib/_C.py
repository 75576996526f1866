"""``mcoplib._C`` (the reference's torch library, op/vllm/torch_bindings.cpp:19,506) is
``mcoplib_amd._C``: importing it registers the ``torch.ops._C`` schemas and kernels.

The module object under the reference's name is the implementation module itself, so both
names give the same functions (and registration happens once)."""

import sys

from mcoplib_amd import _C as _impl

sys.modules[__name__] = _impl
