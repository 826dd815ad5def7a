"""``decode_kernels._C`` is ``decodekernels_amd._C`` (reference: setup.py:19-20, csrc/module.cpp)."""

import sys

from decodekernels_amd import _C as _impl

sys.modules[__name__] = _impl
