"""``decode_kernels.testing`` is ``decodekernels_amd.testing`` (reference: decode_kernels/testing.py)."""

import sys

from decodekernels_amd import testing as _impl

sys.modules[__name__] = _impl
