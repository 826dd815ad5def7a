"""``decode_kernels.ops`` is ``decodekernels_amd.ops`` (reference: decode_kernels/ops.py)."""

import sys

from decodekernels_amd import ops as _impl

sys.modules[__name__] = _impl
