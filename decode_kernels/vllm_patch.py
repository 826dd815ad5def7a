"""``decode_kernels.vllm_patch`` is ``decodekernels_amd.vllm_patch`` (reference: decode_kernels/vllm_patch.py)."""

import sys

from decodekernels_amd import vllm_patch as _impl

sys.modules[__name__] = _impl
