"""``decode_kernels.vllm_plugin`` is ``decodekernels_amd.vllm_plugin`` (reference: decode_kernels/vllm_plugin.py)."""

import sys

from decodekernels_amd import vllm_plugin as _impl

sys.modules[__name__] = _impl
