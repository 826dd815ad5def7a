"""``decode_kernels``: DecodeKernels' import name for this package.

Callers written against the reference (``import decode_kernels as dk``,
``from decode_kernels import ops``, ``decode_kernels.vllm_patch.apply()``,
``import decode_kernels._C`` for ``torch.ops.decode_kernels.*``; reference:
decode_kernels/__init__.py:7-27) run unchanged on ``decodekernels_amd``. Each
submodule here is the implementation's own module object (the stub files
replace themselves in ``sys.modules``), so module state -- the vLLM patch's
counters, monkeypatched functions -- is shared between the two names.
"""

from decodekernels_amd import *  # noqa: F401,F403
from decodekernels_amd import __all__, __version__  # noqa: F401
