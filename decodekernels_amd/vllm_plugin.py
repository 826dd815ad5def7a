"""vLLM general-plugin entry point (reference: decode_kernels/vllm_plugin.py:14-20).

vLLM imports this in every process it starts. It does nothing unless
DECODE_KERNELS_VLLM=1, so installing the package never changes vLLM by itself.

    DECODE_KERNELS_VLLM=1                                 enable
    DECODE_KERNELS_OPS=attention,rms_norm,silu_and_mul   ops to swap (default: all)

The package registers it under the reference's entry-point name (pyproject.toml):
``[project.entry-points."vllm.general_plugins"] decode_kernels = "decode_kernels.vllm_plugin:register"``
(``decode_kernels.vllm_plugin`` is this module under the reference's import name).
"""

import os


def register() -> None:
    if os.environ.get("DECODE_KERNELS_VLLM", "0") != "1":
        return
    from .vllm_patch import apply

    ops = os.environ.get("DECODE_KERNELS_OPS", "attention,rms_norm,silu_and_mul")
    apply([o.strip() for o in ops.split(",") if o.strip()])
