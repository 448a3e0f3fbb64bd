"""MI355X (gfx950) quantized lm_head and fused sampler kernels for vLLM.

Drop-in for the ``vllm_quant_kernels`` plugin: same ``vllm.general_plugins`` entry point
(``quant_kernels = vllm_quant_kernels:register``), same env vars and priority, same
``lm_head`` packing attributes and ``Sampler.sample`` hook; the kernels are hand-written
HIP for gfx950 behind a C ABI (include/vqk.h, libvqk_hip.so).
"""

__version__ = "0.1.0"


def register() -> None:
    """vLLM plugin entry point (reference src/vllm_quant_kernels/__init__.py:6-10)."""
    from ._registration import register_all

    register_all()
