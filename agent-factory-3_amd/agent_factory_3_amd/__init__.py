"""MI355X (gfx950) implementation of agent-factory-3's MXFP4 MoE expert hot path.

Drop-in for ``agent_factory_3.models.gpt_oss``'s compute path: MXFP4 -> bf16
dequant, grouped expert GEMMs with the dequant fused into the tile load,
gpt-oss clamped SwiGLU, routing permutation, and expert-LoRA gradients, as
hand-written HIP kernels behind the C ABI of ``libaf3_mi355x.so``.

Public modules mirror the reference's file names:
``kernels``, ``quantization``, ``quantizer_config``, ``routing_replay``,
``fsdp2_fix``; ``routing`` holds the routing objects the reference imports
from ``triton_kernels``.
"""
from . import _capi  # noqa: F401

__all__ = ["Mxfp4Bf16DequantConfig", "enable_routing_replay"]


def __getattr__(name):
    # the HF-integration names need transformers; import them lazily
    if name == "Mxfp4Bf16DequantConfig":
        from .quantizer_config import Mxfp4Bf16DequantConfig
        return Mxfp4Bf16DequantConfig
    if name == "enable_routing_replay":
        from .routing_replay import enable_routing_replay
        return enable_routing_replay
    raise AttributeError(name)
