"""HF quantization config + quantizer ``"mxfp4_bf16_dequant"`` for the MI355X path.

Same registration name, config fields and loading behaviour as the
reference's ``quantizer_config.py:49-226``:

* ``Mxfp4Bf16DequantConfig(dequant_dtype="bf16", fuse_swiglu=False, **Mxfp4Config kwargs)``;
* before weight loading the ``GptOssExperts`` modules are swapped for
  ``Mxfp4Bf16DequantGptOssExperts`` and ``GptOssMLP.forward`` is re-bound to
  ``mlp_forward``;
* checkpoint ``*_blocks`` / ``*_scales`` are stored as-is (bf16 containers),
  or, with ``dequantize=True``, expanded to bf16 weights by the HIP dequant.

Differences: the environment check asks for a ROCm GPU with the built HIP
library instead of Triton / the kernels hub, and nothing is fetched from the
network.  ``dequant_dtype`` "bf16" and "fp8" are both served by the HIP path.  Importing this module registers the config (once per process).
"""
from __future__ import annotations

import logging

import torch
from transformers.quantizers.base import HfQuantizer
from transformers.utils.quantization_config import Mxfp4Config

logger = logging.getLogger(__name__)

QUANT_METHOD = "mxfp4_bf16_dequant"


class Mxfp4Bf16DequantConfig(Mxfp4Config):
    def __init__(self, dequant_dtype="bf16", fuse_swiglu=False, **kwargs):
        super().__init__(**kwargs)
        self.quant_method = QUANT_METHOD
        self.dequant_dtype = dequant_dtype
        self.fuse_swiglu = fuse_swiglu

    def to_dict(self):
        d = super().to_dict()
        d["dequant_dtype"] = self.dequant_dtype
        d["fuse_swiglu"] = self.fuse_swiglu
        return d


class Mxfp4Bf16DequantQuantizer(HfQuantizer):
    """MXFP4 weights kept packed; dequantised inside the grouped GEMM on MI355X."""

    requires_calibration = False

    def __init__(self, quantization_config, **kwargs):
        super().__init__(quantization_config, **kwargs)

    def validate_environment(self, *args, **kwargs):
        if getattr(self.quantization_config, "dequantize", False):
            return
        if getattr(self.quantization_config, "dequant_dtype", "bf16") not in ("bf16", "fp8"):
            raise ValueError("dequant_dtype must be 'bf16' or 'fp8'")
        if not torch.cuda.is_available():
            raise RuntimeError("MXFP4 dequant requires a GPU")
        from . import _capi
        _capi.load()  # raises if the HIP library is missing

    def param_needs_quantization(self, model, param_name, **kwargs):
        from transformers.quantizers.quantizers_utils import get_module_from_name

        from .quantization import Mxfp4Bf16DequantGptOssExperts
        module, tensor_name = get_module_from_name(model, param_name)
        if isinstance(module, Mxfp4Bf16DequantGptOssExperts):
            return tensor_name not in ("down_proj_bias", "gate_up_proj_bias")
        return False

    def _process_model_after_weight_loading(self, model, **kwargs):
        if torch.cuda.is_available():
            torch.cuda.empty_cache()

    def _process_model_before_weight_loading(self, model, use_kernels=False, **kwargs):
        from .quantization import replace_with_dequant_experts
        if use_kernels:
            self.quantization_config.dequantize = True
        self.modules_to_not_convert = self.get_modules_to_not_convert(
            model, self.quantization_config.modules_to_not_convert, model._keep_in_fp32_modules)
        replace_with_dequant_experts(model, modules_to_not_convert=self.modules_to_not_convert,
                                     quantization_config=self.quantization_config)

    def update_tp_plan(self, config):
        return self._grouped_gemm_plan(config, "base_model_tp_plan")

    def update_ep_plan(self, config):
        return self._grouped_gemm_plan(config, "base_model_ep_plan")

    @staticmethod
    def _grouped_gemm_plan(config, attr):
        plan = getattr(config, attr, None)
        if "GptOssConfig" in config.__class__.__name__ and plan is not None:
            for proj in ("gate_up_proj", "down_proj"):
                for part in ("blocks", "scales"):
                    plan[f"layers.*.mlp.experts.{proj}_{part}"] = "grouped_gemm"
        return config

    def get_state_dict_and_metadata(self, model):
        return model.state_dict(), {}

    def is_serializable(self, *args, **kwargs):
        return True

    @property
    def is_trainable(self):
        return True

    def get_quantize_ops(self):
        from .quantization import Mxfp4Fp8DequantQuantize
        return Mxfp4Fp8DequantQuantize(self)

    def get_weight_conversions(self):
        from transformers.core_model_loading import WeightConverter

        from .quantization import Mxfp4Fp8DequantDequantize, Mxfp4Fp8DequantDeserialize
        if not self.pre_quantized:
            return []
        op = Mxfp4Fp8DequantDequantize if self.quantization_config.dequantize else Mxfp4Fp8DequantDeserialize
        return [WeightConverter(source_patterns=["_blocks", "_scales"], target_patterns="", operations=[op(self)])]


def register() -> None:
    """Register config + quantizer under "mxfp4_bf16_dequant" (no-op if present)."""
    from transformers.quantizers import auto
    cfg_map = getattr(auto, "AUTO_QUANTIZATION_CONFIG_MAPPING", {})
    q_map = getattr(auto, "AUTO_QUANTIZER_MAPPING", {})
    if QUANT_METHOD not in cfg_map:
        auto.register_quantization_config(QUANT_METHOD)(Mxfp4Bf16DequantConfig)
    if QUANT_METHOD not in q_map:
        auto.register_quantizer(QUANT_METHOD)(Mxfp4Bf16DequantQuantizer)


register()
