"""Expert-LoRA save / resume (CPU): the adapters of every experts module go
out under PEFT's saved-key form with their scaling, through a safetensors
file, and come back into freshly built modules bit for bit (rank and scaling
restored, PEFT's ``base_model.model.`` prefix accepted)."""
import types

import pytest
import torch
from safetensors.torch import load_file, save_file

from agent_factory_3_amd import quantization as Q


def _model(E=4, H=64, I=64, layers=2):
    cfg = types.SimpleNamespace(num_local_experts=E, intermediate_size=I, hidden_size=H, swiglu_limit=7.0)
    root = torch.nn.Module()
    root.layers = torch.nn.ModuleList()
    for _ in range(layers):
        blk = torch.nn.Module()
        blk.mlp = torch.nn.Module()
        blk.mlp.experts = Q.Mxfp4Bf16DequantGptOssExperts(cfg)
        root.layers.append(blk)
    return root


def test_round_trip_through_safetensors(tmp_path):
    src = _model()
    g = torch.Generator().manual_seed(3)
    Q.enable_expert_lora(src.layers[0].mlp.experts, r=16, lora_alpha=32, init="normal", generator=g)
    Q.enable_expert_lora(src.layers[1].mlp.experts, r=8, lora_alpha=4, init="normal", generator=g)
    sd = Q.expert_lora_state_dict(src)
    assert set(sd) == {f"layers.{l}.mlp.experts.{p}" for l in (0, 1) for p in Q.EXPERT_LORA_PARAMS} | \
        {f"layers.{l}.mlp.experts.expert_lora_scaling" for l in (0, 1)}
    # PEFT's saved keys carry the base_model.model. prefix of the wrapped model
    save_file({"base_model.model." + k: v for k, v in sd.items()}, str(tmp_path / "adapter.safetensors"))

    dst = _model()
    done = Q.load_expert_lora_state_dict(dst, load_file(str(tmp_path / "adapter.safetensors")))
    assert done == ["layers.0.mlp.experts", "layers.1.mlp.experts"]
    for l, (r, s) in enumerate(((16, 2.0), (8, 0.5))):
        a, b = src.layers[l].mlp.experts, dst.layers[l].mlp.experts
        assert b.expert_lora_r == r and b.expert_lora_scaling == s
        for p in Q.EXPERT_LORA_PARAMS:
            assert getattr(b, p).dtype == torch.bfloat16 and getattr(b, p).requires_grad
            assert torch.equal(getattr(a, p), getattr(b, p)), p


def test_only_modules_with_adapters_and_errors():
    src = _model()
    Q.enable_expert_lora(src.layers[1].mlp.experts, r=8, init="normal")
    sd = Q.expert_lora_state_dict(src)
    assert all(k.startswith("layers.1.") for k in sd)        # the module without LoRA contributes nothing
    dst = _model()
    Q.enable_expert_lora(dst.layers[1].mlp.experts, r=8, lora_alpha=64)  # same rank, other scaling: overwritten
    assert Q.load_expert_lora_state_dict(dst, sd) == ["layers.1.mlp.experts"]
    assert dst.layers[1].mlp.experts.expert_lora_scaling == src.layers[1].mlp.experts.expert_lora_scaling
    assert dst.layers[0].mlp.experts.expert_lora_r == 0
    bad = {"layers.7.mlp.experts." + k.split(".")[-1]: v for k, v in sd.items()}
    with pytest.raises(KeyError):
        Q.load_expert_lora_state_dict(dst, bad)
    assert Q.load_expert_lora_state_dict(dst, bad, strict=False) == []
    wrong = dict(sd)
    wrong["layers.1.mlp.experts.down_proj_lora_B"] = torch.zeros(3, 3, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        Q.load_expert_lora_state_dict(dst, wrong)
