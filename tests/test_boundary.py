"""Drop-in boundary: module/API surface, HF registration, routing-replay plumbing (CPU)."""
import inspect

import pytest
import torch


def test_reference_names_exported():
    from agent_factory_3_amd import kernels, quantization, routing
    for name in ("mxfp4_to_bf16", "SwiGLUFunction", "DequantMoEMatmul", "Mxfp4Bf16DequantGptOssExperts",
                 "mlp_forward", "routing_replay", "routing_torch_dist", "replace_with_dequant_experts",
                 "FP4_VALUES", "_pack_uint8_as_bf16", "_unpack_bf16_as_uint8", "_store_mxfp4_weights",
                 "convert_moe_packed_tensors", "on_device", "Mxfp4Fp8DequantDeserialize"):
        assert hasattr(quantization, name), name
    for name in ("mxfp4_to_bf16_triton", "_swiglu_forward_triton", "_swiglu_backward"):
        assert hasattr(kernels, name), name
    for name in ("RoutingData", "GatherIndx", "ScatterIndx", "compute_expt_data_torch", "routing"):
        assert hasattr(routing, name), name
    sig = inspect.signature(quantization.DequantMoEMatmul.forward)
    assert list(sig.parameters)[1:] == ["x", "blocks", "scales", "bias", "routing_data", "fwd_gather_indx",
                                        "fwd_scatter_indx", "fwd_gammas", "bwd_gather_indx", "bwd_scatter_indx",
                                        "bwd_gammas", "dequant_dtype", "n_expts_act", "experts_module",
                                        "proj_name"]


def test_routing_dataclass_field_order():
    from agent_factory_3_amd.routing import GatherIndx, RoutingData, ScatterIndx
    rd = RoutingData("g", "h", 4, 2, "ed")
    assert (rd.gate_scal, rd.expt_hist, rd.n_expts_tot, rd.n_expts_act, rd.expt_data) == ("g", "h", 4, 2, "ed")
    assert GatherIndx("s", "d").src_indx == "s" and ScatterIndx("s", "d").dst_indx == "d"


def test_pack_unpack_roundtrip_keeps_nan_patterns():
    from agent_factory_3_amd import quantization as Q
    u8 = torch.arange(256, dtype=torch.uint8).repeat(5)[:1023]      # odd length, includes NaN bf16 patterns
    packed = Q._pack_uint8_as_bf16(u8)
    assert packed.dtype == torch.bfloat16 and packed.numel() == 512
    assert torch.equal(Q._unpack_bf16_as_uint8(packed, (1023,)), u8)


def test_fsdp2_fix_preserves_bits():
    import agent_factory_3_amd.fsdp2_fix  # noqa: F401
    src = torch.arange(0, 65536, 7, dtype=torch.int32).to(torch.int16).view(torch.bfloat16)
    dst = torch.empty_like(src)
    torch._foreach_copy_([dst], [src])
    assert torch.equal(dst.view(torch.int16), src.view(torch.int16))


def test_quantizer_registration():
    from transformers.quantizers import auto

    from agent_factory_3_amd import quantizer_config as qc
    assert auto.AUTO_QUANTIZATION_CONFIG_MAPPING["mxfp4_bf16_dequant"] is qc.Mxfp4Bf16DequantConfig
    cfg = qc.Mxfp4Bf16DequantConfig(dequant_dtype="bf16")
    d = cfg.to_dict()
    assert d["quant_method"] == "mxfp4_bf16_dequant" and d["dequant_dtype"] == "bf16" and not d["fuse_swiglu"]
    qc.register()  # idempotent


def test_replace_and_routing_replay_plumbing():
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssModel

    from agent_factory_3_amd import quantization as Q
    from agent_factory_3_amd import routing_replay
    cfg = GptOssConfig(num_hidden_layers=2, hidden_size=64, intermediate_size=64, num_local_experts=4,
                       num_experts_per_tok=2, num_attention_heads=2, num_key_value_heads=1, head_dim=32,
                       vocab_size=128, layer_types=["sliding_attention", "full_attention"])
    with torch.device("meta"):
        model = GptOssModel(cfg)
    Q.replace_with_dequant_experts(model, quantization_config=type("C", (), {"dequantize": False})())
    assert isinstance(model.layers[0].mlp.experts, Q.Mxfp4Bf16DequantGptOssExperts)
    assert model.layers[0].mlp.forward.__func__ is Q.mlp_forward
    routing_replay.enable_routing_replay(model)
    seen = {}

    def fake_mlp(self, hidden_states, router_indices=None):
        seen[self] = routing_replay.current_router_indices(self)
        return hidden_states, None

    import types
    layer = model.layers[1]
    layer.mlp.forward = types.MethodType(fake_mlp, layer.mlp)
    ri = torch.arange(1 * 3 * 2 * 2).view(1, 3, 2, 2)
    # call the wrapped decoder layer the way GptOssModel.forward does (kwargs flow through)
    layer.input_layernorm = torch.nn.Identity()
    layer.post_attention_layernorm = torch.nn.Identity()
    layer.self_attn.forward = lambda hidden_states, **kw: (torch.zeros_like(hidden_states), None)
    h = torch.zeros(1, 3, 64)
    layer(h, routing_indices=ri)
    assert torch.equal(seen[layer.mlp], ri[:, :, 1, :])
    assert routing_replay.current_router_indices(layer.mlp) is None  # cleared after the layer call


def test_router_kernel_predicate_on_cpu_tensors():
    """The router kernel's operand check (routing.router_kernel_supports): CPU
    tensors never qualify; router_linear refuses them."""
    import pytest
    import torch

    from agent_factory_3_amd import routing as R
    x = torch.zeros(4, 128, dtype=torch.bfloat16)
    w = torch.zeros(8, 128, dtype=torch.bfloat16)
    assert not R.router_kernel_supports(x, w, None)
    with pytest.raises(RuntimeError, match="GPU tensor"):
        R.router_linear(x, w, None)
