"""Expert-LoRA merge for weight sync (af3_mxfp4_lora_merge) on the GPU.

Against oracle.moe.lora_merge (the reference's merge arithmetic,
model_trainer.py:710-712, over the MXFP4 dequant): bit-exact where the r-term
sum is exact in fp32 (grid-valued adapters, every scale byte 0..255) and for
B = 0 (the dequant itself); within one bf16 step elsewhere, because the
MFMA's fp32 accumulation order differs from an exact sum rounded once (where
base and delta cancel, a few fp32 ulps of the summed magnitudes).  Both
output layouts, partial 64x64 tiles, ranks 8-64 (prefetching kernel) and 136
(the general kernel for ranks above 64).  End to end: the merged
[E, K, N] weights loaded into transformers' own GptOssExperts reproduce the
drop-in module's LoRA forward.
"""
import numpy as np
import pytest
import torch
from torch import nn

from agent_factory_3_amd import kernels
from agent_factory_3_amd import quantization as Q
from agent_factory_3_amd import routing as R
from agent_factory_3_amd import workloads
from oracle import moe, mxfp4

pytestmark = pytest.mark.gpu


def _inputs(E, N, G, r, seed, lo=118, hi=130):
    g = torch.Generator().manual_seed(seed)
    blocks = torch.randint(0, 256, (E, N, G, 16), generator=g, dtype=torch.uint8)
    scales = torch.randint(lo, hi + 1, (E, N, G), generator=g, dtype=torch.uint8)
    A = (torch.randn(E, r, 32 * G, generator=g) * 0.1).to(torch.bfloat16)
    B = (torch.randn(E, N, r, generator=g) * 0.05).to(torch.bfloat16)
    return blocks, scales, A, B


def _bits(t):
    return t.detach().cpu().contiguous().view(torch.int16).numpy().astype(np.int64)


def _check_close(got, blocks, scales, A, B, s, layout, max_frac):
    """Within one bf16 step of the oracle, or, where base and delta cancel, within a
    few fp32 ulps of the magnitudes summed (the accumulation order is not fixed)."""
    ref = moe.lora_merge(blocks, scales, A, B, s, layout)
    assert got.shape == ref.shape
    d = np.abs(_bits(got) - _bits(ref))
    mag = mxfp4.dequant_f32(blocks, scales).double().abs()
    mag += s * torch.matmul(B.double().abs(), A.double().abs())
    if layout == "hf":
        mag = mag.transpose(1, 2)
    err = (got.detach().cpu().double() - ref.double()).abs()
    ok = torch.from_numpy(d <= 1) | (err <= 2.0 ** -20 * mag)
    assert bool(ok.all()), float((err / mag.clamp_min(1e-30))[~ok].max())
    assert (d > 0).mean() < max_frac


def _merge(dev, blocks, scales, A, B, s, layout):
    print(f"merge E,N,G,r={tuple(blocks.shape[:3]) + (A.shape[1],)} layout={layout}", flush=True)
    out = kernels.mxfp4_lora_merge(blocks.to(dev), scales.to(dev), A.to(dev), B.to(dev), s, layout)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("E,N,G,r", [(3, 96, 3, 8), (2, 64, 2, 16), (2, 130, 5, 32), (1, 36, 2, 64),
                                     (2, 70, 3, 136)])
@pytest.mark.parametrize("layout", ["rows", "hf"])
def test_merge_within_one_step(dev, E, N, G, r, layout):
    blocks, scales, A, B = _inputs(E, N, G, r, seed=E * 1000 + N + r)
    s = 32.0 / r
    got = _merge(dev, blocks, scales, A, B, s, layout)
    _check_close(got, blocks, scales, A, B, s, layout, 2e-3)


@pytest.mark.parametrize("layout", ["rows", "hf"])
def test_merge_exact_sums_every_scale_byte(dev, layout):
    # adapters on a 2^-4 / 2^-3 grid: the r-term sum is exact in fp32 in any order,
    # so the kernel must equal the oracle bit for bit, including the integer-rule
    # scale bytes 0, 1, 253-255 (flush to zero) planted across the tile
    E, N, G, r = 2, 100, 6, 24
    blocks, _, _, _ = _inputs(E, N, G, r, seed=77)
    scales = (torch.arange(E * N * G) % 256).to(torch.uint8).reshape(E, N, G)
    g = torch.Generator().manual_seed(78)
    A = (torch.randint(-8, 9, (E, r, 32 * G), generator=g).double() / 16).to(torch.bfloat16)
    B = (torch.randint(-8, 9, (E, N, r), generator=g).double() / 8).to(torch.bfloat16)
    got = _merge(dev, blocks, scales, A, B, 0.5, layout)
    ref = moe.lora_merge(blocks, scales, A, B, 0.5, layout)
    assert (_bits(got) == _bits(ref)).all()


def test_merge_with_zero_b_is_the_dequant(dev):
    blocks, scales, A, B = _inputs(2, 64, 4, 16, seed=3)
    got = _merge(dev, blocks, scales, A, torch.zeros_like(B), 2.0, "rows")
    deq = kernels.mxfp4_to_bf16_hip(blocks.to(dev), scales.to(dev))
    want = _bits(deq)
    want[want == -0x8000] = 0            # -0.0 + 0.0 = +0.0 in the fp32 add
    assert (_bits(got) == want).all()


def test_merge_gpt_oss_shape(dev):
    blocks, scales, A, B = _inputs(2, 5760, 90, 32, seed=11)
    got = _merge(dev, blocks, scales, A, B, 1.0, "hf")
    assert got.shape == (2, 2880, 5760)
    _check_close(got, blocks, scales, A, B, 1.0, "hf", 1e-3)


def test_merge_argument_errors(dev):
    blocks, scales, A, B = _inputs(1, 64, 2, 16, seed=1)
    with pytest.raises(ValueError):
        kernels.mxfp4_lora_merge(blocks.to(dev), scales.to(dev), A[:, :, :32].to(dev), B.to(dev), 1.0)
    with pytest.raises(RuntimeError):   # rank not a multiple of 8: rejected by the C ABI
        kernels.mxfp4_lora_merge(blocks.to(dev), scales.to(dev), A[:, :12].to(dev), B[..., :12].to(dev), 1.0)


def _nest(experts, peft_prefix):
    layer = nn.Module()
    layer.mlp = nn.Module()
    layer.mlp.experts = experts
    inner = nn.Module()
    inner.model = nn.Module()
    inner.model.layers = nn.ModuleList([layer])
    if not peft_prefix:
        return inner
    outer = nn.Module()
    outer.base_model = nn.Module()
    outer.base_model.model = inner
    return outer


@pytest.mark.parametrize("peft_prefix", [False, True])
def test_merged_state_dict_in_transformers_experts(dev, peft_prefix):
    from transformers import GptOssConfig
    from transformers.models.gpt_oss.modeling_gpt_oss import GptOssExperts

    T, E, k, H, I, r = 37, 4, 2, 64, 64, 16
    inp = workloads.layer(3, T=T, E=E, k=k, H=H, I=I, lora_r=r, scale_lo=118, scale_hi=121)
    inp.lora["Bgu"] = (inp.lora["Bgu"].float() * 40).to(torch.bfloat16)   # make the delta visible
    inp.lora["Bdn"] = (inp.lora["Bdn"].float() * 40).to(torch.bfloat16)
    m = workloads.make_experts(inp, dev)
    model = _nest(m, peft_prefix)
    sd = Q.build_merged_expert_state_dict(model, to_cpu=False)
    assert sorted(sd) == ["model.layers.0.mlp.experts.down_proj", "model.layers.0.mlp.experts.gate_up_proj"]
    gu, dn = sd["model.layers.0.mlp.experts.gate_up_proj"], sd["model.layers.0.mlp.experts.down_proj"]
    assert gu.shape == (E, H, 2 * I) and dn.shape == (E, I, H) and gu.dtype == torch.bfloat16

    rd, gi, si = R.routing_replay(inp.logits.to(dev), inp.expt_indx.to(dev), k)
    with torch.no_grad():
        ours = m(inp.x.to(dev), rd, gi, si).float()

    cfg = GptOssConfig(hidden_size=H, intermediate_size=I, num_local_experts=E, num_experts_per_tok=k,
                       num_hidden_layers=1, num_attention_heads=2, num_key_value_heads=1, head_dim=32,
                       vocab_size=128)
    cfg._experts_implementation = "eager"
    hf = GptOssExperts(cfg).to(device=dev, dtype=torch.bfloat16)
    ids = inp.expt_indx.long().to(dev)
    wts = torch.softmax(inp.logits.to(dev).float().gather(1, ids), -1).to(torch.bfloat16)
    with torch.no_grad():
        hf.gate_up_proj_bias.copy_(inp.gu_bias)
        hf.down_proj_bias.copy_(inp.dn_bias)
        hf.gate_up_proj.copy_(gu)
        hf.down_proj.copy_(dn)
        merged = hf(inp.x.to(dev), ids, wts).float()
        hf.gate_up_proj.copy_(kernels.mxfp4_to_bf16_hip(inp.gu_blocks.to(dev), inp.gu_scales.to(dev)).transpose(1, 2))
        hf.down_proj.copy_(kernels.mxfp4_to_bf16_hip(inp.dn_blocks.to(dev), inp.dn_scales.to(dev)).transpose(1, 2))
        base = hf(inp.x.to(dev), ids, wts).float()
    scale = float(ours.abs().max())
    err = float((merged - ours).abs().max())
    assert err <= 2e-2 * scale, (err, scale)
    # the adapters move the output far more than the merge's rounding does
    assert float((base - ours).abs().max()) > 10 * err
