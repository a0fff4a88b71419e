"""Routing-weight (gamma) gradients on the GPU (routing.GAMMA_GRAD).

The reference returns no gradient for the routing weights
(quantization.py:421); with GAMMA_GRAD the router logits receive the gradient
of the softmax routing weights.  Checked against float64 autograd of the
dense layer (oracle.moe.dense_reference) with gamma = softmax over each
token's K selected logits, for the fused SwiGLU module path (with and without
expert LoRA) and the unfused DequantMoEMatmul path; the input gradient must be
bit-identical to a run without GAMMA_GRAD, and the default stays the
reference's (no gradient reaches the logits).
"""
import pytest
import torch

from agent_factory_3_amd import quantization as Q
from agent_factory_3_amd import routing as R
from agent_factory_3_amd import workloads
from oracle import moe, mxfp4

pytestmark = pytest.mark.gpu


def _inp(lora):
    inp = workloads.layer(3, T=300, E=8, k=4, H=128, I=128, lora_r=16 if lora else 0, scale_lo=118,
                          scale_hi=121, zipf=False)
    if lora:
        inp.lora = dict(inp.lora, Bgu=inp.lora["Bgu"] * 30, Bdn=inp.lora["Bdn"] * 30)
    return inp


def _run(inp, dev, gamma_grad, fused):
    prev = (R.GAMMA_GRAD, Q.FUSED_SWIGLU)
    R.GAMMA_GRAD, Q.FUSED_SWIGLU = gamma_grad, fused
    try:
        print(f"gamma_grad={gamma_grad} fused={fused} lora={inp.lora is not None}", flush=True)
        m = workloads.make_experts(inp, dev)
        logits = inp.logits.to(dev).requires_grad_(True)
        rd, gi, si = R.routing_replay(logits, inp.expt_indx.to(dev), inp.k)
        x = inp.x.to(dev).requires_grad_(True)
        y = m(x, rd, gi, si)
        y.backward(inp.dy.to(dev))
        torch.cuda.synchronize()
        return x.grad, logits.grad
    finally:
        R.GAMMA_GRAD, Q.FUSED_SWIGLU = prev


def _reference_dlogits(inp):
    p = dict(Wgu=mxfp4.dequant_f32(inp.gu_blocks, inp.gu_scales), bgu=inp.gu_bias,
             Wdn=mxfp4.dequant_f32(inp.dn_blocks, inp.dn_scales), bdn=inp.dn_bias)
    lo = None
    if inp.lora is not None:
        lo = dict(Agu=inp.lora["Agu"], Bgu=inp.lora["Bgu"], Adn=inp.lora["Adn"], Bdn=inp.lora["Bdn"],
                  s=inp.lora["alpha"] / inp.lora["r"])
    ids = inp.expt_indx.long()
    lg = inp.logits.double().requires_grad_(True)
    scal = torch.softmax(torch.take_along_dim(lg, ids, dim=-1), -1)
    Y = moe.dense_reference(inp.x, p, ids, scal, lora=lo)
    Y.backward(inp.dy.double())
    return lg.grad


@pytest.mark.parametrize("lora,fused", [(False, True), (True, True), (False, False)])
def test_router_gradient_through_gammas(dev, lora, fused):
    inp = _inp(lora)
    dx, dlog = _run(inp, dev, True, fused)
    dx0, dlog0 = _run(inp, dev, False, fused)
    assert dlog0 is None                      # the reference's behaviour by default
    assert torch.equal(dx, dx0)               # the input gradient is untouched
    ref = _reference_dlogits(inp)
    got = dlog.float().cpu().double()
    scale = float(ref.abs().max())
    err = (got - ref).abs()
    assert float(err.max()) <= 3e-2 * scale, (float(err.max()), scale)
    assert float((err > 1e-2 * scale + 2e-2 * ref.abs()).float().mean()) < 1e-2
    # unselected logits get exactly zero
    sel = torch.zeros_like(ref, dtype=torch.bool).scatter_(1, inp.expt_indx.long(), True)
    assert bool((got[~sel] == 0).all())


def test_gamma_grad_with_expert_lora_unfused_is_rejected(dev):
    inp = _inp(True)
    with pytest.raises(NotImplementedError):
        _run(inp, dev, True, False)
