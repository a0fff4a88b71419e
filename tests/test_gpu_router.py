"""Router-logit GEMM (af3_router_logits) vs the oracle (quantization.py:653-654).

mlp_forward computes the router logits with this kernel (routing.router_linear)
before the top-k / replay routing; its backward is two plain GEMMs.
"""
import pytest
import torch

from agent_factory_3_amd import routing as R
from agent_factory_3_amd import workloads
from oracle import routing as O
from tests._tol import check_close

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("T,H,E,bias", [(1, 64, 8, True), (37, 128, 32, False), (300, 256, 200, True),
                                        (4096, 2880, 32, True), (16384, 2880, 128, True)])
def test_router_logits_match_oracle(dev, T, H, E, bias):
    g = torch.Generator().manual_seed(T + E)
    x = workloads.normal_bf16(g, (T, H), 1.0)
    w = workloads.normal_bf16(g, (E, H), 1.0 / H)
    b = workloads.normal_bf16(g, (E,), 0.01) if bias else None
    got = R.router_logits_hip(x.to(dev), w.to(dev), b.to(dev) if bias else None)
    ref, mag = O.router_logits(x, w, b)
    check_close(got, ref, mag=mag, n=H, what=f"router logits T={T} H={H} E={E}")


def test_router_logits_strided_rows(dev):
    g = torch.Generator().manual_seed(5)
    xx = workloads.normal_bf16(g, (70, 192), 1.0)
    x = xx[:, :128]                                   # row stride 192
    w = workloads.normal_bf16(g, (40, 128), 0.01)
    got = R.router_logits_hip(x.to(dev), w.to(dev), None)
    ref, mag = O.router_logits(x, w, None)
    check_close(got, ref, mag=mag, n=128, what="strided")


def test_router_linear_autograd(dev):
    """Backward of the router linear: float64 autograd of the same expression."""
    g = torch.Generator().manual_seed(7)
    T, H, E = 96, 128, 32
    x = workloads.normal_bf16(g, (T, H), 1.0)
    w = workloads.normal_bf16(g, (E, H), 0.05)
    b = workloads.normal_bf16(g, (E,), 0.05)
    dl = workloads.normal_bf16(g, (T, E), 1.0)
    xs, ws, bs = (t.to(dev).requires_grad_(True) for t in (x, w, b))
    y = R.router_linear(xs, ws, bs)
    y.backward(dl.to(dev))
    x64, w64, b64 = (t.double().requires_grad_(True) for t in (x, w, b))
    (x64 @ w64.T + b64).backward(dl.double())
    check_close(y, (x.double() @ w.double().T + b.double()), what="forward")
    for got, ref, n in ((xs.grad, x64.grad, E), (ws.grad, w64.grad, T), (bs.grad, b64.grad, T)):
        check_close(got, ref, what="grad")


def test_router_rejects_unsupported_shapes(dev):
    x = torch.zeros(4, 96, dtype=torch.bfloat16, device=dev)
    w = torch.zeros(8, 96, dtype=torch.bfloat16, device=dev)
    with pytest.raises(RuntimeError, match="multiple of 64"):
        R.router_logits_hip(x, w, None)
    with pytest.raises(TypeError):
        R.router_logits_hip(x.float(), w.float(), None)


@pytest.mark.parametrize("case", ["h96", "fp32_weight", "e300"])
def test_router_linear_falls_back_for_operands_the_kernel_does_not_take(dev, case):
    """router_linear (what mlp_forward calls) still gives the reference's
    nn.functional.linear for a router the kernel does not take."""
    g = torch.Generator().manual_seed(11)
    T, H, E = 33, (96 if case == "h96" else 128), (300 if case == "e300" else 16)
    x = workloads.normal_bf16(g, (T, H), 1.0).to(dev)
    w = workloads.normal_bf16(g, (E, H), 0.05).to(dev)
    b = workloads.normal_bf16(g, (E,), 0.05).to(dev)
    if case == "fp32_weight":
        x, w, b = x.float(), w.float(), b.float()
    assert not R.router_kernel_supports(x, w, b)
    got = R.router_linear(x, w, b)
    ref = torch.nn.functional.linear(x, w, b)
    assert got.dtype == ref.dtype and torch.equal(got, ref)
