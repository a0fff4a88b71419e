"""Pins oracle.routing (CPU) by invariants and brute force."""
import torch

from oracle import routing


def _brute_sorted(ids):
    flat = ids.reshape(-1).tolist()
    return sorted(range(len(flat)), key=lambda i: (flat[i], i))


def test_replay_invariants_and_brute_force():
    g = torch.Generator().manual_seed(3)
    T, E, K = 97, 9, 3
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16)
    ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32)
    rt = routing.routing_replay(logits, ids, K)
    ti, gi = rt["topk_indx"].long(), rt["gate_indx"].long()
    assert ti.tolist() == _brute_sorted(ids)
    assert (gi[ti] == torch.arange(T * K)).all()
    assert int(rt["hist"].sum()) == T * K
    w = torch.zeros(T, dtype=torch.float64)
    w.index_add_(0, ti // K, rt["gate_scal"].double())
    assert torch.allclose(w, torch.ones(T, dtype=torch.float64), atol=2e-2)
    # each weight is the softmax over the token's K selected logits
    t, j = divmod(int(ti[0]), K)
    sel = logits[t, ids[t].long()].float()
    assert abs(float(rt["gate_scal"][0]) - float(torch.softmax(sel, 0)[j])) < 1e-2


def test_topk_ties_go_to_lower_id():
    logits = torch.zeros(2, 6, dtype=torch.bfloat16)
    logits[1, 5] = 1.0
    ids, scal = routing.topk_ids(logits, 2)
    assert ids[0].tolist() == [0, 1]
    assert ids[1].tolist() == [0, 5]


def test_expt_data_tiles():
    hist = torch.tensor([0, 130, 5, 0, 256], dtype=torch.int32)
    offs_pad, pid = routing.expt_data(hist, 128, 12)
    assert offs_pad.tolist() == [0, 0, 2, 3, 3, 5]
    assert pid[:5].tolist() == [1, (1 << 16) | 1, 2, 4, (1 << 16) | 4]
    assert (pid[5:] == -1).all()


def test_router_logits_oracle_against_float64():
    """oracle.routing.router_logits: fp32 sums of bf16 inputs, one bf16 rounding
    (quantization.py:654's F.linear), within one bf16 rounding of the exact
    float64 value; the magnitude bound dominates the result."""
    g = torch.Generator().manual_seed(11)
    x = torch.randn(64, 2880, generator=g).to(torch.bfloat16)
    w = (torch.randn(128, 2880, generator=g) * 0.02).to(torch.bfloat16)
    b = (torch.randn(128, generator=g) * 0.1).to(torch.bfloat16)
    got, mag = routing.router_logits(x, w, b)
    exact = x.double() @ w.double().T + b.double()
    assert ((got.double() - exact).abs() <= 2.0 ** -8 * exact.abs() + 1e-6).all()
    assert (mag.double() + b.double().abs() >= exact.abs() - 1e-3).all()
    # the reference's own expression on the CPU gives the same bits
    assert torch.equal(got, torch.nn.functional.linear(x.float(), w.float(), b.float()).to(torch.bfloat16))
