"""af3_routing_replay_noalloc (the allocation-free routing entry point) against
af3_routing_replay with a caller workspace, through the C ABI.

Two calls in a row on one device, the second with a smaller input, so the
second runs over the first call's leftovers in the built-in scratch array;
outputs must equal the workspace entry point's bit for bit.  (The rejection
of shapes beyond the array is checked on the CPU in tests/test_capi.py.)
"""
import pytest
import torch

from agent_factory_3_amd import _capi, workloads

pytestmark = pytest.mark.gpu


def _outputs(T, E, K, dev):
    R = T * K
    return dict(gate_scal=torch.empty(R, dtype=torch.bfloat16, device=dev),
                hist=torch.empty(E, dtype=torch.int32, device=dev),
                topk_indx=torch.empty(R, dtype=torch.int32, device=dev),
                gate_indx=torch.empty(R, dtype=torch.int32, device=dev),
                offs=torch.empty(E + 1, dtype=torch.int32, device=dev))


def _args(o):
    return (o["gate_scal"].data_ptr(), o["hist"].data_ptr(), o["topk_indx"].data_ptr(), o["gate_indx"].data_ptr(),
            o["offs"].data_ptr())


def _case(T, E, K, seed, dev, zipf, own_stream=False):
    g = torch.Generator().manual_seed(seed)
    logits = workloads.normal_bf16(g, (T, E), 1.0).to(dev)
    if zipf:
        ids = workloads.zipf_routing(g, T, E, K, n_idle=8).to(dev)
    else:
        ids = torch.stack([torch.randperm(E, generator=g)[:K] for _ in range(T)]).to(torch.int32).to(dev)
    stream = _capi.stream_of(dev)
    side = torch.cuda.Stream(device=dev) if own_stream else None   # default priority
    if side is not None:
        torch.cuda.synchronize()
    ref = _outputs(T, E, K, dev)
    ws = torch.empty(_capi.workspace_bytes(T, E, K), dtype=torch.uint8, device=dev)
    _capi.call("af3_routing_replay", logits.data_ptr(), E, ids.data_ptr(), T, E, K, *_args(ref), ws.data_ptr(),
               ws.numel(), stream)
    got = _outputs(T, E, K, dev)
    for o in got.values():
        o.fill_(0x55) if o.dtype != torch.bfloat16 else o.fill_(-3.0)
    torch.cuda.synchronize()
    # (a stream object of its own: the scratch array is the one of the stream's device)
    _capi.call("af3_routing_replay_noalloc", logits.data_ptr(), E, ids.data_ptr(), T, E, K, *_args(got),
               side.cuda_stream if side is not None else stream)
    torch.cuda.synchronize()
    for k in ref:
        a, b = got[k].cpu(), ref[k].cpu()
        if a.dtype == torch.bfloat16:
            a, b = a.view(torch.int16), b.view(torch.int16)
        assert torch.equal(a, b), (T, E, K, k)


def test_noalloc_matches_workspace_entry_point_two_calls(dev):
    assert int(_capi.load().af3_routing_scratch_bytes()) == 4 << 20
    _case(16384, 128, 4, 1, dev, zipf=True)    # the 120b layer's routing (Zipf, idle experts)
    _case(3000, 32, 4, 2, dev, zipf=False)     # smaller, over the first call's leftovers
    _case(37, 6, 2, 3, dev, zipf=False)
    _case(2000, 64, 4, 4, dev, zipf=False, own_stream=True)

