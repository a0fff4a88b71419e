"""Routing restated with torch CPU ops (test infrastructure only).

* ``routing_replay``  — quantization.py:593-636.
* ``routing_topk``    — quantization.py:551-590 (routing_torch_dist) at world
  size 1: stable descending sort, softmax over the K, per-token sort by id.
* ``router_logits``   — quantization.py:653-654 (nn.functional.linear of the
  hidden states with the router weight and bias): fp32 sums, one bf16 rounding.
* ``expt_data``       — triton_kernels.routing.compute_expt_data_torch as
  called at quantization.py:588,627: token_offs_raw, token_offs_pad[BM] and
  block_pid_map[BM] ((block << 16) | expert, -1 padding).
"""
from __future__ import annotations

import torch


def routing_replay(logits: torch.Tensor, expt_indx: torch.Tensor, k: int):
    """-> dict(gate_scal bf16 [R], hist [E], topk_indx [R], gate_indx [R], offs [E+1])."""
    T, E = logits.shape
    ei = expt_indx.to(torch.long)
    logits_topk = torch.take_along_dim(logits, ei, dim=-1)
    expt_scal = torch.softmax(logits_topk, dim=-1).reshape(-1)
    flat = ei.reshape(-1)
    sorted_expts, topk_indx = torch.sort(flat, stable=True)
    n = topk_indx.numel()
    gate_indx = torch.empty_like(topk_indx)
    gate_indx[topk_indx] = torch.arange(n, dtype=topk_indx.dtype)
    gate_scal = expt_scal[topk_indx]
    hist = torch.bincount(sorted_expts, minlength=E).to(torch.int32)
    offs = torch.zeros(E + 1, dtype=torch.int32)
    offs[1:] = torch.cumsum(hist, 0)
    return dict(gate_scal=gate_scal, hist=hist, topk_indx=topk_indx.to(torch.int32),
                gate_indx=gate_indx.to(torch.int32), offs=offs, expt_indx=ei.to(torch.int32))


def topk_ids(logits: torch.Tensor, k: int):
    """Top-k ids and softmax weights per token, ids of a token ascending (quantization.py:564-576)."""
    tk = torch.argsort(-logits.float(), dim=1, stable=True)[:, :k]
    val = torch.take_along_dim(logits, tk, dim=1)
    scal = torch.softmax(val, dim=-1)
    ids, order = torch.sort(tk, dim=1)
    scal = torch.gather(scal, 1, order)
    return ids.to(torch.int32), scal


def routing_topk(logits: torch.Tensor, k: int):
    ids, scal = topk_ids(logits, k)
    T, E = logits.shape
    flat = ids.reshape(-1).to(torch.long)
    topk_indx = torch.argsort(flat, stable=True)
    gate_indx = torch.argsort(topk_indx)
    gate_scal = scal.reshape(-1)[topk_indx]
    hist = torch.bincount(flat, minlength=E).to(torch.int32)
    offs = torch.zeros(E + 1, dtype=torch.int32)
    offs[1:] = torch.cumsum(hist, 0)
    return dict(gate_scal=gate_scal, hist=hist, topk_indx=topk_indx.to(torch.int32),
                gate_indx=gate_indx.to(torch.int32), offs=offs, expt_indx=ids)


def expt_data(hist: torch.Tensor, block_m: int, max_tiles: int):
    n_tiles = (hist.to(torch.long) + block_m - 1) // block_m
    offs_pad = torch.zeros(hist.numel() + 1, dtype=torch.int32)
    offs_pad[1:] = torch.cumsum(n_tiles, 0)
    pid = -torch.ones(max_tiles, dtype=torch.int32)
    for e in range(hist.numel()):
        o = int(offs_pad[e])
        for b in range(int(n_tiles[e])):
            pid[o + b] = (b << 16) + e
    return offs_pad, pid


def router_logits(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None):
    """-> (bf16 logits [T, E], float32 sum of |x_k w_k| per logit for tolerances)."""
    xf, wf = x.to(torch.float32), weight.to(torch.float32)
    out = xf @ wf.T
    if bias is not None:
        out = out + bias.to(torch.float32)
    return out.to(torch.bfloat16), xf.abs() @ wf.abs().T
