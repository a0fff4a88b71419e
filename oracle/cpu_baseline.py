"""PyTorch-eager CPU baseline of the MoE expert layer (reported baseline, not the target).

The reference's eager path restated for the CPU: transformers-style MXFP4
dequant (LUT + ldexp, quantization.py:137-163) of every expert's weights,
then the per-expert bf16 matmul loop of GptOssExperts.forward
(transformers/models/gpt_oss/modeling_gpt_oss.py, expert loop over routed
tokens) with gpt-oss's clamped SwiGLU, the expert-LoRA deltas, and torch
autograd for the backward.  Test/bench infrastructure only.

``run_layer`` times the whole layer once, unscaled: every expert's weights
dequantized for the forward, the per-expert loop (forward + autograd
backward) over all routed rows with each token's k weighted rows added into
the layer output and the rows' input gradients added into dX, and every
expert's weights dequantized again for the backward (DequantMoEMatmul
re-derives them, quantization.py:364-373); a forward-only workload (no output
gradient) runs the forward part alone.
``run_dequant`` / ``run_swiglu`` time the standalone dequant (cfg0) and
SwiGLU forward + backward (cfg1).
``run_sample`` times a bounded sample (the rows of a few experts, fwd + bwd,
plus the dequant of those experts) and scales it to the whole layer:
    t_layer = t_dequant_per_expert * E * 2   (forward and backward re-dequant,
                                              as DequantMoEMatmul does)
            + t_loop_per_row * T * K
"""
from __future__ import annotations

import os
import time

import torch

from . import mxfp4 as _mx

ALPHA, LIMIT = 1.702, 7.0


def _swiglu(gu):
    gate, up = gu[..., 0::2], gu[..., 1::2]
    gate = gate.clamp(max=LIMIT)
    up = up.clamp(min=-LIMIT, max=LIMIT)
    return (up + 1) * (gate * torch.sigmoid(gate * ALPHA))


def threads() -> int:
    """Every core this process may run on (its affinity mask), limited only by
    OMP_NUM_THREADS where the environment sets it (the GPU box sets it to the
    one-GPU share of the host)."""
    n = len(os.sched_getaffinity(0))
    cap = os.environ.get("OMP_NUM_THREADS")
    return max(1, min(n, int(cap))) if cap and cap.isdigit() and int(cap) > 0 else n


def host_info() -> dict:
    """CPU model, affinity core count and the OMP_NUM_THREADS setting of this host."""
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"cpu_model": model, "affinity_cores": len(os.sched_getaffinity(0)),
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS"), "threads": threads()}


def _expert_step(inp, e, W, ids, gam, s, acc):
    """Forward (+ autograd backward when the workload has an output gradient) of
    expert e's routed rows, combined into the layer's outputs the way
    GptOssExperts.forward does (``next_states.index_add_`` of the weighted rows
    in the activation dtype): ``acc["Y"]`` [T, H] bf16, and with a gradient
    ``acc["dX"]`` [T, H] fp32 (the expert's input-row gradients added at their
    tokens) and the expert's LoRA gradients in ``acc["lora"]``.  Returns the
    row count."""
    lora = inp.lora
    tok, slot = torch.nonzero(ids == e, as_tuple=True)
    if tok.numel() == 0:
        return 0
    Wgu, Wdn = W
    if inp.dy is None:
        with torch.no_grad():
            xe = inp.x[tok]
            act = _swiglu(xe @ Wgu.T + inp.gu_bias[e])
            y = (act @ Wdn.T + inp.dn_bias[e]) * gam[tok, slot, None]
            acc["Y"].index_add_(0, tok, y.to(acc["Y"].dtype))
        return tok.numel()
    xe = inp.x[tok].clone().requires_grad_(True)
    gu = xe @ Wgu.T + inp.gu_bias[e]
    if lora:
        A, B = (lora["Agu"][e].clone().requires_grad_(True), lora["Bgu"][e].clone().requires_grad_(True))
        gu = gu + ((xe @ A.T) @ B.T) * s
    act = _swiglu(gu)
    y = act @ Wdn.T + inp.dn_bias[e]
    if lora:
        A2, B2 = (lora["Adn"][e].clone().requires_grad_(True), lora["Bdn"][e].clone().requires_grad_(True))
        y = y + ((act @ A2.T) @ B2.T) * s
    y = y * gam[tok, slot, None]
    acc["Y"].index_add_(0, tok, y.detach().to(acc["Y"].dtype))
    y.backward(inp.dy[tok])
    acc["dX"].index_add_(0, tok, xe.grad.float())
    if lora:
        for name, t in (("Agu", A), ("Bgu", B), ("Adn", A2), ("Bdn", B2)):
            acc["lora"][name][e] = t.grad
    return tok.numel()


def run_layer(inp, warmup: int = 1, runs: int = 1) -> dict:
    """The whole layer on the CPU (inp: workloads.LayerInputs on the CPU):
    ``warmup`` untimed passes, then the median of ``runs`` timed passes."""
    torch.set_num_threads(threads())
    res = [_layer_once(inp) for _ in range(warmup + runs)][warmup:]
    res.sort(key=lambda r: r["t_layer_s"])
    out = dict(res[len(res) // 2])
    out.update(host_info(), warmup=warmup, runs=runs)
    return out


def _layer_once(inp, keep: bool = False) -> dict:
    """One timed pass over the whole layer.  ``keep``: also return the layer's
    outputs (Y, and with a gradient dX and the LoRA gradients) for checking."""
    E = inp.gu_blocks.shape[0]
    ids = inp.expt_indx.long()
    T = inp.x.shape[0]
    gam = torch.softmax(torch.take_along_dim(inp.logits, ids, 1), dim=-1)
    s = (inp.lora["alpha"] / inp.lora["r"]) if inp.lora else 0.0
    acc = {"Y": torch.zeros_like(inp.x)}
    if inp.dy is not None:
        acc["dX"] = torch.zeros(inp.x.shape, dtype=torch.float32)
        if inp.lora:
            acc["lora"] = {k: torch.zeros_like(inp.lora[k]) for k in ("Agu", "Bgu", "Adn", "Bdn")}

    def dequant_all():
        return [(_mx.dequant_lut_ldexp(inp.gu_blocks[e], inp.gu_scales[e]),
                 _mx.dequant_lut_ldexp(inp.dn_blocks[e], inp.dn_scales[e])) for e in range(E)]

    t0 = time.perf_counter()
    W = dequant_all()
    t1 = time.perf_counter()
    rows = sum(_expert_step(inp, e, W[e], ids, gam, s, acc) for e in range(E))
    dX = acc["dX"].to(inp.x.dtype) if "dX" in acc else None
    t2 = time.perf_counter()
    del W
    if inp.dy is not None:
        W = dequant_all()  # the backward re-dequant
        del W
    t3 = time.perf_counter()
    t_layer = t3 - t0
    t_deq = (t1 - t0) + (t3 - t2)
    n_deq = 2 * E if inp.dy is not None else E
    out = dict(tokens_per_s=T / t_layer, t_layer_s=t_layer, dequant_s=t_deq, dequant_s_per_expert=t_deq / n_deq,
               loop_s=t2 - t1, loop_s_per_row=(t2 - t1) / max(1, rows), rows=rows,
               threads_used=torch.get_num_threads())
    if keep:
        out["outputs"] = dict(Y=acc["Y"], dX=dX, lora=acc.get("lora"))
    return out


def _median_time(fn, warmup=1, runs=3) -> float:
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def run_dequant(blocks, scales) -> dict:
    """cfg0 on the CPU: the LUT + ldexp dequant of one weight (median of 3 after a warm-up)."""
    torch.set_num_threads(threads())
    t = _median_time(lambda: _mx.dequant_lut_ldexp(blocks, scales))
    return dict(seconds=t, threads=torch.get_num_threads())


def run_swiglu(gate_up, dout) -> dict:
    """cfg1 on the CPU: the clamped SwiGLU forward + autograd backward in bf16 eager
    (median of 3 after a warm-up)."""
    torch.set_num_threads(threads())

    def once():
        g = gate_up.clone().requires_grad_(True)
        _swiglu(g).backward(dout)
    t = _median_time(once)
    return dict(seconds=t, threads=torch.get_num_threads())


def run_sample(inp, ranks=(0, 10, 60, 110)) -> dict:
    """inp: workloads.LayerInputs on the CPU.  ``ranks`` picks sample experts by popularity."""
    torch.set_num_threads(threads())
    E = inp.gu_blocks.shape[0]
    K = inp.k
    ids = inp.expt_indx.long()
    hist = torch.bincount(ids.flatten(), minlength=E)
    order = torch.argsort(-hist, stable=True)
    experts = [int(order[r]) for r in ranks if r < E and int(hist[order[r]]) > 0]
    T, H = inp.x.shape
    gam = torch.softmax(torch.take_along_dim(inp.logits, ids, 1), dim=-1)
    lora = inp.lora
    s = (lora["alpha"] / lora["r"]) if lora else 0.0

    # dequant of the sample experts (both projections)
    t0 = time.perf_counter()
    W = {}
    for e in experts:
        W[e] = (_mx.dequant_lut_ldexp(inp.gu_blocks[e], inp.gu_scales[e]),
                _mx.dequant_lut_ldexp(inp.dn_blocks[e], inp.dn_scales[e]))
    t_deq = (time.perf_counter() - t0) / max(1, len(experts))

    # per-expert loop, forward + backward (torch autograd), bf16 eager
    rows = 0
    t0 = time.perf_counter()
    for e in experts:
        tok, slot = torch.nonzero(ids == e, as_tuple=True)
        rows += tok.numel()
        xe = inp.x[tok].clone().requires_grad_(True)
        Wgu, Wdn = W[e]
        params = []
        gu = xe @ Wgu.T + inp.gu_bias[e]
        if lora:
            A, B = (lora["Agu"][e].clone().requires_grad_(True), lora["Bgu"][e].clone().requires_grad_(True))
            params += [A, B]
            gu = gu + ((xe @ A.T) @ B.T) * s
        act = _swiglu(gu)
        y = act @ Wdn.T + inp.dn_bias[e]
        if lora:
            A2, B2 = (lora["Adn"][e].clone().requires_grad_(True), lora["Bdn"][e].clone().requires_grad_(True))
            params += [A2, B2]
            y = y + ((act @ A2.T) @ B2.T) * s
        y = y * gam[tok, slot, None]
        y.backward(inp.dy[tok])
    t_loop = time.perf_counter() - t0
    per_row = t_loop / max(1, rows)
    t_layer = t_deq * E * 2 + per_row * T * K
    return dict(tokens_per_s=T / t_layer, t_layer_s=t_layer, dequant_s_per_expert=t_deq,
                loop_s_per_row=per_row, sample_experts=experts, sample_rows=rows, threads=torch.get_num_threads(),
                sample_wall_s=t_deq * len(experts) + t_loop)
