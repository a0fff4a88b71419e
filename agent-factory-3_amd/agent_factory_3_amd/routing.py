"""Routing metadata for the grouped expert GEMMs (HIP-backed).

Own restatement of the routing objects the reference imports from the
un-vendored ``triton_kernels`` package (``quantization.py:42-48``) and of the
routing functions built on them:

* ``GatherIndx(src_indx, dst_indx)``, ``ScatterIndx(src_indx, dst_indx)``,
  ``RoutingData(gate_scal, expt_hist, n_expts_tot, n_expts_act, expt_data)``
  with the field order used at ``quantization.py:586-590,632-636``;
* ``ExptData`` / ``compute_expt_data`` (``compute_expt_data_torch`` at
  ``quantization.py:588,627``): raw and padded expert offsets and the
  ``block_pid_map`` that drives the ragged GEMM grid;
* ``routing_replay`` (``quantization.py:593-636``) and top-k ``routing``
  (``routing_torch_dist`` at world size 1, ``quantization.py:551-590``).

All index work runs in HIP kernels on the caller's stream (no host sync).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import torch

from . import _capi

# block sizes for which tile maps are built: 128- and 256-row GEMM tiles and
# the 512-row chunks of the LoRA weight-gradient reduction
BLOCK_MS = (128, 256, 512)
GEMM_ORDER_BMS = (128,)  # tile sizes whose full-first work order is made with the routing (the
# default GEMMs and the LoRA row tiles); other sizes get theirs on first use (gemm_order_for)


@dataclass
class GatherIndx:
    """Row gather: sorted row i reads token ``src_indx[i] // n_expts_act``."""
    src_indx: torch.Tensor
    dst_indx: torch.Tensor


@dataclass
class ScatterIndx:
    """Row scatter: token t sums sorted rows ``src_indx[t*k + j]``."""
    src_indx: torch.Tensor
    dst_indx: torch.Tensor


@dataclass
class ExptData:
    hist: torch.Tensor                      # [E] int32 rows per expert
    token_offs_raw: torch.Tensor            # [E+1] int32 exclusive scan of hist
    token_offs_pad: dict = field(default_factory=dict)  # BM -> [E+1] int32 scan of ceil(hist/BM)
    block_pid_map: dict = field(default_factory=dict)   # BM -> [max_tiles] int32 (b<<16)|e or -1
    # BM -> the block_pid_map entries in grouped-GEMM work order (full tiles
    # first, then partial tiles by decreasing rows); not part of the
    # reference's ExptData, filled for GEMM_ORDER_BMS and by gemm_order_for
    gemm_order: dict = field(default_factory=dict)
    n_gates: int = 0                        # routed rows (for the work orders made on first use)


@dataclass
class RoutingData:
    gate_scal: torch.Tensor | None
    expt_hist: torch.Tensor | None
    n_expts_tot: int
    n_expts_act: int
    expt_data: ExptData | None = None


def max_tiles(n_gates: int, n_expts_tot: int, block_m: int) -> int:
    """Upper bound of sum_e ceil(hist[e]/block_m) given sum_e hist[e] = n_gates."""
    return min(n_gates, (n_gates + block_m - 1) // block_m + n_expts_tot) if n_gates > 0 else 0


_BMS_CACHE: dict = {}


def _block_ms_on(dev) -> torch.Tensor:
    key = (str(dev), BLOCK_MS)
    t = _BMS_CACHE.get(key)
    if t is None:
        t = torch.tensor(BLOCK_MS, dtype=torch.int32).to(dev)
        _BMS_CACHE[key] = t
    return t


def compute_expt_data(hist: torch.Tensor, n_expts_tot: int, n_gates: int,
                      token_offs_raw: torch.Tensor | None = None) -> ExptData:
    """Tile metadata from the expert histogram (compute_expt_data_torch semantics)."""
    dev = hist.device
    hist = hist.to(torch.int32).contiguous()
    if token_offs_raw is None:
        token_offs_raw = torch.zeros(n_expts_tot + 1, dtype=torch.int32, device=dev)
        token_offs_raw[1:] = torch.cumsum(hist, 0)
    bms = _block_ms_on(dev)
    mt = max(max_tiles(n_gates, n_expts_tot, bm) for bm in BLOCK_MS)
    offs_pad = torch.empty(len(BLOCK_MS), n_expts_tot + 1, dtype=torch.int32, device=dev)
    pid_map = torch.empty(len(BLOCK_MS), max(mt, 1), dtype=torch.int32, device=dev)
    _capi.call("af3_expt_data", hist.data_ptr(), n_expts_tot, bms.data_ptr(), len(BLOCK_MS), mt,
               offs_pad.data_ptr(), pid_map.data_ptr(), _capi.stream_of(dev))
    ed = ExptData(hist, token_offs_raw, n_gates=int(n_gates))
    for i, bm in enumerate(BLOCK_MS):
        ed.token_offs_pad[bm] = offs_pad[i]
        ed.block_pid_map[bm] = pid_map[i, :mt]
    for bm in GEMM_ORDER_BMS:
        gemm_order_for(ed, bm)
    return ed


def gemm_order_for(ed: ExptData, bm: int):
    """The grouped-GEMM work order of the bm-row tiles (af3_tile_order), made
    on first use and kept in ed.gemm_order; None where it cannot be made
    (more than 4096 experts, or an ExptData built without n_gates), and the
    callers then take block_pid_map's order."""
    order = ed.gemm_order.get(bm)
    n_expts_tot = ed.hist.numel()
    if order is not None or ed.n_gates <= 0 or n_expts_tot > 4096 or bm not in ed.token_offs_pad:
        return order
    n = max_tiles(ed.n_gates, n_expts_tot, bm)
    order = torch.empty(max(n, 1), dtype=torch.int32, device=ed.hist.device)
    _capi.call("af3_tile_order", ed.hist.data_ptr(), n_expts_tot, bm, ed.token_offs_pad[bm].data_ptr(), n,
               order.data_ptr(), _capi.stream_of(ed.hist.device))
    ed.gemm_order[bm] = order[:n]
    return ed.gemm_order[bm]


# the reference's name (triton_kernels.routing.compute_expt_data_torch)
def compute_expt_data_torch(hist, n_expts_tot, n_gates):
    return compute_expt_data(hist, n_expts_tot, n_gates)


def _bf16_logits(logits: torch.Tensor) -> torch.Tensor:
    if not logits.is_cuda:
        raise RuntimeError("router logits must be a GPU tensor (the MI355X path has no CPU implementation)")
    if logits.dtype != torch.bfloat16:
        logits = logits.to(torch.bfloat16)
    if logits.stride(-1) != 1:
        logits = logits.contiguous()
    return logits


# Routing-weight (gamma) gradients.  The reference's expert layer returns no gradient
# for the routing weights (quantization.py:421), so its router only learns through
# other paths; with GAMMA_GRAD set, gate_scal stays attached to the router logits
# (softmax over each token's K selected logits) and the down projection returns
# d gamma, so a trainable router receives the gradient of the routing weights.
GAMMA_GRAD = False


class _GateScal(torch.autograd.Function):
    """gate_scal (sorted rows) as a differentiable function of the router logits:
    forward passes the routing kernel's softmax weights through; backward is the
    softmax backward over each token's K slots, scattered to the selected logits."""

    @staticmethod
    def forward(ctx, logits, gate_scal, topk_indx, hist, K):
        ctx.save_for_backward(gate_scal, topk_indx, hist)
        ctx.K, ctx.shape, ctx.dtype = int(K), tuple(logits.shape), logits.dtype
        return gate_scal.view_as(gate_scal)

    @staticmethod
    def backward(ctx, grad):
        gs, topk, hist = ctx.saved_tensors
        T, E = ctx.shape
        K = ctx.K
        R = T * K
        dev = gs.device
        tk = topk.long()
        gam = torch.empty(R, dtype=torch.float32, device=dev)
        gam[tk] = gs.float()
        d = torch.empty(R, dtype=torch.float32, device=dev)
        d[tk] = grad.float()
        ids = torch.empty(R, dtype=torch.long, device=dev)
        ids[tk] = torch.repeat_interleave(torch.arange(E, device=dev), hist.long(), output_size=R)
        gam, d, ids = gam.view(T, K), d.view(T, K), ids.view(T, K)
        dl = gam * (d - (gam * d).sum(-1, keepdim=True))
        dlogits = torch.zeros(T, E, dtype=torch.float32, device=dev).scatter_add_(1, ids, dl)
        return dlogits.to(ctx.dtype), None, None, None, None


def _run_routing(logits: torch.Tensor, n_expts_act: int, expt_indx: torch.Tensor | None):
    out_dtype = logits.dtype
    lg = _bf16_logits(logits)
    T, E = lg.shape
    K = int(n_expts_act)
    R = T * K
    dev = lg.device
    gate_scal = torch.empty(R, dtype=torch.bfloat16, device=dev)
    hist = torch.empty(E, dtype=torch.int32, device=dev)
    topk_indx = torch.empty(R, dtype=torch.int32, device=dev)
    gate_indx = torch.empty(R, dtype=torch.int32, device=dev)
    offs = torch.empty(E + 1, dtype=torch.int32, device=dev)
    ws_n = _capi.workspace_bytes(T, E, K)
    ws = torch.empty(ws_n, dtype=torch.uint8, device=dev)
    stream = _capi.stream_of(dev)
    ld = lg.stride(0) if T > 1 else E
    if expt_indx is not None:
        ei = expt_indx.to(device=dev, dtype=torch.int32).contiguous()
        if ei.shape != (T, K):
            raise ValueError(f"expt_indx shape {tuple(ei.shape)} != ({T}, {K})")
        _capi.call("af3_routing_replay", lg.data_ptr(), ld, ei.data_ptr(), T, E, K, gate_scal.data_ptr(),
                   hist.data_ptr(), topk_indx.data_ptr(), gate_indx.data_ptr(), offs.data_ptr(), ws.data_ptr(),
                   ws_n, stream)
    else:
        _capi.call("af3_routing_topk", lg.data_ptr(), ld, T, E, K, gate_scal.data_ptr(), hist.data_ptr(),
                   topk_indx.data_ptr(), gate_indx.data_ptr(), offs.data_ptr(), ws.data_ptr(), ws_n, stream)
    expt_data = compute_expt_data(hist, E, R, token_offs_raw=offs)
    if out_dtype != torch.bfloat16 and out_dtype.is_floating_point:
        gate_scal = gate_scal.to(out_dtype)
    if GAMMA_GRAD and torch.is_grad_enabled() and logits.requires_grad:
        gate_scal = _GateScal.apply(logits, gate_scal, topk_indx, hist, K)
    return (
        RoutingData(gate_scal, hist, E, K, expt_data),
        GatherIndx(src_indx=topk_indx, dst_indx=gate_indx),
        ScatterIndx(src_indx=gate_indx, dst_indx=topk_indx),
    )


def routing_replay(logits: torch.Tensor, expt_indx: torch.Tensor, n_expts_act: int):
    """Routing structures from given expert ids (quantization.py:593-636).

    Args:
        logits: [T, E] router logits (softmax over the K selected only)
        expt_indx: [T, K] int expert ids per token
        n_expts_act: K
    Returns:
        (RoutingData, GatherIndx, ScatterIndx)
    """
    return _run_routing(logits, n_expts_act, expt_indx)


def routing(logits: torch.Tensor, n_expts_act: int, sm_first: bool = False, expt_indx=None,
            simulated_ep: int = 1, n_rows=None):
    """Top-k routing with the call signature of triton_kernels.routing.routing.

    Top-``n_expts_act`` logits per token (ties to the lower expert id), softmax
    over the selected ones, ids of a token ordered by expert id
    (quantization.py:564-576).  ``expt_indx`` given -> replay.
    """
    if sm_first:
        raise NotImplementedError("sm_first=True is not used on the gpt-oss path")
    if simulated_ep != 1:
        raise NotImplementedError("simulated expert parallelism is not supported (single GPU)")
    if n_rows is not None:
        logits = logits[:n_rows]
    return _run_routing(logits, n_expts_act, expt_indx)


def dense_routing(n_rows: int, device) -> RoutingData:
    """Single-expert routing (matmul_ogs with routing_data=None)."""
    hist = torch.tensor([n_rows], dtype=torch.int32, device=device)
    return RoutingData(None, hist, 1, 1, compute_expt_data(hist, 1, n_rows))


# ---------------------------------------------------------------------------
# router logits (quantization.py:653-654: nn.functional.linear(hidden, router.weight, router.bias))
# ---------------------------------------------------------------------------

def router_logits_hip(hidden: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """logits [T, E] bf16 = bf16(hidden @ weight^T + bias) with fp32 sums (af3_router_logits).
    hidden [T, H] bf16, weight [E, H] bf16, bias [E] bf16 or None; H % 64 == 0, E <= 256."""
    if not hidden.is_cuda:
        raise RuntimeError("router_logits: hidden must be a GPU tensor (no CPU implementation)")
    for name, t in (("hidden", hidden), ("weight", weight)) + ((("bias", bias),) if bias is not None else ()):
        if t.dtype != torch.bfloat16:
            raise TypeError(f"router_logits: {name} must be bfloat16 (got {t.dtype})")
    x = hidden if hidden.stride(-1) == 1 and hidden.data_ptr() % 16 == 0 and hidden.stride(0) % 8 == 0 \
        else hidden.contiguous()
    w = weight.contiguous()
    T, H = x.shape
    E = w.shape[0]
    if w.shape[1] != H:
        raise ValueError(f"router_logits: weight is {tuple(w.shape)}, hidden has {H} columns")
    b = bias.contiguous() if bias is not None else None
    out = torch.empty(T, E, dtype=torch.bfloat16, device=x.device)
    if T:
        _capi.call("af3_router_logits", x.data_ptr(), x.stride(0) if T > 1 else H, w.data_ptr(), w.stride(0),
                   _capi.ptr(b), T, H, E, out.data_ptr(), E, _capi.stream_of(x.device))
    return out


class RouterLinear(torch.autograd.Function):
    """Router logits with the HIP kernel in the forward; the backward (needed
    only when a loss reads the logits, e.g. routing-weight gradients or an
    auxiliary loss) is two plain GEMMs and a column sum, as F.linear's."""

    @staticmethod
    def forward(ctx, hidden, weight, bias):
        ctx.save_for_backward(hidden, weight)
        ctx.has_bias = bias is not None
        return router_logits_hip(hidden, weight, bias)

    @staticmethod
    def backward(ctx, g):
        hidden, weight = ctx.saved_tensors
        g = g.to(torch.bfloat16)
        dh = g @ weight if ctx.needs_input_grad[0] else None
        dw = g.t() @ hidden if ctx.needs_input_grad[1] else None
        db = g.float().sum(0).to(torch.bfloat16) if ctx.has_bias and ctx.needs_input_grad[2] else None
        return dh, dw, db


def router_kernel_supports(hidden: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> bool:
    """Whether af3_router_logits takes these operands: GPU tensors, all bf16,
    hidden [T, H] / weight [E, H] with H % 64 == 0 and E <= 256."""
    ts = (hidden, weight) + ((bias,) if bias is not None else ())
    return (all(t.is_cuda and t.dtype == torch.bfloat16 for t in ts) and hidden.dim() == 2 and weight.dim() == 2
            and weight.shape[1] == hidden.shape[1] and hidden.shape[1] % 64 == 0 and 0 < weight.shape[0] <= 256
            and (bias is None or bias.shape == (weight.shape[0],)))


def router_linear(hidden: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None) -> torch.Tensor:
    """The router's nn.functional.linear (quantization.py:654), on the HIP
    kernel (autograd-aware) for the operands it takes (gpt-oss: bf16, H = 2880,
    E = 32 / 128).  Other GPU operands (another dtype, H % 64 != 0, E > 256)
    go to nn.functional.linear as in the reference, so such a router still
    works; CPU operands raise, as the expert layer after it needs the GPU."""
    if not hidden.is_cuda:
        raise RuntimeError("router_logits: hidden must be a GPU tensor (no CPU implementation)")
    if not router_kernel_supports(hidden, weight, bias):
        return torch.nn.functional.linear(hidden, weight, bias)
    return RouterLinear.apply(hidden, weight, bias)
