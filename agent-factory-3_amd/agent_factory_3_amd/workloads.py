"""Seeded synthetic inputs of the benchmark configurations (CPU-generated).

Every tensor is drawn on the CPU from ``torch.Generator().manual_seed(20260000
+ cfg)`` so the GPU path and any CPU baseline see identical bits; callers move
them to the device.  ``N(0, v)`` takes a variance, as in the configuration
text ("N(0, 3^2)").

cfg 0  MXFP4 dequant of one gate_up weight [5760, 2880]
cfg 1  clamped SwiGLU fwd/bwd, 8192 rows, gate_up N(0, 9), dO N(0, 1)
cfg 2  gpt-oss-20b layer forward, T=4096, E=32, top-4
cfg 3  gpt-oss-20b layer fwd+bwd, T=16384, E=32, top-4, expert LoRA r=16
cfg 4  gpt-oss-120b layer fwd+bwd, T=16384, E=128, top-4, Zipf(1.1) routing
       with 8 idle experts, expert LoRA r=32
"""
from __future__ import annotations

from dataclasses import dataclass

import numpy as np
import torch

HIDDEN = 2880
INTER = 2880
SEED_BASE = 20260000


def gen(cfg: int) -> torch.Generator:
    return torch.Generator().manual_seed(SEED_BASE + cfg)


def mxfp4_weight(g: torch.Generator, shape_rows: tuple, k: int, scale_lo: int = 118, scale_hi: int = 130):
    """Packed codes uniform over all 16 nibbles, e8m0 scales uniform in [lo, hi]."""
    G = k // 32
    blocks = torch.randint(0, 256, (*shape_rows, G, 16), generator=g, dtype=torch.uint8)
    scales = torch.randint(scale_lo, scale_hi + 1, (*shape_rows, G), generator=g, dtype=torch.uint8)
    return blocks, scales


def normal_bf16(g: torch.Generator, shape, var: float) -> torch.Tensor:
    return (torch.randn(shape, generator=g, dtype=torch.float32) * float(np.sqrt(var))).to(torch.bfloat16)


def cfg0(rows: int = 2 * INTER, k: int = HIDDEN):
    g = gen(0)
    return mxfp4_weight(g, (rows,), k)


def cfg1(M: int = 8192, N: int = INTER):
    g = gen(1)
    gu = normal_bf16(g, (M, 2 * N), 9.0)
    dout = normal_bf16(g, (M, N), 1.0)
    return gu, dout


@dataclass
class LayerInputs:
    x: torch.Tensor            # [T, H] bf16
    logits: torch.Tensor       # [T, E] bf16
    expt_indx: torch.Tensor    # [T, K] int32
    gu_blocks: torch.Tensor    # [E, 2I, H/32, 16] u8
    gu_scales: torch.Tensor    # [E, 2I, H/32] u8
    gu_bias: torch.Tensor      # [E, 2I] bf16
    dn_blocks: torch.Tensor    # [E, H, I/32, 16] u8
    dn_scales: torch.Tensor    # [E, H, I/32] u8
    dn_bias: torch.Tensor      # [E, H] bf16
    dy: torch.Tensor | None    # [T, H] bf16 upstream gradient
    lora: dict | None          # Agu [E,r,H], Bgu [E,2I,r], Adn [E,r,I], Bdn [E,H,r] bf16; r; alpha
    k: int

    def to(self, device):
        def mv(t):
            return t.to(device) if isinstance(t, torch.Tensor) else t
        lora = None if self.lora is None else {k: mv(v) for k, v in self.lora.items()}
        return LayerInputs(*(mv(getattr(self, f)) for f in
                             ("x", "logits", "expt_indx", "gu_blocks", "gu_scales", "gu_bias", "dn_blocks",
                              "dn_scales", "dn_bias", "dy")), lora, self.k)


def topk_stable(logits: torch.Tensor, k: int) -> torch.Tensor:
    """Top-k ids by a stable descending sort (ties -> lower id), ascending per token."""
    ids = torch.argsort(-logits.float(), dim=1, stable=True)[:, :k]
    return torch.sort(ids, dim=1).values.to(torch.int32)


def zipf_counts(total: int, n_active: int, s: float) -> np.ndarray:
    """Counts proportional to rank^-s, largest-remainder rounding to ``total``."""
    r = np.arange(1, n_active + 1, dtype=np.float64)
    w = r ** -s
    raw = w / w.sum() * total
    c = np.floor(raw).astype(np.int64)
    rem = total - int(c.sum())
    order = np.argsort(-(raw - c), kind="stable")
    c[order[:rem]] += 1
    return c


def zipf_routing(g: torch.Generator, T: int, E: int, k: int, s: float = 1.1, n_idle: int = 8) -> torch.Tensor:
    """[T, k] distinct expert ids per token with Zipf(s) expert loads and idle experts."""
    perm = torch.randperm(E, generator=g)            # perm[rank] = expert
    counts = zipf_counts(T * k, E - n_idle, s)       # by rank, descending
    if counts.max() > T:
        raise ValueError("an expert would need more than one slot per token")
    multiset = np.repeat(perm[: E - n_idle].numpy(), counts)
    ids = np.empty((T, k), dtype=np.int64)
    j = np.arange(T * k)
    ids[j % T, j // T] = multiset
    tperm = torch.randperm(T, generator=g).numpy()
    ids = ids[tperm]
    return torch.from_numpy(np.sort(ids, axis=1)).to(torch.int32)


def layer(cfg: int, T: int | None = None, E: int | None = None, k: int = 4, H: int = HIDDEN, I: int = INTER,
          lora_r: int | None = None, backward: bool | None = None, zipf: bool | None = None,
          scale_lo: int = 118, scale_hi: int = 130, n_idle: int = 8) -> LayerInputs:
    """Inputs of layer configuration ``cfg`` (2, 3, 4); sizes overridable for tests."""
    defaults = {2: (4096, 32, 0, False, False), 3: (16384, 32, 16, True, False), 4: (16384, 128, 32, True, True)}
    dT, dE, dr, dbwd, dz = defaults[cfg]
    T = dT if T is None else T
    E = dE if E is None else E
    lora_r = dr if lora_r is None else lora_r
    backward = dbwd if backward is None else backward
    zipf = dz if zipf is None else zipf
    g = gen(cfg)
    x = normal_bf16(g, (T, H), 1.0)
    logits = normal_bf16(g, (T, E), 1.0)
    if zipf:
        expt_indx = zipf_routing(g, T, E, k, n_idle=n_idle)
    else:
        expt_indx = topk_stable(logits, k)
    gu_blocks, gu_scales = mxfp4_weight(g, (E, 2 * I), H, scale_lo, scale_hi)
    dn_blocks, dn_scales = mxfp4_weight(g, (E, H), I, scale_lo, scale_hi)
    gu_bias = normal_bf16(g, (E, 2 * I), 0.02)
    dn_bias = normal_bf16(g, (E, H), 0.02)
    dy = normal_bf16(g, (T, H), 1.0) if backward else None
    lora = None
    if lora_r:
        lora = dict(Agu=normal_bf16(g, (E, lora_r, H), 0.01), Bgu=normal_bf16(g, (E, 2 * I, lora_r), 1e-3),
                    Adn=normal_bf16(g, (E, lora_r, I), 0.01), Bdn=normal_bf16(g, (E, H, lora_r), 1e-3),
                    r=lora_r, alpha=32.0)
    return LayerInputs(x, logits, expt_indx, gu_blocks, gu_scales, gu_bias, dn_blocks, dn_scales, dn_bias, dy,
                       lora, k)


def layer_flops(T: int, k: int, H: int = HIDDEN, I: int = INTER, backward: bool = True, lora_r: int = 0) -> dict:
    """Algorithmic flops of the expert GEMMs (no padding credited)."""
    R = T * k
    fwd = 2 * R * H * 2 * I + 2 * R * I * H
    base = fwd * (2 if backward else 1)
    lora = 0
    if lora_r:
        # per projection 2*R*r*(K+N) forward, twice that backward (dX, dA/dB)
        per = lambda K, N: 2 * R * lora_r * (K + N) * (3 if backward else 1)  # noqa: E731
        lora = per(H, 2 * I) + per(I, H)
    return dict(base=base, lora=lora, total=base + lora)


def make_experts(inp: LayerInputs, device, swiglu_limit: float = 7.0):
    """Mxfp4Bf16DequantGptOssExperts holding ``inp``'s weights on ``device``
    (weights stored the way the quantizer's loader stores them)."""
    from types import SimpleNamespace

    from torch import nn

    from .quantization import Mxfp4Bf16DequantGptOssExperts, _store_mxfp4_weights

    E, I2 = inp.gu_blocks.shape[:2]
    H = inp.dn_blocks.shape[1]
    cfg = SimpleNamespace(num_local_experts=E, intermediate_size=I2 // 2, hidden_size=H, swiglu_limit=swiglu_limit)
    with torch.device("meta"):
        m = Mxfp4Bf16DequantGptOssExperts(cfg)
    _store_mxfp4_weights(inp.gu_blocks, inp.gu_scales, m, "gate_up_proj", device)
    _store_mxfp4_weights(inp.dn_blocks, inp.dn_scales, m, "down_proj", device)
    m.gate_up_proj_bias = nn.Parameter(inp.gu_bias.to(device), requires_grad=False)
    m.down_proj_bias = nn.Parameter(inp.dn_bias.to(device), requires_grad=False)
    if inp.lora is not None:
        for name, key in (("gate_up_proj_lora_A", "Agu"), ("gate_up_proj_lora_B", "Bgu"),
                          ("down_proj_lora_A", "Adn"), ("down_proj_lora_B", "Bdn")):
            m.register_parameter(name, nn.Parameter(inp.lora[key].to(device).clone()))
        m.expert_lora_r = int(inp.lora["r"])
        m.expert_lora_scaling = float(inp.lora["alpha"]) / int(inp.lora["r"])
    return m
