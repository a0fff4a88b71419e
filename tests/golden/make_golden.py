"""Write the golden fixtures of this directory (run from the repo root).

The reference holds no tests or vectors for this path, so the fixtures come
from mathematics independent of the oracle's bit formulas:

* ``mxfp4_table.npy`` [256 scales, 16 codes] uint16: the bf16 bits of
  e2m1(code) * 2^(S-127) computed in float64 (MX definition), with the
  reference kernel's rule that a value whose bf16 exponent would fall outside
  [1, 254] becomes a zero of the code's sign (kernels.py:151-156).
* ``tiny_moe.npz``: a T=8, H=I=64, E=4, K=2 layer (MXFP4 weights with small
  scales) and its float64 dense-math forward output and input gradient.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]

E2M1 = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]


def mxfp4_table() -> np.ndarray:
    out = np.zeros((256, 16), dtype=np.uint16)
    for s in range(256):
        for code in range(16):
            neg = code >= 8
            mag = E2M1[code & 7]
            sign_bits = 0x8000 if neg else 0
            if mag == 0.0:
                out[s, code] = sign_bits
                continue
            v = np.ldexp(mag, s - 127)             # exact in float64
            m, e2 = np.frexp(v)                    # v = m * 2^e2, m in [0.5, 1)
            biased = e2 - 1 + 127                  # bf16/fp32 biased exponent
            if biased < 1 or biased > 254:
                out[s, code] = sign_bits           # flush to signed zero
                continue
            bits = np.array([v], dtype=np.float32).view(np.uint32)[0] >> 16
            out[s, code] = sign_bits | int(bits)
    return out


def tiny_moe() -> dict:
    g = torch.Generator().manual_seed(7)
    T, H, I, E, K = 8, 64, 64, 4, 2
    gu_blocks = torch.randint(0, 256, (E, 2 * I, H // 32, 16), generator=g).to(torch.uint8)
    gu_scales = torch.randint(122, 126, (E, 2 * I, H // 32), generator=g).to(torch.uint8)
    dn_blocks = torch.randint(0, 256, (E, H, I // 32, 16), generator=g).to(torch.uint8)
    dn_scales = torch.randint(122, 126, (E, H, I // 32), generator=g).to(torch.uint8)
    gu_bias = (torch.randn(E, 2 * I, generator=g) * 0.1).to(torch.bfloat16)
    dn_bias = (torch.randn(E, H, generator=g) * 0.1).to(torch.bfloat16)
    x = torch.randn(T, H, generator=g).to(torch.bfloat16)
    logits = torch.randn(T, E, generator=g).to(torch.bfloat16)
    dy = torch.randn(T, H, generator=g).to(torch.bfloat16)
    ids = torch.argsort(-logits.float(), dim=1, stable=True)[:, :K]
    ids = torch.sort(ids, dim=1).values
    scal = torch.softmax(torch.take_along_dim(logits, ids, 1), dim=-1)  # bf16 like the reference

    def deq(blocks, scales):  # float64 MX value of every element
        vals = torch.tensor(E2M1 + [-v for v in E2M1], dtype=torch.float64)
        lo = vals[(blocks & 0xF).long()]
        hi = vals[(blocks >> 4).long()]
        w = torch.stack([lo, hi], -1).reshape(*blocks.shape[:-1], 32)
        w = w * torch.pow(2.0, scales.to(torch.float64) - 127)[..., None]
        return w.reshape(*blocks.shape[:-2], -1)

    Wgu, Wdn = deq(gu_blocks, gu_scales), deq(dn_blocks, dn_scales)
    xe = x.to(torch.float64).requires_grad_(True)
    h = torch.einsum("th,tkoh->tko", xe, Wgu[ids]) + gu_bias.double()[ids]
    gate = torch.clamp(h[..., 0::2], max=7.0)
    up = torch.clamp(h[..., 1::2], -7.0, 7.0)
    act = gate * torch.sigmoid(1.702 * gate) * (up + 1.0)
    y = torch.einsum("tki,tkhi->tkh", act, Wdn[ids]) + dn_bias.double()[ids]
    Y = (y * scal.double()[..., None]).sum(1)
    Y.backward(dy.double())

    def u8(t):
        return t.numpy().astype(np.uint8)

    def bits(t):
        return t.view(torch.int16).numpy().view(np.uint16)

    return dict(gu_blocks=u8(gu_blocks), gu_scales=u8(gu_scales), dn_blocks=u8(dn_blocks),
                dn_scales=u8(dn_scales), gu_bias=bits(gu_bias), dn_bias=bits(dn_bias), x=bits(x),
                logits=bits(logits), dy=bits(dy), ids=ids.numpy().astype(np.int32),
                Y=Y.detach().numpy(), dX=xe.grad.numpy())


def main() -> None:
    np.save(HERE / "mxfp4_table.npy", mxfp4_table(), allow_pickle=False)
    np.savez(HERE / "tiny_moe.npz", **tiny_moe())
    print("wrote", HERE / "mxfp4_table.npy", HERE / "tiny_moe.npz", file=sys.stderr)


if __name__ == "__main__":
    main()
