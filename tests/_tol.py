"""Element-wise tolerance checks shared by the GPU parity tests.

The bar is rtol 2e-2 / atol 1e-2 per element.  A GEMM output is a sum of n
products accumulated in fp32 on both sides (the MFMA's order on the GPU, the
CPU BLAS order in the oracle), so the two fp32 sums may differ by more than
atol where the terms are large and cancel.  Such outputs get an allowance
from the probabilistic rounding-error bound for an n-term fp32 sum
(Higham & Mary, "A new approach to probabilistic rounding error analysis",
SIAM J. Sci. Comput. 41(5), 2019): |fl(s) - s| <= lambda * sqrt(n) * u * sum|terms|,
u = 2^-24, taken with lambda = 1 for each of the two sums:

    |gpu - ref| <= atol + rtol * |ref| + 2 * sqrt(n) * 2^-24 * sum|terms|

``sum|terms|`` is computed by the oracle (the same products over absolute
values).  A single dropped, duplicated or sign-flipped term moves an output by
about sum|terms| / n, i.e. sqrt(n) / 2 times this allowance (27x at n = 2880),
so the allowance hides no such mistake.  tests/test_tolerance.py shows on the
CPU that the oracle's own fp32 sums stay inside it against exact float64 sums
at gpt-oss sizes while plain rtol / atol does not.
"""
from __future__ import annotations

import math

import torch

RTOL, ATOL = 2e-2, 1e-2
U32 = 2.0 ** -24


def accum_allowance(mag: torch.Tensor, n: int) -> torch.Tensor:
    """Allowance for two independently ordered fp32 sums of n terms with magnitude sum ``mag``."""
    return 2.0 * math.sqrt(max(n, 1)) * U32 * mag.to(torch.float64)


def combined_slack(rows, gate_indx, k):
    """Extra tolerance of a k-way sum of bf16 rows computed on both sides: each
    row may differ by one bf16 rounding (2^-8 of its value) on each side, so
    2^-7 times the sum of the rows' magnitudes."""
    gi = gate_indx.view(-1, k).long()
    ra = rows.detach().to("cpu", torch.float64).abs()
    out = torch.zeros(gi.shape[0], ra.shape[1], dtype=torch.float64)
    for j in range(k):
        ok = gi[:, j] >= 0
        out[ok] += ra[gi[ok, j]]
    return 2.0 ** -7 * out


def _lowp(t) -> bool:
    return t.dtype in (torch.bfloat16, torch.float16)


def check_close(got, ref, *, rtol=RTOL, atol=ATOL, mag=None, n=None, extra=None, what=""):
    """Assert |got - ref| <= atol + rtol*|ref| (+ the accumulation allowance for
    n-term sums of magnitude ``mag``) (+ ``extra``, a derived per-element or
    scalar slack) for every element.  Returns the largest error / tolerance.

    When both sides are 16-bit floats the comparison runs in float32, chunk by
    chunk: the difference of two bf16 values is exact in float32 unless their
    exponents are more than 16 apart (then it is within 2^-24 of the larger),
    and the tolerance only needs a few significant bits."""
    g0, r0 = got.detach().cpu(), ref.detach().cpu()
    assert g0.shape == r0.shape, f"{what}: shape {tuple(g0.shape)} != {tuple(r0.shape)}"
    wd = torch.float32 if _lowp(g0) and _lowp(r0) else torch.float64
    if g0.dim() == 0 or g0.numel() == 0:
        g0, r0 = g0.reshape(-1), r0.reshape(-1)
    ex = extra.detach().cpu() if isinstance(extra, torch.Tensor) else extra
    mg = mag.detach().cpu() if mag is not None else None
    c = 2.0 * math.sqrt(max(n or 1, 1)) * U32
    rows = g0.shape[0]
    per_row = max(1, g0[0].numel()) if rows else 1
    step = max(1, (1 << 24) // per_row)
    worst, n_bad, first = 0.0, 0, []

    def part(t, lo, hi):
        if not isinstance(t, torch.Tensor):
            return t
        if t.dim() == g0.dim() and t.shape[0] == rows and rows > 1:
            return t[lo:hi]
        return t

    for lo in range(0, rows, step):
        hi = min(rows, lo + step)
        g = g0[lo:hi].to(wd)
        r = r0[lo:hi].to(wd)
        assert torch.isfinite(g).all(), f"{what}: non-finite values"
        err = (g - r).abs_()
        tol = r.abs().mul_(rtol).add_(atol)
        if mg is not None:
            tol.add_(part(mg, lo, hi).to(wd), alpha=c)
        if ex is not None:
            e = part(ex, lo, hi)
            tol.add_(e.to(wd) if isinstance(e, torch.Tensor) else float(e))
        bad = err > tol
        if bool(bad.any()):
            n_bad += int(bad.sum())
            for i in bad.nonzero()[:5 - len(first)].tolist():
                i = tuple(i)
                first.append(((lo + i[0],) + i[1:], float(g[i]), float(r[i]), float(tol[i])))
        if err.numel():
            worst = max(worst, float((err / tol).max()))
    if n_bad:
        raise AssertionError(f"{what}: {n_bad} of {g0.numel()} elements outside tolerance; "
                             f"(index, got, ref, tol) {first}")
    return worst


def check_equal(got, ref, what=""):
    """Bit-exact equality (integer / byte work, and fp sums taken in the same order)."""
    g, r = got.detach().cpu(), ref.detach().cpu()
    assert g.shape == r.shape and g.dtype == r.dtype, f"{what}: {g.shape}/{g.dtype} vs {r.shape}/{r.dtype}"
    if g.is_floating_point():
        g, r = g.view(torch.int16 if g.element_size() == 2 else torch.int32), \
            r.view(torch.int16 if r.element_size() == 2 else torch.int32)
    diff = g != r
    assert not bool(diff.any()), f"{what}: {int(diff.sum())} of {diff.numel()} elements differ, " \
                                 f"first at {diff.nonzero()[:3].tolist()}"
