"""MoE expert layer restated as per-expert fp32 loops on the CPU (test infrastructure only).

``rows`` is matmul_ogs without its scatter as the reference calls it
(quantization.py:358-362 forward with ``w.transpose(-1, -2)``, 409-418
backward with ``w``): for each expert e, over its expert-sorted rows,
``Y = X[gather] @ W[e]^T (+ bias[e]) (* gammas)`` in fp32, one bf16 rounding.
``combine`` is the scatter-sum over each token's K rows.  ``layer_forward`` /
``layer_backward`` compose them as Mxfp4Bf16DequantGptOssExperts.forward
(quantization.py:507-544) and the backward of its autograd functions
(quantization.py:376-421, 442-444), with the expert-LoRA terms of the build
(scaling s = lora_alpha / r, PEFT convention model_trainer.py:665,711).
``lora_merge`` folds the expert adapters into bf16 weights the way the
reference merges its attention adapters for weight sync (model_trainer.py:710-712).
"""
from __future__ import annotations

import torch

from . import swiglu as _sw

BF16 = torch.bfloat16
F32 = torch.float32


def _rnd(t, rd):
    return t.to(rd) if rd == torch.float64 else t.to(F32).to(rd)


def rows(x, W, offs, gather=None, k=1, bias=None, gammas=None, trans=False, lora_l=None, lora_b=None, rd=BF16):
    """Expert-sorted bf16 rows.

    x [Tx, Kx] (bf16); W float32 [E, N, K] (trans False: y = x W[e]^T, out N)
    or the same W with trans True (y = x W[e], out K); lora_l [R, r],
    lora_b [E, N, r] (trans False) / [E, r, K] (trans True).
    """
    E = W.shape[0]
    n_out = W.shape[2] if trans else W.shape[1]
    R = gather.numel() if gather is not None else x.shape[0]
    acc = torch.float64 if rd == torch.float64 else F32
    y = torch.zeros(R, n_out, dtype=acc)
    xf = x.to(acc)
    for e in range(E):
        lo, hi = int(offs[e]), int(offs[e + 1])
        if hi <= lo:
            continue
        idx = (gather[lo:hi].long() // k) if gather is not None else torch.arange(lo, hi)
        y[lo:hi] = _expert_acc(xf[idx], W[e], trans, None if lora_l is None else lora_l[lo:hi],
                               None if lora_b is None else lora_b[e], None if bias is None else bias[e],
                               None if gammas is None else gammas[lo:hi], acc)
    return y.to(rd)


def _expert_acc(xe, We, trans, Le, Be, be, ge, acc, mag=False):
    """One expert's rows in ``acc``: xe @ We^T (trans: xe @ We) [+ Le @ Be^T (Le @ Be)]
    [+ be] [* ge].  ``mag``: the same products over absolute values instead
    (the sum of |term| per output, scaled by |ge|; bias not included)."""
    f = (lambda t: t.to(acc).abs()) if mag else (lambda t: t.to(acc))  # noqa: E731
    W = f(We)
    out = f(xe) @ (W if trans else W.T)
    if Le is not None:
        B = f(Be)
        out = out + f(Le) @ (B if trans else B.T)
    if be is not None and not mag:
        out = out + be.to(acc)
    if ge is not None:
        out = out * f(ge)[:, None]
    return out


def expert_rows(x, We, idx, trans=False, lora_l=None, lora_b=None, bias=None, gammas=None):
    """Rows of one expert as ``rows`` computes them (fp32 sums, one bf16
    rounding) and, for tolerances, the fp32 sum of the magnitudes of their
    terms: (bf16 [n, N], float32 [n, N]).  ``idx``: the source rows of x;
    ``We`` [N, K] float32; lora_l / gammas: the expert's rows; lora_b, bias:
    the expert's slices."""
    xe = x[idx]
    out = _expert_acc(xe, We, trans, lora_l, lora_b, bias, gammas, F32)
    mag = _expert_acc(xe, We, trans, lora_l, lora_b, None, gammas, F32, mag=True)
    return out.to(BF16), mag


def expert_lora_rows(x, Wl, idx, scale, trans=False):
    """One expert of ``lora_rows``: s * x[idx] @ Wl^T (trans: @ Wl) and its term magnitudes."""
    xe = x[idx].to(F32)
    W = Wl.to(F32)
    out = scale * (xe @ (W if trans else W.T))
    mag = abs(scale) * (xe.abs() @ (W.abs() if trans else W.abs().T))
    return out.to(BF16), mag


def expert_wgrad(a_e, b_e, rowscale=None):
    """One expert of ``wgrad``: bf16(rs * a_e)^T @ b_e (fp32 sum, one bf16
    rounding) and the magnitudes of its terms.  a_e, b_e: the expert's rows
    (already gathered), rowscale its row scales."""
    ae = a_e.to(F32)
    if rowscale is not None:
        ae = (ae * rowscale.to(F32)[:, None]).to(BF16).to(F32)
    bf = b_e.to(F32)
    return (ae.T @ bf).to(BF16), ae.abs().T @ bf.abs()


def combine(r, gate_indx, k, rd=BF16):
    """out[t] = bf16(sum_j r[gate_indx[t*k+j]]) in fp32; -1 skipped."""
    T = gate_indx.numel() // k
    acc = torch.float64 if rd == torch.float64 else F32
    out = torch.zeros(T, r.shape[1], dtype=acc)
    gi = gate_indx.view(T, k).long()
    rf = r.to(acc)
    for j in range(k):
        col = gi[:, j]
        ok = col >= 0
        out[ok] += rf[col[ok]]
    return out.to(rd)


def lora_rows(x, A_or_B, offs, gather=None, k=1, scale=1.0, trans=False, rd=BF16):
    """Skinny per-expert product: trans False: s * X[a(r)] A[e]^T (A [E, r, K]);
    trans True: s * X[a(r)] B[e] (B [E, K, r])."""
    acc = torch.float64 if rd == torch.float64 else F32
    Wf = A_or_B.to(acc)
    E = Wf.shape[0]
    n_out = Wf.shape[2] if trans else Wf.shape[1]
    R = gather.numel() if gather is not None else x.shape[0]
    y = torch.zeros(R, n_out, dtype=acc)
    xf = x.to(acc)
    for e in range(E):
        lo, hi = int(offs[e]), int(offs[e + 1])
        if hi <= lo:
            continue
        idx = (gather[lo:hi].long() // k) if gather is not None else torch.arange(lo, hi)
        y[lo:hi] = scale * (xf[idx] @ (Wf[e] if trans else Wf[e].T))
    return y.to(rd)


def wgrad(a, b, offs, a_gather=None, a_div=1, a_rowscale=None, b_gather=None, b_div=1, rd=BF16):
    """G[e] = sum_{r in e} bf16(rs[r] * a[a(r)])^T b[b(r)]  -> bf16 [E, Ma, Nb]."""
    E = offs.numel() - 1
    acc = torch.float64 if rd == torch.float64 else F32
    af, bf = a.to(acc), b.to(acc)
    G = torch.zeros(E, a.shape[1], b.shape[1], dtype=acc)
    for e in range(E):
        lo, hi = int(offs[e]), int(offs[e + 1])
        if hi <= lo:
            continue
        ia = (a_gather[lo:hi].long() // a_div) if a_gather is not None else torch.arange(lo, hi)
        ib = (b_gather[lo:hi].long() // b_div) if b_gather is not None else torch.arange(lo, hi)
        ae = af[ia]
        if a_rowscale is not None:
            # the row-scaled operand is a bf16 tensor (the product rounds it
            # before the matrix core, as autograd of a bf16 multiply does)
            ae = _rnd(ae * a_rowscale[lo:hi, None].to(acc), rd).to(acc)
        G[e] = ae.T @ bf[ib]
    return G.to(rd)


def layer_forward(x, p, rt, k, alpha=_sw.ALPHA, limit=_sw.LIMIT, lora=None, rd=BF16):
    """Expert layer forward.  p: dict(Wgu [E,2I,H] f32, bgu [E,2I], Wdn [E,H,I] f32, bdn [E,H]);
    rt: routing dict (oracle.routing); lora: None or dict(Agu, Bgu, Adn, Bdn, s).
    ``rd`` is the dtype intermediates are rounded to (bf16 as on the GPU;
    float64 gives the exact math used to pin the formulas).
    Returns dict of intermediates and Y [T, H]."""
    offs, ti, gi, gs = rt["offs"], rt["topk_indx"], rt["gate_indx"], rt["gate_scal"]
    st = {}
    if lora is not None:
        st["Lgu"] = lora_rows(x, lora["Agu"], offs, ti, k, lora["s"], rd=rd)
        GU = rows(x, p["Wgu"], offs, ti, k, bias=p["bgu"], lora_l=st["Lgu"], lora_b=lora["Bgu"], rd=rd)
    else:
        GU = rows(x, p["Wgu"], offs, ti, k, bias=p["bgu"], rd=rd)
    act = _rnd(_sw.forward(GU, alpha, limit)[0], rd)
    if lora is not None:
        st["Ldn"] = lora_rows(act, lora["Adn"], offs, None, 1, lora["s"], rd=rd)
        Yr = rows(act, p["Wdn"], offs, None, 1, bias=p["bdn"], gammas=gs, lora_l=st["Ldn"], lora_b=lora["Bdn"],
                  rd=rd)
    else:
        Yr = rows(act, p["Wdn"], offs, None, 1, bias=p["bdn"], gammas=gs, rd=rd)
    Y = combine(Yr, gi, k, rd=rd)
    st.update(GU=GU, act=act, Yr=Yr, Y=Y)
    return st


def layer_backward(x, p, rt, k, st, dY, alpha=_sw.ALPHA, limit=_sw.LIMIT, lora=None, rd=BF16):
    """Backward of layer_forward given dY [T, H] bf16 -> dict(dX, dAct, dGU, [dA*, dB*])."""
    offs, ti, gi, gs = rt["offs"], rt["topk_indx"], rt["gate_indx"], rt["gate_scal"]
    g = {}
    if lora is not None:
        s = lora["s"]
        # down projection (forward scatter + gammas -> backward gather + gammas)
        u_dn = lora_rows(dY, lora["Bdn"], offs, ti, k, s, trans=True, rd=rd)
        dAct = rows(dY, p["Wdn"], offs, ti, k, gammas=gs, trans=True, lora_l=u_dn, lora_b=lora["Adn"], rd=rd)
        g["dAdn"] = wgrad(u_dn, st["act"], offs, a_rowscale=gs, rd=rd)
        g["dBdn"] = wgrad(dY, st["Ldn"], offs, a_gather=ti, a_div=k, a_rowscale=gs, rd=rd)
    else:
        dAct = rows(dY, p["Wdn"], offs, ti, k, gammas=gs, trans=True, rd=rd)
    dGU = _rnd(_sw.backward_from_raw(dAct, st["GU"], alpha, limit), rd)
    if lora is not None:
        u_gu = lora_rows(dGU, lora["Bgu"], offs, None, 1, s, trans=True, rd=rd)
        dXr = rows(dGU, p["Wgu"], offs, None, 1, trans=True, lora_l=u_gu, lora_b=lora["Agu"], rd=rd)
        g["dAgu"] = wgrad(u_gu, x, offs, b_gather=ti, b_div=k, rd=rd)
        g["dBgu"] = wgrad(dGU, st["Lgu"], offs, rd=rd)
    else:
        dXr = rows(dGU, p["Wgu"], offs, None, 1, trans=True, rd=rd)
    g.update(dAct=dAct, dGU=dGU, dXr=dXr, dX=combine(dXr, gi, k, rd=rd))
    return g


def dense_reference(x, p, expt_ids, scal, alpha=_sw.ALPHA, limit=_sw.LIMIT, lora=None, dtype=torch.float64):
    """The layer as plain math in float64 (no sorting, no rounding): for every
    token t and slot j, y_tj = gamma_tj * (act(x_t W_gu[e]^T + b) W_dn[e]^T + b_dn),
    Y_t = sum_j y_tj.  Differentiable w.r.t. x and the LoRA tensors."""
    T, K = expt_ids.shape
    Wgu, Wdn = p["Wgu"].to(dtype), p["Wdn"].to(dtype)
    ids = expt_ids.long()
    xe = x.to(dtype)
    Wg = Wgu[ids]                     # [T, K, 2I, H]
    h = torch.einsum("th,tkoh->tko", xe, Wg) + p["bgu"].to(dtype)[ids]
    if lora is not None:
        s = lora["s"]
        A, B = lora["Agu"].to(dtype)[ids], lora["Bgu"].to(dtype)[ids]
        h = h + s * torch.einsum("tkor,tkr->tko", B, torch.einsum("tkrh,th->tkr", A, xe))
    gate, up = h[..., 0::2], h[..., 1::2]
    gate = torch.clamp(gate, max=limit)
    up = torch.clamp(up, -limit, limit)
    act = gate * torch.sigmoid(alpha * gate) * (up + 1.0)
    Wd = Wdn[ids]                     # [T, K, H, I]
    y = torch.einsum("tki,tkhi->tkh", act, Wd) + p["bdn"].to(dtype)[ids]
    if lora is not None:
        A, B = lora["Adn"].to(dtype)[ids], lora["Bdn"].to(dtype)[ids]
        y = y + s * torch.einsum("tkhr,tkr->tkh", B, torch.einsum("tkri,tki->tkr", A, act))
    return (y * scal.to(dtype)[..., None]).sum(1)


def lora_merge(blocks, scales, A, B, s, layout="hf"):
    """Expert weight with the LoRA delta folded in, as the reference merges
    adapters for weight sync (model_trainer.py:710-712):
    ``(base.float() + (B.float() @ A.float()) * s).to(bf16)`` per expert, with
    base = the MXFP4 -> bf16 dequant (oracle.mxfp4) and the r-term sum taken
    exactly (float64) and rounded once to float32.  blocks [E, N, G, 16],
    A [E, r, K], B [E, N, r] -> bf16 [E, K, N] ("hf") or [E, N, K] ("rows")."""
    from . import mxfp4 as _mx
    base = _mx.dequant_f32(blocks, scales)                                   # [E, N, K] f32
    delta = torch.matmul(B.to(torch.float64), A.to(torch.float64)).to(F32)   # exact sum, one rounding
    w = (base + delta * torch.tensor(s, dtype=F32)).to(BF16)
    return w.transpose(1, 2).contiguous() if layout == "hf" else w
