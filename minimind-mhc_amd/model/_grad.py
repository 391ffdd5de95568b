"""Backward formulas of the mHC ops, evaluated with fp32 torch ops on the GPU.

Interim implementation until the HIP backward kernels exist.  The formulas
are the reference's analytic gradients:
  pre phase   model/mhc_fused.py:271-413 (kernel), :644-717 (grad_W GEMM and
              alpha/bias reductions); no-H_res: model/mhc_fused_no_hres.py:148-281
  post phase  model/mhc_fused.py:462-526, :747-772
  Sinkhorn    recompute + autograd, model/mhc_fused.py:131-137
  MHCHead     model/mhc_common.py:198-295, :359-400
Every product is formed in fp32 (no bf16 batched GEMM on transposed views).
"""
from __future__ import annotations

import torch


def pre_backward(x2, phi, a_pre, b_pre, a_post, b_post, a_res, inv_rms, mixes, n, C,
                 post_mult, pre_eps, g_sub, g_hpre, g_hpost, g_hres_raw):
    """Gradients of the pre phase.  mixes is the fp32 [M, FD] projection.

    Returns (g_x [M, nC] fp32, g_phi [nC, FD] fp32, g_a_pre, g_b_pre, g_a_post,
    g_b_post, g_a_res, g_b_res) with None for absent segments.
    """
    M = x2.shape[0]
    x = x2.float()
    xn = x * inv_rms[:, None]
    a_pre_f, b_pre_f = a_pre.float(), b_pre.float()
    a_post_f, b_post_f = a_post.float(), b_post.float()
    pre = mixes[:, :n]
    post = mixes[:, n:2 * n]
    sp = torch.sigmoid(pre * a_pre_f + b_pre_f)
    so = torch.sigmoid(post * a_post_f + b_post_f)
    h_pre = sp + pre_eps
    x3 = x.view(M, n, C)
    zeros_n = x.new_zeros(M, n)
    g_sub_f = g_sub.float().view(M, C) if g_sub is not None else x.new_zeros(M, C)
    g_hp = (g_hpre.float().view(M, n) if g_hpre is not None else zeros_n) + \
        torch.bmm(x3, g_sub_f.unsqueeze(-1)).squeeze(-1)
    g_pre_raw = g_hp * sp * (1.0 - sp)
    g_ho = g_hpost.float().view(M, n) if g_hpost is not None else zeros_n
    g_post_raw = g_ho * so * (1.0 - so) * post_mult
    segs = [g_pre_raw * a_pre_f, g_post_raw * a_post_f]
    g_res = None
    if a_res is not None:
        g_res = g_hres_raw.float().view(M, n * n) if g_hres_raw is not None else x.new_zeros(M, n * n)
        segs.append(g_res * a_res.float())
    g_mix = torch.cat(segs, dim=1)
    g_xn = g_mix @ phi.float().t().contiguous()
    mean = (xn * g_xn).sum(-1, keepdim=True) / (n * C)
    g_x = inv_rms[:, None] * (g_xn - xn * mean)
    g_x = g_x + (h_pre.unsqueeze(-1) * g_sub_f.unsqueeze(1)).reshape(M, n * C)
    g_phi = xn.t().contiguous() @ g_mix
    out = [g_x, g_phi,
           (g_pre_raw * pre).sum(), g_pre_raw.sum(0),
           (g_post_raw * post).sum(), g_post_raw.sum(0)]
    if a_res is not None:
        res = mixes[:, 2 * n:2 * n + n * n]
        out += [(g_res * res).sum(), g_res.sum(0).view(n, n)]
    else:
        out += [None, None]
    return out


def post_backward(x2, h_res, h_post, f_out, n, C, g_out):
    """Gradients of out = H_res . x + H_post (x) F (h_res None: identity)."""
    M = x2.shape[0]
    g = g_out.float().reshape(M, n, C)
    f = f_out.float().reshape(M, C)
    hp = h_post.float().reshape(M, n)
    if h_res is not None:
        hr = h_res.float().reshape(M, n, n)
        g_x = torch.bmm(hr.transpose(1, 2).contiguous(), g)
        g_hr = torch.bmm(g, x2.float().view(M, n, C).transpose(1, 2).contiguous())
    else:
        g_x, g_hr = g, None
    g_hp = torch.bmm(g, f.unsqueeze(-1)).squeeze(-1)
    g_f = torch.bmm(hp.unsqueeze(1), g).squeeze(1)
    return g_x.reshape(M, n * C), g_hr, g_hp, g_f


def sinkhorn_recompute(m: torch.Tensor, iters: int, eps: float) -> torch.Tensor:
    """Differentiable fp32 restatement of the Sinkhorn schedule (softmax row,
    column, then iters-1 row/column pairs), used only to form gradients."""
    x = m.float().softmax(dim=-1) + eps
    x = x / (x.sum(dim=-2, keepdim=True) + eps)
    for _ in range(iters - 1):
        x = x / (x.sum(dim=-1, keepdim=True) + eps)
        x = x / (x.sum(dim=-2, keepdim=True) + eps)
    return x


def sinkhorn_backward(m: torch.Tensor, iters: int, eps: float, g: torch.Tensor) -> torch.Tensor:
    with torch.enable_grad():
        leaf = m.detach().float().requires_grad_(True)
        y = sinkhorn_recompute(leaf, iters, eps)
        (gm,) = torch.autograd.grad(y, leaf, g.float())
    return gm


def head_backward(x2, phi, alpha, bias, inv_rms, mix_raw, n, C, pre_eps, g_out):
    """Gradients of MHCHead (n > 1)."""
    M = x2.shape[0]
    x = x2.float()
    xn = x * inv_rms[:, None]
    a = alpha.float().reshape(())
    s = torch.sigmoid(mix_raw * a + bias.float())
    g = g_out.float().reshape(M, C)
    g_mix = torch.bmm(x.view(M, n, C), g.unsqueeze(-1)).squeeze(-1)
    g_act = g_mix * s * (1.0 - s)
    g_raw = g_act * a
    g_xn = g_raw @ phi.float().t().contiguous()
    mean = (xn * g_xn).sum(-1, keepdim=True) / (n * C)
    g_x = inv_rms[:, None] * (g_xn - xn * mean)
    g_x = g_x + ((s + pre_eps).unsqueeze(-1) * g.unsqueeze(1)).reshape(M, n * C)
    g_phi = xn.t().contiguous() @ g_raw
    return g_x, g_phi, (g_act * mix_raw).sum().reshape(1), g_act.sum(0)


def rms_backward(x2, inv_rms, g_out):
    """Gradient of y = x * inv_rms(x) (MHCHead with n == 1)."""
    x = x2.float()
    xn = x * inv_rms[:, None]
    g = g_out.float().reshape_as(x)
    mean = (xn * g).sum(-1, keepdim=True) / x.shape[-1]
    return inv_rms[:, None] * (g - xn * mean)
