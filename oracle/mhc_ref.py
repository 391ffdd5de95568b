"""CPU restatement of the reference mHC forward path -- TEST INFRASTRUCTURE ONLY.

This is the parity oracle.  Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import it, and only as the checker (or, in
bench.py, as the timed CPU baseline).  The product package (minimind-mhc_amd/)
never imports it; its forward has no CPU path.

Each function restates one reference function op for op, with the same
rounding points, so that in bf16 it follows the reference's rounding
trajectory (torch ops on CPU tensors):
  sinkhorn           model/mhc_fused.py:47-56       (_sinkhorn_ref)
  pre_full           model/mhc_fused.py:533-559     (_pre_phase_full_ref)
  post_full          model/mhc_fused.py:562-568     (_post_phase_full_ref)
  mhc_full_forward   model/mhc_fused.py:836-864     (MHCConnection_Fused._forward_ref)
  pre_nohres         model/mhc_fused_no_hres.py:364-386
  post_nohres        model/mhc_fused_no_hres.py:389-394
  mhc_nohres_forward model/mhc_fused_no_hres.py:635-659
  head               model/mhc_common.py:298-308, n == 1 branch :438-442
  stream_expand      model/mhc_common.py:115-119

Parameters are passed as a dict of tensors named like the reference module's
parameters (phi_weight, alpha_pre, bias_pre, ...).  How each function is
pinned (golden vectors from the reference, closed forms, float64 brute force)
is listed in tests/test_oracle.py.
"""
from __future__ import annotations

from typing import Callable, Dict

import torch

Params = Dict[str, torch.Tensor]


def sinkhorn(M: torch.Tensor, iters: int, eps: float) -> torch.Tensor:
    """Softmax over rows (+eps), one column pass, then iters-1 (row, column)
    passes, each dividing by (sum + eps).  model/mhc_fused.py:47-56."""
    P = M.softmax(dim=-1) + eps
    P = P / (P.sum(dim=-2, keepdim=True) + eps)
    for _ in range(iters - 1):
        P = P / (P.sum(dim=-1, keepdim=True) + eps)
        P = P / (P.sum(dim=-2, keepdim=True) + eps)
    return P


def _inv_rms(x_flat: torch.Tensor, eps: float) -> torch.Tensor:
    # model/mhc_fused.py:843-844: fp32 mean of squares, + eps, rsqrt
    return x_flat.float().pow(2).mean(-1, keepdim=True).add(eps).rsqrt()


def _x_norm(x_flat: torch.Tensor, inv: torch.Tensor) -> torch.Tensor:
    # model/mhc_fused.py:845: normalised row rounded back to the stream dtype
    return (x_flat.float() * inv).to(x_flat.dtype)


def pre_full(x_flat: torch.Tensor, p: Params, n: int, C: int, *, post_mult: float = 2.0,
             pre_eps: float = 1e-6, rms_eps: float = 1e-6):
    """model/mhc_fused.py:533-559 -> (sublayer_in, h_pre, h_post, h_res_raw, inv_rms, mixes_raw)."""
    B, L, NC = x_flat.shape
    assert NC == n * C
    inv = _inv_rms(x_flat, rms_eps)
    mixes = _x_norm(x_flat, inv) @ p["phi_weight"]
    pre, post = mixes[..., :n], mixes[..., n:2 * n]
    res = mixes[..., 2 * n:2 * n + n * n].view(B, L, n, n)
    h_pre = torch.sigmoid(pre * p["alpha_pre"] + p["bias_pre"]) + pre_eps
    h_post = torch.sigmoid(post * p["alpha_post"] + p["bias_post"]) * post_mult
    h_res_raw = res * p["alpha_res"] + p["bias_res"]
    x = x_flat.view(B, L, n, C)
    sub_in = (h_pre.unsqueeze(-1) * x).sum(dim=-2)
    return sub_in, h_pre, h_post, h_res_raw, inv.squeeze(-1).float(), mixes.float()


def post_full(x_flat: torch.Tensor, h_res: torch.Tensor, h_post: torch.Tensor,
              f_out: torch.Tensor, n: int, C: int) -> torch.Tensor:
    """model/mhc_fused.py:562-568: einsum res-mix + H_post (x) F."""
    B, L, NC = x_flat.shape
    x = x_flat.view(B, L, n, C)
    mixed = torch.einsum("blij,bljc->blic", h_res, x)
    return (mixed + h_post.unsqueeze(-1) * f_out.unsqueeze(-2)).reshape(B, L, NC)


def mhc_full_forward(x_flat: torch.Tensor, p: Params, sublayer_fn: Callable, n: int, C: int, *,
                     eps: float = 1e-6, pre_eps: float = 1e-6, post_mult: float = 2.0,
                     sinkhorn_iters: int = 10, sinkhorn_eps: float = 1e-6):
    """MHCConnection_Fused._forward_ref, model/mhc_fused.py:836-864.

    Returns a dict with every intermediate (sub_in, h_pre, h_post, h_res_raw,
    h_res, f_out, out) so tests can compare each stage.
    """
    B, L, _ = x_flat.shape
    x = x_flat.view(B, L, n, C)
    inv = _inv_rms(x_flat, eps)
    mixes = _x_norm(x_flat, inv) @ p["phi_weight"]
    pre, post = mixes[..., :n], mixes[..., n:2 * n]
    res = mixes[..., 2 * n:2 * n + n * n].view(B, L, n, n)
    h_pre = torch.sigmoid(pre * p["alpha_pre"] + p["bias_pre"]) + pre_eps
    h_post = torch.sigmoid(post * p["alpha_post"] + p["bias_post"]) * post_mult
    h_res_raw = res * p["alpha_res"] + p["bias_res"]
    h_res = sinkhorn(h_res_raw.float(), sinkhorn_iters, sinkhorn_eps).to(x_flat.dtype)
    sub_in = (h_pre.unsqueeze(-1) * x).sum(dim=-2)
    f_out = sublayer_fn(sub_in)
    mixed = torch.einsum("blij,bljc->blic", h_res, x)
    out = (mixed + h_post.unsqueeze(-1) * f_out.unsqueeze(-2)).reshape(B, L, n * C)
    return dict(sub_in=sub_in, h_pre=h_pre, h_post=h_post, h_res_raw=h_res_raw, h_res=h_res,
                f_out=f_out, out=out, inv_rms=inv.squeeze(-1), mixes=mixes)


def pre_nohres(x_flat: torch.Tensor, p: Params, n: int, C: int, *, post_mult: float = 2.0,
               pre_eps: float = 1e-6, rms_eps: float = 1e-6):
    """model/mhc_fused_no_hres.py:364-386 -> (sublayer_in, h_pre, h_post, inv_rms, mixes_raw)."""
    B, L, NC = x_flat.shape
    assert NC == n * C
    inv = _inv_rms(x_flat, rms_eps)
    mixes = _x_norm(x_flat, inv) @ p["phi_weight"]
    h_pre = torch.sigmoid(mixes[..., :n] * p["alpha_pre"] + p["bias_pre"]) + pre_eps
    h_post = torch.sigmoid(mixes[..., n:2 * n] * p["alpha_post"] + p["bias_post"]) * post_mult
    sub_in = (h_pre.unsqueeze(-1) * x_flat.view(B, L, n, C)).sum(dim=-2)
    return sub_in, h_pre, h_post, inv.squeeze(-1).float(), mixes.float()


def post_nohres(x_flat: torch.Tensor, h_post: torch.Tensor, f_out: torch.Tensor, n: int,
                C: int) -> torch.Tensor:
    """model/mhc_fused_no_hres.py:389-394: x + H_post (x) F."""
    B, L, NC = x_flat.shape
    x = x_flat.view(B, L, n, C)
    return (x + h_post.unsqueeze(-1) * f_out.unsqueeze(-2)).reshape(B, L, NC)


def mhc_nohres_forward(x_flat: torch.Tensor, p: Params, sublayer_fn: Callable, n: int, C: int, *,
                       eps: float = 1e-6, pre_eps: float = 1e-6, post_mult: float = 2.0):
    """MHCConnection_FusedNoHres._forward_ref, model/mhc_fused_no_hres.py:635-659."""
    B, L, _ = x_flat.shape
    x = x_flat.view(B, L, n, C)
    inv = _inv_rms(x_flat, eps)
    mixes = _x_norm(x_flat, inv) @ p["phi_weight"]
    h_pre = torch.sigmoid(mixes[..., :n] * p["alpha_pre"] + p["bias_pre"]) + pre_eps
    h_post = torch.sigmoid(mixes[..., n:2 * n] * p["alpha_post"] + p["bias_post"]) * post_mult
    sub_in = (h_pre.unsqueeze(-1) * x).sum(dim=-2)
    f_out = sublayer_fn(sub_in)
    out = (x + h_post.unsqueeze(-1) * f_out.unsqueeze(-2)).reshape(B, L, n * C)
    return dict(sub_in=sub_in, h_pre=h_pre, h_post=h_post, f_out=f_out, out=out)


def head(x_flat: torch.Tensor, p: Params, n: int, C: int, *, pre_eps: float = 1e-6,
         rms_eps: float = 1e-6) -> torch.Tensor:
    """MHCHead forward: model/mhc_common.py:298-308, and :438-442 for n == 1."""
    B, L, NC = x_flat.shape
    inv = _inv_rms(x_flat, rms_eps)
    if n == 1:
        return (x_flat.float() * inv).to(x_flat.dtype).view(B, L, C)
    mix_raw = _x_norm(x_flat, inv) @ p["phi_weight"]
    mix = torch.sigmoid(mix_raw * p["alpha"] + p["bias"]) + pre_eps
    return (mix.unsqueeze(-1) * x_flat.view(B, L, n, C)).sum(dim=-2)


def stream_expand(x: torch.Tensor, n: int) -> torch.Tensor:
    """model/mhc_common.py:115-119: n identical copies along the last dim."""
    if n == 1:
        return x
    B, L, D = x.shape
    return x.unsqueeze(-2).expand(B, L, n, D).reshape(B, L, n * D)


def module_params(module: torch.nn.Module, device="cpu") -> Params:
    """Copy a module's parameters to CPU tensors keyed by parameter name."""
    return {k: v.detach().to(device) for k, v in module.named_parameters()}
