"""mHC with H_res frozen to I_n (use_mhc = 2) on MI355X HIP kernels.

Drop-in for the reference module model/mhc_fused_no_hres.py
(MHCConnection_FusedNoHres, model/mhc_fused_no_hres.py:584-659): the same
pre-phase kernel with FD = 2n and no Sinkhorn, and the post kernel with
H_res = I, out = x + H_post (x) F.  No CPU or PyTorch forward path.
"""
from __future__ import annotations

import math
from typing import Callable

import torch
import torch.nn as nn

from . import _ops
from . import _hip as H
from .mhc_common import fusable_norm, norm_eps


def _is_pow2(n: int) -> bool:
    return n >= 1 and (n & (n - 1)) == 0


class _PrePhaseFn(_ops.GradAwareFunction):
    """Pre phase -> (sublayer_in, h_pre, h_post) (model/mhc_fused_no_hres.py:397-529)."""

    @staticmethod
    def forward(ctx, x_flat, w_phi, alpha_pre, bias_pre, alpha_post, bias_post,
                post_mult, pre_eps, rms_eps, n, c, packed=None, ssq=None):
        B, L, NC = x_flat.shape
        train = _ops.grad_wanted(ctx)
        if packed is None:  # called as the reference's Function, without the module's pack
            packed = _ops.packed_phi(w_phi, n, c, H.MODE_NOHRES, training=_ops.grad_wanted(ctx, 1))
        o = _ops.pre_nohres(x_flat, w_phi, packed, alpha_pre, bias_pre, alpha_post, bias_post,
                            n, c, post_mult, pre_eps, rms_eps, want_h_pre=True, want_saved=train,
                            ssq=ssq)
        if train:
            ctx.save_for_backward(x_flat.detach().contiguous().view(B * L, NC), w_phi,
                                  alpha_pre, bias_pre, alpha_post, bias_post,
                                  o["inv_rms"], o["mixes_raw"])
        ctx.cfg = (n, c, float(post_mult), float(pre_eps), (B, L, NC))
        return (o["sub_in"].view(B, L, c), o["h_pre"].view(B, L, n), o["h_post"].view(B, L, n))

    @staticmethod
    def backward(ctx, g_sub, g_hpre, g_hpost):
        x2, w, a_pre, b_pre, a_post, b_post, inv, mixes = ctx.saved_tensors
        n, c, post_mult, pre_eps, shape = ctx.cfg
        alphas, biases = (a_pre, a_post, None), (b_pre, b_post, None)
        g_x, g_raw = _ops.pre_bwd(x2, w, alphas, biases, inv, mixes, n, c, H.MODE_NOHRES,
                                  post_mult, pre_eps, g_sub, g_hpre, g_hpost)
        g_w, g_a, g_b = _ops.pre_bwd_weights(x2, inv, mixes, g_raw, w, alphas, n, c,
                                             H.MODE_NOHRES)
        return (g_x.view(shape), g_w,
                g_a[0].to(a_pre.dtype).reshape(a_pre.shape), g_b[0].to(b_pre.dtype).view(b_pre.shape),
                g_a[1].to(a_post.dtype).reshape(a_post.shape), g_b[1].to(b_post.dtype).view(b_post.shape),
                None, None, None, None, None, None, None)


class _PostPhaseFn(_ops.GradAwareFunction):
    """out = x + H_post (x) F_out (model/mhc_fused_no_hres.py:532-581)."""

    @staticmethod
    def forward(ctx, x_flat, h_post, f_out, n, c, ssq_out=None):
        B, L, NC = x_flat.shape
        out = _ops.post(x_flat, None, h_post, f_out, n, c, ssq_out=ssq_out)
        if _ops.grad_wanted(ctx):
            ctx.save_for_backward(h_post, f_out)
        ctx.cfg = (n, c, (B, L, NC))
        return out.view(B, L, NC)

    @staticmethod
    def backward(ctx, g_out):
        h_post, f_out = ctx.saved_tensors
        n, c, shape = ctx.cfg
        g_x, _, g_hp, g_f = _ops.post_bwd(None, None, h_post, f_out, n, c, g_out)
        return (g_x.view(shape), g_hp.view(h_post.shape), g_f.view(f_out.shape), None, None, None)


class MHCConnection_FusedNoHres(nn.Module):
    """mHC sublayer wrapper with H_res = I_n: x' = x + H_post (x) F(H_pre . x).

    Same constructor and parameters as the reference
    (model/mhc_fused_no_hres.py:584-659); phi_weight is (n*dim, 2n) row-major.
    """

    def __init__(self, n: int, dim: int, alpha_init: float = 0.01,
                 post_mult_value: float = 2.0, eps: float = 1e-6,
                 pre_eps: float = 1e-6):
        super().__init__()
        assert n >= 1 and isinstance(n, int)
        assert _is_pow2(n) and n <= 16, f"n must be in {{1,2,4,8,16}}, got {n}"
        assert post_mult_value > 1.0
        self.n = n
        self.dim = dim
        self.nC = n * dim
        self.fused_dim = 2 * n
        self.post_mult_value = post_mult_value
        self.pre_eps = pre_eps
        self.eps = eps

        self.phi_weight = nn.Parameter(torch.empty(self.nC, self.fused_dim))
        nn.init.kaiming_uniform_(self.phi_weight, a=math.sqrt(5))
        self.alpha_pre = nn.Parameter(torch.tensor(alpha_init))
        self.bias_pre = nn.Parameter(torch.zeros(n))
        self.alpha_post = nn.Parameter(torch.tensor(alpha_init))
        self.bias_post = nn.Parameter(torch.zeros(n))
        self._phi_pack = _ops.PhiPack(H.MODE_NOHRES)

    def extra_repr(self) -> str:
        return (f"n={self.n}, dim={self.dim}, fused_dim={self.fused_dim}, "
                f"post_mult_value={self.post_mult_value}, backend=hip-gfx950")

    def forward(self, x_flat: torch.Tensor, sublayer_fn: Callable,
                in_norm: nn.Module = None, chain: _ops.StreamChain = None) -> torch.Tensor:
        """in_norm, chain: as MHCConnection_Fused.forward (F(z) =
        sublayer_fn(in_norm(z)), fused into the pre launch when no autograd is
        needed; the rows' sums of squares handed along the chain)."""
        packed = self._phi_pack.get(self.phi_weight, self.n, self.dim) if x_flat.is_cuda else None
        ssq = chain.take(x_flat, self.n, self.dim) if chain is not None else None
        ssq_out = chain.buffer(x_flat, self.n, self.dim) if chain is not None else None
        if in_norm is not None:
            if fusable_norm(in_norm, self.dim, x_flat):
                o = _ops.pre_nohres(x_flat, self.phi_weight, packed, self.alpha_pre, self.bias_pre,
                                    self.alpha_post, self.bias_post, self.n, self.dim,
                                    self.post_mult_value, self.pre_eps, self.eps,
                                    norm=(in_norm.weight, norm_eps(in_norm, x_flat)), ssq=ssq)
                B, L, NC = x_flat.shape
                f_out = sublayer_fn(o["sub_in"].view(B, L, self.dim))
                out = _ops.post(x_flat, None, o["h_post"], f_out, self.n, self.dim,
                                ssq_out=ssq_out).view(B, L, NC)
                return chain.put(out, ssq_out) if chain is not None else out
            fn = sublayer_fn
            sublayer_fn = lambda z: fn(in_norm(z))  # noqa: E731
        sublayer_in, _h_pre, h_post = _PrePhaseFn.apply(
            x_flat, self.phi_weight, self.alpha_pre, self.bias_pre,
            self.alpha_post, self.bias_post,
            self.post_mult_value, self.pre_eps, self.eps, self.n, self.dim, packed, ssq)
        f_out = sublayer_fn(sublayer_in)
        out = _PostPhaseFn.apply(x_flat, h_post, f_out, self.n, self.dim, ssq_out)
        return chain.put(out, ssq_out) if chain is not None else out
