"""mHC with dynamic H_pre / H_post / H_res (use_mhc = 1) on MI355X HIP kernels.

Drop-in for the reference module model/mhc_fused.py: same class and function
names, constructor signatures, parameter names/shapes and forward contract
(model/mhc_fused.py:775-834, :140-154).  The forward runs two hand-written
gfx950 kernels through the C ABI of libmhc_amd.so:

  pre  : RMSNorm(n*C) + projection + gates + Sinkhorn-Knopp + pre-aggregate
  post : out = H_res . x + H_post (x) F(sublayer_in)

There is no CPU or PyTorch forward path: tensors must be on a ROCm device and
the library must be built.  The backward pass runs the library's backward
kernels (mhc_post_bwd, mhc_sinkhorn_bwd, mhc_pre_bwd, mhc_pre_bwd_weights).
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


# ---------------------------------------------------------------- Sinkhorn op

class _SinkhornFn(_ops.GradAwareFunction):
    """Sinkhorn-Knopp forward on the HIP kernel; backward by recompute
    (model/mhc_fused.py:96-137)."""

    @staticmethod
    def forward(ctx, M: torch.Tensor, iters: int, eps: float) -> torch.Tensor:
        if _ops.grad_wanted(ctx, 0):
            _ops.check_sinkhorn_bwd_iters(M.shape[-1], iters)
        out = _ops.sinkhorn(M, iters, eps)
        ctx.save_for_backward(M)
        ctx.iters, ctx.eps = iters, eps
        return out

    @staticmethod
    def backward(ctx, dy):
        (M,) = ctx.saved_tensors
        return _ops.sinkhorn_bwd(M, dy, ctx.iters, ctx.eps), None, None


@torch.amp.autocast("cuda", enabled=False)
def sinkhorn_normalize(M: torch.Tensor, iters: int = 10, eps: float = 1e-6) -> torch.Tensor:
    """(..., n, n) raw -> Birkhoff polytope (model/mhc_fused.py:140-154).

    Softmax over each row + eps, one column normalisation, then iters - 1
    (row, column) normalisations, each dividing by (sum + eps).  Computed in
    fp32, returned in M's dtype.  Requires a ROCm tensor.
    """
    return _SinkhornFn.apply(M, iters, eps)


# --------------------------------------------------------- pre / post phases

def _pre_full_grads(x2, w, alphas, biases, inv, mixes, n, c, post_mult, pre_eps, shape,
                    g_sub, g_hpre, g_hpost, g_hres_raw):
    """(g_x, g_phi, g_alpha_pre, g_bias_pre, g_alpha_post, g_bias_post, g_alpha_res,
    g_bias_res) of the full pre phase, each in its forward input's dtype and shape."""
    g_x, g_raw = _ops.pre_bwd(x2, w, alphas, biases, inv, mixes, n, c, H.MODE_FULL, post_mult,
                              pre_eps, g_sub, g_hpre, g_hpost, g_hres_raw)
    g_w, g_a, g_b = _ops.pre_bwd_weights(x2, inv, mixes, g_raw, w, alphas, n, c, H.MODE_FULL)
    out = [g_x.view(shape), g_w]
    for a, b, ga, gb in zip(alphas, biases, g_a, g_b):
        out += [ga.to(a.dtype).reshape(a.shape), gb.to(b.dtype).view(b.shape)]
    return out


class _PrePhaseFullFn(_ops.GradAwareFunction):
    """Pre phase -> (sublayer_in, h_pre, h_post, h_res_raw), h_res_raw before
    Sinkhorn, as the reference Function (model/mhc_fused.py:571-717)."""

    @staticmethod
    def forward(ctx, x_flat, w_phi, alpha_pre, bias_pre, alpha_post, bias_post,
                alpha_res, bias_res, post_mult, pre_eps, rms_eps, n, c):
        B, L, NC = x_flat.shape
        train = _ops.grad_wanted(ctx)
        packed = _ops.packed_phi(w_phi, n, c, H.MODE_FULL, training=_ops.grad_wanted(ctx, 1))
        o = _ops.pre_full(x_flat, w_phi, packed, alpha_pre, bias_pre, alpha_post, bias_post,
                          alpha_res, bias_res, n, c, post_mult, pre_eps, rms_eps, 0, 0.0,
                          sinkhorn=False, want_h_pre=True, want_raw=True, want_saved=train)
        if train:
            ctx.save_for_backward(x_flat.detach().contiguous().view(B * L, NC), w_phi, alpha_pre,
                                  bias_pre, alpha_post, bias_post, alpha_res, bias_res,
                                  o["inv_rms"], o["mixes_raw"])
        ctx.cfg = (n, c, float(post_mult), float(pre_eps), (B, L, NC))
        return (o["sub_in"].view(B, L, c), o["h_pre"].view(B, L, n),
                o["h_post"].view(B, L, n), o["h_res_raw"].view(B, L, n, n))

    @staticmethod
    def backward(ctx, g_sub, g_hpre, g_hpost, g_hres_raw):
        x2, w, a_pre, b_pre, a_post, b_post, a_res, b_res, inv, mixes = ctx.saved_tensors
        n, c, post_mult, pre_eps, shape = ctx.cfg
        return (*_pre_full_grads(x2, w, (a_pre, a_post, a_res), (b_pre, b_post, b_res), inv,
                                 mixes, n, c, post_mult, pre_eps, shape,
                                 g_sub, g_hpre, g_hpost, g_hres_raw),
                None, None, None, None, None)


class _PreSinkhornFn(_ops.GradAwareFunction):
    """Fused pre phase + Sinkhorn -> (sublayer_in, h_post, h_res): the single
    launch MHCConnection_Fused.forward uses in place of the reference's
    _PrePhaseFullFn + sinkhorn_normalize pair (model/mhc_fused.py:820-830)."""

    @staticmethod
    def forward(ctx, x_flat, w_phi, packed, alpha_pre, bias_pre, alpha_post, bias_post,
                alpha_res, bias_res, post_mult, pre_eps, rms_eps, n, c, iters, sk_eps, ssq=None):
        B, L, NC = x_flat.shape
        train = _ops.grad_wanted(ctx)
        if train:
            _ops.check_sinkhorn_bwd_iters(n, iters)
        o = _ops.pre_full(x_flat, w_phi, packed, alpha_pre, bias_pre, alpha_post, bias_post,
                          alpha_res, bias_res, n, c, post_mult, pre_eps, rms_eps, iters, sk_eps,
                          sinkhorn=True, want_raw=train, want_saved=train, ssq=ssq)
        if train:
            ctx.save_for_backward(x_flat.detach().contiguous().view(B * L, NC), w_phi,
                                  alpha_pre, bias_pre, alpha_post, bias_post, alpha_res,
                                  bias_res, o["inv_rms"], o["mixes_raw"], o["h_res_raw"])
        ctx.cfg = (n, c, float(post_mult), float(pre_eps), (B, L, NC), iters, float(sk_eps))
        return (o["sub_in"].view(B, L, c), o["h_post"].view(B, L, n),
                o["h_res"].view(B, L, n, n))

    @staticmethod
    def backward(ctx, g_sub, g_hpost, g_hres):
        x2, w, a_pre, b_pre, a_post, b_post, a_res, b_res, inv, mixes, raw = ctx.saved_tensors
        n, c, post_mult, pre_eps, shape, iters, sk_eps = ctx.cfg
        g_raw = None
        if g_hres is not None:
            # The reference runs Sinkhorn on h_res_raw.float() and casts back, so the
            # gradient reaching the pre phase is rounded to the stream dtype.
            g_raw = _ops.sinkhorn_bwd(raw, g_hres.reshape(raw.shape), iters, sk_eps,
                                      out_dtype=x2.dtype)
        g = _pre_full_grads(x2, w, (a_pre, a_post, a_res), (b_pre, b_post, b_res), inv, mixes,
                            n, c, post_mult, pre_eps, shape, g_sub, None, g_hpost, g_raw)
        return (g[0], g[1], None, *g[2:], None, None, None, None, None, None, None, None)


class _PostPhaseFullFn(_ops.GradAwareFunction):
    """out = H_res . x + H_post (x) F_out (model/mhc_fused.py:720-772)."""

    @staticmethod
    def forward(ctx, x_flat, h_res, h_post, f_out, n, c, ssq_out=None):
        B, L, NC = x_flat.shape
        out = _ops.post(x_flat, h_res, h_post, f_out, n, c, ssq_out=ssq_out)
        if _ops.grad_wanted(ctx):
            ctx.save_for_backward(x_flat.detach().contiguous().view(B * L, NC), h_res, h_post,
                                  f_out)
        ctx.cfg = (n, c, (B, L, NC))
        return out.view(B, L, NC)

    @staticmethod
    def backward(ctx, g_out):
        x2, h_res, h_post, f_out = ctx.saved_tensors
        n, c, shape = ctx.cfg
        g_x, g_hr, g_hp, g_f = _ops.post_bwd(x2, h_res, h_post, f_out, n, c, g_out)
        return (g_x.view(shape), g_hr.view(h_res.shape), g_hp.view(h_post.shape),
                g_f.to(f_out.dtype).view(f_out.shape), None, None, None)


# ------------------------------------------------------------------- module

class MHCConnection_Fused(nn.Module):
    """One mHC-wrapped sublayer: x' = H_res . x + H_post (x) F(H_pre . x).

    Same constructor, parameters and forward contract as the reference
    (model/mhc_fused.py:775-834).  phi_weight is (n*dim, 2n + n^2) row-major
    with columns [pre 0:n | post n:2n | res 2n:, row-major (i, j)].
    """

    def __init__(self, n: int, dim: int, alpha_init: float = 0.01,
                 sinkhorn_iters: int = 10, post_mult_value: float = 2.0,
                 eps: float = 1e-6, pre_eps: float = 1e-6, sinkhorn_eps: float = 1e-6):
        super().__init__()
        assert _is_pow2(n) and n <= 16, f"n must be in {{1,2,4,8,16}}, got {n}"
        assert post_mult_value > 1.0
        self.n = n
        self.dim = dim
        self.nC = n * dim
        self.N2 = n * n
        self.fused_dim = 2 * n + self.N2
        self.sinkhorn_iters = sinkhorn_iters
        self.post_mult_value = post_mult_value
        self.pre_eps = pre_eps
        self.sinkhorn_eps = sinkhorn_eps
        self.eps = eps

        self.phi_weight = nn.Parameter(torch.empty(self.nC, self.fused_dim))
        nn.init.kaiming_uniform_(self.phi_weight, a=math.sqrt(5))
        self.alpha_pre = nn.Parameter(torch.tensor(alpha_init))
        self.bias_pre = nn.Parameter(torch.zeros(n))
        self.alpha_post = nn.Parameter(torch.tensor(alpha_init))
        self.bias_post = nn.Parameter(torch.zeros(n))
        self.alpha_res = nn.Parameter(torch.tensor(alpha_init))
        self.bias_res = nn.Parameter(torch.eye(n))
        self._phi_pack = _ops.PhiPack(H.MODE_FULL)

    def extra_repr(self) -> str:
        return (f"n={self.n}, dim={self.dim}, fused_dim={self.fused_dim}, "
                f"sinkhorn_iters={self.sinkhorn_iters}, post_mult_value={self.post_mult_value}, "
                f"backend=hip-gfx950")

    def forward(self, x_flat: torch.Tensor, sublayer_fn: Callable,
                in_norm: nn.Module = None, chain: _ops.StreamChain = None) -> torch.Tensor:
        """PRE (+Sinkhorn, one HIP launch) -> sublayer F -> POST (one HIP launch).

        in_norm (optional, not in the reference signature): an nn.RMSNorm over
        dim that F applies to its input first, i.e. F(z) = sublayer_fn(in_norm(z)).
        Without autograd it runs inside the pre launch; otherwise it is applied
        as a separate op, as when F contains it.
        chain (optional, not in the reference signature): a _ops.StreamChain
        shared by consecutive mHC calls.  The post launch then also writes the
        output rows' sums of squares, and the next call's pre launch takes
        them instead of a pass over its input of its own (shapes where that
        pass exists: n >= 8 or dim > 1024)."""
        packed = self._phi_pack.get(self.phi_weight, self.n, self.dim) if x_flat.is_cuda else None
        ssq = chain.take(x_flat, self.n, self.dim) if chain is not None else None
        ssq_out = chain.buffer(x_flat, self.n, self.dim) if chain is not None else None
        if in_norm is not None:
            if fusable_norm(in_norm, self.dim, x_flat):
                o = _ops.pre_full(x_flat, self.phi_weight, packed, self.alpha_pre, self.bias_pre,
                                  self.alpha_post, self.bias_post, self.alpha_res, self.bias_res,
                                  self.n, self.dim, self.post_mult_value, self.pre_eps, self.eps,
                                  self.sinkhorn_iters, self.sinkhorn_eps,
                                  norm=(in_norm.weight, norm_eps(in_norm, x_flat)), ssq=ssq)
                B, L, NC = x_flat.shape
                f_out = sublayer_fn(o["sub_in"].view(B, L, self.dim))
                out = _ops.post(x_flat, o["h_res"], o["h_post"], f_out, self.n, self.dim,
                                ssq_out=ssq_out).view(B, L, NC)
                return chain.put(out, ssq_out) if chain is not None else out
            fn = sublayer_fn
            sublayer_fn = lambda z: fn(in_norm(z))  # noqa: E731
        sublayer_in, h_post, h_res = _PreSinkhornFn.apply(
            x_flat, self.phi_weight, packed,
            self.alpha_pre, self.bias_pre, self.alpha_post, self.bias_post,
            self.alpha_res, self.bias_res,
            self.post_mult_value, self.pre_eps, self.eps, self.n, self.dim,
            self.sinkhorn_iters, self.sinkhorn_eps, ssq)
        f_out = sublayer_fn(sublayer_in)
        out = _PostPhaseFullFn.apply(x_flat, h_res, h_post, f_out, self.n, self.dim, ssq_out)
        return chain.put(out, ssq_out) if chain is not None else out
