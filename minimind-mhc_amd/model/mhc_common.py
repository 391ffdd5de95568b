"""mHC stream entry / exit on MI355X HIP kernels.

Drop-in for the reference module model/mhc_common.py:
  StreamExpand(n, D) : (B, L, D)   -> (B, L, n*D)   model/mhc_common.py:104-119
  MHCHead(n, D)      : (B, L, n*D) -> (B, L, D)     model/mhc_common.py:403-450
Both run hand-written gfx950 kernels through libmhc_amd.so; there is no CPU
or PyTorch forward path.
"""
from __future__ import annotations

import math

import torch
import torch.nn as nn

from . import _ops
from . import _hip as H


def _is_pow2(n: int) -> bool:
    return n >= 1 and (n & (n - 1)) == 0


def fusable_norm(norm, dim: int, x: torch.Tensor) -> bool:
    """True when an nn.RMSNorm over `dim` can run inside a HIP launch for this
    call: grad mode off (torch.no_grad / inference_mode) and an affine norm
    over exactly (dim,).  With grad mode on the norm stays a separate op even
    when nothing visible here requires grad: the sublayer F is opaque, and the
    fused launches record no autograd graph that gradients to F's parameters
    could flow through."""
    if not isinstance(norm, nn.RMSNorm) or norm.weight is None:
        return False
    if tuple(norm.normalized_shape) != (dim,) or not x.is_cuda:
        return False
    return not torch.is_grad_enabled()


def norm_eps(norm: nn.RMSNorm, x: torch.Tensor) -> float:
    """nn.RMSNorm's eps (None means the dtype's machine epsilon, as torch uses)."""
    return float(norm.eps) if norm.eps is not None else float(torch.finfo(x.dtype).eps)


class _StreamExpandFn(_ops.GradAwareFunction):
    @staticmethod
    def forward(ctx, x, n):
        ctx.n = n
        return _ops.stream_expand(x, n)

    @staticmethod
    def backward(ctx, g):
        B, L, ND = g.shape
        return g.view(B, L, ctx.n, ND // ctx.n).sum(dim=2), None


class StreamExpand(nn.Module):
    """(B, L, D) -> (B, L, n*D): n identical copies of the stream (no parameters)."""

    def __init__(self, n: int, dim: int):
        super().__init__()
        self.n = n
        self.dim = dim

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.n == 1:
            return x
        return _StreamExpandFn.apply(x, self.n)

    def forward_normed(self, x: torch.Tensor, in_norm: nn.Module,
                       chain: _ops.StreamChain = None) -> torch.Tensor:
        """self(in_norm(x)), the model's entry (model/model_minimind.py:365):
        one HIP launch (RMSNorm + n copies) when no autograd is needed.  With a
        chain (see MHCConnection_Fused.forward) that launch also writes the
        stream's per-row sums of squares for the first connection."""
        if fusable_norm(in_norm, self.dim, x):
            ssq = (chain.buffer(x, self.n, self.dim, rows=x.numel() // self.dim)
                   if chain is not None and self.n > 1 else None)
            out = _ops.expand_norm(x, in_norm.weight, norm_eps(in_norm, x), self.n, ssq_out=ssq)
            return chain.put(out, ssq) if chain is not None else out
        out = self(in_norm(x))
        return chain.put(out, None) if chain is not None else out


class _MHCHeadFn(_ops.GradAwareFunction):
    """MHCHead forward on the HIP kernel (model/mhc_common.py:311-400)."""

    @staticmethod
    def forward(ctx, x_flat, w_phi, alpha, bias, pre_eps, rms_eps, n, c, packed=None, ssq=None):
        B, L, NC = x_flat.shape
        train = _ops.grad_wanted(ctx)
        if packed is None and n > 1:  # called without the module's pack
            packed = _ops.packed_phi(w_phi, n, c, H.MODE_HEAD, training=_ops.grad_wanted(ctx, 1))
        out, inv, mix = _ops.head(x_flat, w_phi, packed, alpha, bias, n, c, pre_eps, rms_eps,
                                  want_saved=train, ssq=ssq)
        if train:
            ctx.save_for_backward(x_flat.detach().contiguous().view(B * L, NC), w_phi, alpha,
                                  bias, inv, mix)
        ctx.cfg = (n, c, float(pre_eps), (B, L, NC))
        return out.view(B, L, c)

    @staticmethod
    def backward(ctx, g_out):
        x2, w, alpha, bias, inv, mix = ctx.saved_tensors
        n, c, pre_eps, shape = ctx.cfg
        alphas, biases = (alpha, None, None), (bias, None, None)
        g_x, g_raw = _ops.pre_bwd(x2, w, alphas, biases, inv, mix, n, c, H.MODE_HEAD, 0.0,
                                  pre_eps, g_sub=g_out)
        g_w, g_a, g_b = _ops.pre_bwd_weights(x2, inv, mix, g_raw, w, alphas, n, c, H.MODE_HEAD)
        return (g_x.view(shape), g_w, g_a[0].to(alpha.dtype).reshape(alpha.shape),
                g_b[0].to(bias.dtype).view(bias.shape), None, None, None, None, None, None)


class _RMSFn(_ops.GradAwareFunction):
    """y = x * rsqrt(mean(x^2) + eps), no gain (MHCHead with n == 1)."""

    @staticmethod
    def forward(ctx, x_flat, eps):
        B, L, C = x_flat.shape
        out, inv, _ = _ops.head(x_flat, None, None, None, None, 1, C, 0.0, eps,
                                want_saved=_ops.grad_wanted(ctx))
        if inv is not None:
            ctx.save_for_backward(x_flat.detach().contiguous().view(B * L, C), inv)
        return out.view(B, L, C)

    @staticmethod
    def backward(ctx, g_out):
        x2, inv = ctx.saved_tensors
        C = x2.shape[1]
        g_x, _ = _ops.pre_bwd(x2, None, (None,) * 3, (None,) * 3, inv, None, 1, C, H.MODE_RMS,
                              0.0, 0.0, g_sub=g_out)
        return g_x.view(g_out.shape), None


class MHCHead(nn.Module):
    """(B, L, n*D) -> (B, L, D): out = sum_i (sigmoid(alpha * (x_norm . phi)_i + beta_i) + eps) * x_i.

    Same constructor and parameters as the reference (model/mhc_common.py:403-450):
    phi_weight (n*dim, n), bias (n,), alpha of shape (1,).
    """

    def __init__(self, n: int, dim: int, alpha_init: float = 0.01,
                 eps: float = 1e-6, pre_eps: float = 1e-6):
        super().__init__()
        assert _is_pow2(n) and n <= 16, f"n must be in {{1,2,4,8,16}}, got {n}"
        self.n = n
        self.dim = dim
        self.nC = n * dim
        self.eps = eps
        self.pre_eps = pre_eps
        self.phi_weight = nn.Parameter(torch.empty(self.nC, n))
        nn.init.kaiming_uniform_(self.phi_weight, a=math.sqrt(5))
        self.bias = nn.Parameter(torch.zeros(n))
        self.alpha = nn.Parameter(torch.full((1,), alpha_init))
        self._phi_pack = _ops.PhiPack(H.MODE_HEAD)

    def extra_repr(self) -> str:
        return f"n={self.n}, dim={self.dim}, backend=hip-gfx950"

    def forward(self, x_flat: torch.Tensor, out_norm: nn.Module = None,
                chain: _ops.StreamChain = None) -> torch.Tensor:
        """out_norm: an nn.RMSNorm over dim applied to the head output (the
        model's final norm, model/model_minimind.py:367-370); without autograd
        it runs inside the head launch.  chain: as MHCConnection_Fused.forward
        (the head takes the last connection's sums of squares)."""
        ssq = chain.take(x_flat, self.n, self.dim) if chain is not None and self.n > 1 else None
        if out_norm is not None:
            if fusable_norm(out_norm, self.dim, x_flat):
                packed = (self._phi_pack.get(self.phi_weight, self.n, self.dim)
                          if self.n > 1 else None)
                out, _, _ = _ops.head(x_flat, self.phi_weight, packed, self.alpha, self.bias,
                                      self.n, self.dim, self.pre_eps, self.eps,
                                      norm=(out_norm.weight, norm_eps(out_norm, x_flat)), ssq=ssq)
                return out.view(*x_flat.shape[:-1], self.dim)
            return out_norm(self(x_flat, chain=chain))
        if self.n == 1:
            return _RMSFn.apply(x_flat, self.eps)
        packed = self._phi_pack.get(self.phi_weight, self.n, self.dim) if x_flat.is_cuda else None
        return _MHCHeadFn.apply(x_flat, self.phi_weight, self.alpha, self.bias,
                                self.pre_eps, self.eps, self.n, self.dim, packed, ssq)
