"""Tensor-level wrappers of the C-ABI entry points.

Each function validates shapes, allocates the outputs with torch.empty on the
input's device (the library never allocates), and enqueues the kernel on the
current stream.  Inputs are made contiguous, as the reference's Functions do
(model/mhc_fused.py:585-586, :729-732).
"""
from __future__ import annotations

import threading
import weakref
from typing import Optional

import torch

from . import _hip as H

_GRAD = threading.local()


class GradAwareFunction(torch.autograd.Function):
    """An autograd Function whose forward can tell whether the caller had grad
    mode on.  ctx.needs_input_grad follows requires_grad alone, also under
    torch.no_grad(), so a forward that keys on it alone would save tensors,
    write backward-only outputs and repack trainable weights on every
    inference call."""

    @classmethod
    def apply(cls, *args, **kwargs):
        prev = getattr(_GRAD, "on", True)
        _GRAD.on = torch.is_grad_enabled()
        try:
            return super().apply(*args, **kwargs)
        finally:
            _GRAD.on = prev


def grad_wanted(ctx, index: Optional[int] = None) -> bool:
    """Inside a GradAwareFunction's forward: whether a gradient of any input
    (or of input `index`) will be asked for."""
    if not getattr(_GRAD, "on", True):
        return False
    return any(ctx.needs_input_grad) if index is None else bool(ctx.needs_input_grad[index])


class PhiPack:
    """MFMA operand image of a projection weight, rebuilt when the weight changes.

    Policy:
      * A weight that trains (grad mode on and phi.requires_grad) is repacked
        on every call.  Its values change every optimizer step, and in-place
        writes through .data (p.data.copy_ / normal_) do not bump the version
        counter, so no cache key could see them.  The pack is one small launch.
      * Otherwise (inference, frozen weights) the image is cached for one weight
        tensor object (held by weak reference, so a replaced parameter never
        aliases a freed one) at one value of its version counter, which
        optimizer steps, load_state_dict and copy_ bump.  A write through .data
        is invisible to that key: call invalidate() after one.  Inference
        tensors, which have no version counter, are repacked on every call.
    The cache is not pickled or deep-copied; a copy rebuilds it lazily.
    No reference counterpart: the reference's kernels read the row-major weight
    directly (model/mhc_fused.py:217-229).
    """

    def __init__(self, mode: int):
        self.mode = mode
        self.invalidate()

    def invalidate(self) -> None:
        """Drop the cached image; the next call repacks."""
        self._src = None
        self._key = None
        self._buf: Optional[torch.Tensor] = None

    def __getstate__(self):
        return {"mode": self.mode}

    def __setstate__(self, state):
        self.mode = state["mode"]
        self.invalidate()

    def get(self, phi: torch.Tensor, n: int, C: int,
            training: Optional[bool] = None) -> Optional[torch.Tensor]:
        """The image of phi (None when (n, C, dtype) has no MFMA kernel): the
        bf16 operand image for a bf16 phi (kernels for bf16 streams), the
        split hi / lo image for an fp32 phi (kernels for fp32 streams).
        training: whether phi trains in this call; default grad mode and
        phi.requires_grad (inside an autograd Function's forward, where grad
        mode is off, pass grad_wanted(ctx, <phi's index>))."""
        lib = H.load()
        if phi.dtype == torch.bfloat16:
            nbytes = lib.mhc_phi_packed_bytes(n, C, self.mode)
            pack = lib.mhc_phi_pack
        elif phi.dtype == torch.float32:
            nbytes = lib.mhc_phi_split_bytes(n, C, self.mode)
            pack = lib.mhc_phi_pack_split
        else:
            return None
        if nbytes <= 0:
            return None
        if training is None:
            training = torch.is_grad_enabled() and phi.requires_grad
        try:
            version = None if training else phi._version
        except RuntimeError:
            version = None
        key = (phi.data_ptr(), version, phi.device, phi.dtype, n, C)
        src = self._src() if self._src is not None else None
        if version is not None and src is phi and key == self._key and self._buf is not None:
            return self._buf
        w = phi.detach().contiguous()
        buf = torch.empty(nbytes, dtype=torch.uint8, device=phi.device)
        H.check(pack(w.data_ptr(), H.dtype_tag(w), buf.data_ptr(), n, C, self.mode,
                     H.stream(phi.device)), "mhc_phi_pack")
        if version is None:
            self.invalidate()
        else:
            self._src = weakref.ref(phi)
            self._key = key
            self._buf = buf
        return buf


# Packs of weights that no module owns (the reference-style autograd Functions
# called directly): id(phi), mode -> (weak reference to phi, PhiPack).  An entry
# goes (with its device image) as soon as its weight is freed.
_PACKS: dict = {}


def _drop_pack(key, ref) -> None:
    ent = _PACKS.get(key)
    if ent is not None and ent[0] is ref:
        del _PACKS[key]


def packed_phi(phi: torch.Tensor, n: int, C: int, mode: int,
               training: Optional[bool] = None) -> Optional[torch.Tensor]:
    """MFMA image of phi for a caller without a PhiPack of its own (None when
    the shape or dtype has no MFMA kernel); training as in PhiPack.get."""
    if not phi.is_cuda:
        return None
    key = (id(phi), mode)
    ent = _PACKS.get(key)
    if ent is None or ent[0]() is not phi:
        ent = (weakref.ref(phi, lambda ref, key=key: _drop_pack(key, ref)), PhiPack(mode))
        _PACKS[key] = ent
    return ent[1].get(phi, n, C, training)


# ---------------------------------------------- sums of squares along a chain
SSQ_COLS = 128  # one fp32 partial per 128 columns of C (kSsqCols)


def ssq_wanted(dtype: torch.dtype, n: int, C: int) -> bool:
    """Whether a stream of this shape carries its rows' sums of squares from the
    launch that writes it to the pre launch that reads it: bf16, C a multiple
    of 128, and a pre kernel that would otherwise read the stream once more
    to form them (n = 8, n = 16, or C > 1024)."""
    return (dtype == torch.bfloat16 and C % SSQ_COLS == 0
            and (n in (8, 16) or (n >= 2 and C > 1024)))


class StreamChain:
    """Carries per-row sums of squares along a chain of mHC calls.

    The launch that writes a stream (the post phase, or the entry RMSNorm +
    StreamExpand) also writes its rows' partial sums of squares
    ([M, C / 128] fp32); the next pre launch that reads that exact tensor
    takes them instead of a pass over x of its own.  A caller that hands
    each call's output unchanged to the next call (as the MiniMind blocks do)
    creates one chain per forward and passes it to every mHC call; the sums
    are used only when the next call's input is the very tensor object the
    previous call returned.  Writing into that tensor in place between the
    calls is the caller's to avoid (the chain cannot see it).
    No reference counterpart."""

    __slots__ = ("src", "ssq")

    def __init__(self):
        self.src = None
        self.ssq = None

    def take(self, x: torch.Tensor, n: int, C: int) -> Optional[torch.Tensor]:
        """The sums of squares of x's rows, or None when x is not the tensor the
        chain last recorded (or the shape carries none)."""
        if self.ssq is None or self.src is not x:
            return None
        M = x.numel() // (n * C) if n * C else 0
        if tuple(self.ssq.shape) != (M, C // SSQ_COLS) or self.ssq.device != x.device:
            return None
        return self.ssq

    def buffer(self, like: torch.Tensor, n: int, C: int,
               rows: Optional[int] = None) -> Optional[torch.Tensor]:
        """A buffer for the sums of squares of an n-stream of `rows` tokens
        (default: `like` is such a stream, [..., n*C]) with like's dtype and
        device, or None when that shape carries none."""
        if not like.is_cuda or not ssq_wanted(like.dtype, n, C):
            return None
        M = like.numel() // (n * C) if rows is None else rows
        return torch.empty(M, C // SSQ_COLS, dtype=torch.float32, device=like.device)

    def put(self, out: torch.Tensor, ssq: Optional[torch.Tensor]) -> torch.Tensor:
        """Record out (the tensor handed to the next call) and its sums."""
        self.src = out
        self.ssq = ssq
        return out


def _check_numel(name: str, t: torch.Tensor, want: int) -> None:
    # The kernels index biases by stream / matrix element; a short tensor would be
    # read out of bounds, so sizes are enforced here (the C ABI sees only pointers).
    if t.numel() != want:
        raise ValueError(f"mhc_amd: {name} has {t.numel()} elements, expected {want}")


def _rows(x_flat: torch.Tensor, NC: int) -> torch.Tensor:
    if x_flat.shape[-1] != NC:
        raise ValueError(f"mhc_amd: last dim {x_flat.shape[-1]} != n*C = {NC}")
    return x_flat.contiguous().view(-1, NC)


def _norm_args(norm, C: int, dev):
    """(weight pointer, dtype tag, eps, keep-alive tensor) of an RMSNorm over C
    fused into a pre-phase / head launch, or Nones without one."""
    if norm is None:
        return None, 0, 0.0, None
    w, eps = norm
    H.require_device(w)
    wc = w.detach().contiguous()
    _check_numel("norm weight", wc, C)
    if wc.device != dev:
        raise ValueError("mhc_amd: norm weight is on another device")
    return wc.data_ptr(), H.dtype_tag(wc), float(eps), wc


def _ssq_ptr(ssq, M: int, C: int):
    if ssq is None:
        return None
    if ssq.dtype != torch.float32 or tuple(ssq.shape) != (M, C // SSQ_COLS) or not ssq.is_contiguous():
        raise ValueError(f"mhc_amd: sums of squares must be contiguous fp32 [{M}, {C // SSQ_COLS}]")
    return ssq.data_ptr()


def pre_full(x_flat, phi, packed, a_pre, b_pre, a_post, b_post, a_res, b_res, n, C,
             post_mult, pre_eps, rms_eps, sk_iters, sk_eps, *, sinkhorn=True,
             want_h_pre=False, want_raw=False, want_saved=False, norm=None, ssq=None):
    """Fused pre phase (+ Sinkhorn).  Returns a dict of [M, ...] tensors.
    norm=(weight [C], eps): "sub_in" is RMSNorm(pre-aggregate) instead.
    ssq: x's per-row partial sums of squares ([M, C / 128] fp32, from the
    launch that wrote x), or None."""
    dev = H.require_device(x_flat, phi, a_pre, b_pre, a_post, b_post, a_res, b_res)
    NC = n * C
    FD = 2 * n + n * n
    if tuple(phi.shape) != (NC, FD):
        raise ValueError(f"mhc_amd: phi_weight shape {tuple(phi.shape)} != ({NC}, {FD})")
    x2 = _rows(x_flat, NC)
    M = x2.shape[0]
    phi_c = phi.detach().contiguous()
    a_pre, b_pre, a_post, b_post, a_res, b_res = H.params_like(
        x2, a_pre, b_pre, a_post, b_post, a_res, b_res)
    for nm, tt, want in (("alpha_pre", a_pre, 1), ("alpha_post", a_post, 1), ("alpha_res", a_res, 1),
                         ("bias_pre", b_pre, n), ("bias_post", b_post, n), ("bias_res", b_res, n * n)):
        _check_numel(nm, tt, want)
    kw = dict(dtype=x2.dtype, device=dev)
    out = {
        "sub_in": torch.empty(M, C, **kw),
        "h_post": torch.empty(M, n, **kw),
        "h_pre": torch.empty(M, n, **kw) if want_h_pre else None,
        "h_res_raw": torch.empty(M, n, n, **kw) if want_raw else None,
        "h_res": torch.empty(M, n, n, **kw) if sinkhorn else None,
        "inv_rms": torch.empty(M, dtype=torch.float32, device=dev) if want_saved else None,
        "mixes_raw": torch.empty(M, FD, dtype=torch.float32, device=dev) if want_saved else None,
    }
    args = (x2.data_ptr(), H.dtype_tag(x2), phi_c.data_ptr(), H.dtype_tag(phi_c), H.ptr(packed),
            a_pre.data_ptr(), b_pre.data_ptr(), a_post.data_ptr(), b_post.data_ptr(),
            a_res.data_ptr(), b_res.data_ptr(), H.dtype_tag(a_pre),
            out["sub_in"].data_ptr(), H.ptr(out["h_pre"]), out["h_post"].data_ptr(),
            H.ptr(out["h_res_raw"]), H.ptr(out["h_res"]), H.ptr(out["inv_rms"]),
            H.ptr(out["mixes_raw"]), M, n, C, float(post_mult), float(pre_eps), float(rms_eps),
            int(sk_iters), float(sk_eps))
    sp = _ssq_ptr(ssq, M, C)
    if norm is None:
        H.check(H.load().mhc_pre_fwd(*args, sp, H.stream(dev)), "mhc_pre_fwd")
    else:
        wp, wdt, weps, _keep = _norm_args(norm, C, dev)
        H.check(H.load().mhc_pre_norm_fwd(*args, wp, wdt, weps, sp, H.stream(dev)),
                "mhc_pre_norm_fwd")
    return out


def pre_nohres(x_flat, phi, packed, a_pre, b_pre, a_post, b_post, n, C, post_mult, pre_eps,
               rms_eps, *, want_h_pre=False, want_saved=False, norm=None, ssq=None):
    dev = H.require_device(x_flat, phi, a_pre, b_pre, a_post, b_post)
    NC = n * C
    FD = 2 * n
    if tuple(phi.shape) != (NC, FD):
        raise ValueError(f"mhc_amd: phi_weight shape {tuple(phi.shape)} != ({NC}, {FD})")
    x2 = _rows(x_flat, NC)
    M = x2.shape[0]
    phi_c = phi.detach().contiguous()
    a_pre, b_pre, a_post, b_post = H.params_like(x2, a_pre, b_pre, a_post, b_post)
    for nm, tt, want in (("alpha_pre", a_pre, 1), ("alpha_post", a_post, 1),
                         ("bias_pre", b_pre, n), ("bias_post", b_post, n)):
        _check_numel(nm, tt, want)
    kw = dict(dtype=x2.dtype, device=dev)
    out = {
        "sub_in": torch.empty(M, C, **kw),
        "h_post": torch.empty(M, n, **kw),
        "h_pre": torch.empty(M, n, **kw) if want_h_pre else None,
        "inv_rms": torch.empty(M, dtype=torch.float32, device=dev) if want_saved else None,
        "mixes_raw": torch.empty(M, FD, dtype=torch.float32, device=dev) if want_saved else None,
    }
    args = (x2.data_ptr(), H.dtype_tag(x2), phi_c.data_ptr(), H.dtype_tag(phi_c), H.ptr(packed),
            a_pre.data_ptr(), b_pre.data_ptr(), a_post.data_ptr(), b_post.data_ptr(),
            H.dtype_tag(a_pre), out["sub_in"].data_ptr(), H.ptr(out["h_pre"]),
            out["h_post"].data_ptr(), H.ptr(out["inv_rms"]), H.ptr(out["mixes_raw"]),
            M, n, C, float(post_mult), float(pre_eps), float(rms_eps))
    sp = _ssq_ptr(ssq, M, C)
    if norm is None:
        H.check(H.load().mhc_pre_nohres_fwd(*args, sp, H.stream(dev)), "mhc_pre_nohres_fwd")
    else:
        wp, wdt, weps, _keep = _norm_args(norm, C, dev)
        H.check(H.load().mhc_pre_nohres_norm_fwd(*args, wp, wdt, weps, sp, H.stream(dev)),
                "mhc_pre_nohres_norm_fwd")
    return out


def head(x_flat, phi, packed, alpha, bias, n, C, pre_eps, rms_eps, *, want_saved=False,
         norm=None, ssq=None):
    """MHCHead forward; n == 1 is the plain RMSNorm (phi/alpha/bias unused).
    norm=(weight [C], eps): the model's final RMSNorm applied in the same launch."""
    NC = n * C
    x2 = _rows(x_flat, NC)
    M = x2.shape[0]
    if n == 1:
        dev = H.require_device(x_flat)
        phi_p = a_p = b_p = None
        phi_dt = pdt = H.DTYPE_F32
    else:
        dev = H.require_device(x_flat, phi, alpha, bias)
        if tuple(phi.shape) != (NC, n):
            raise ValueError(f"mhc_amd: phi_weight shape {tuple(phi.shape)} != ({NC}, {n})")
        phi_c = phi.detach().contiguous()
        alpha_c, bias_c = H.params_like(x2, alpha, bias)
        _check_numel("alpha", alpha_c, 1)
        _check_numel("bias", bias_c, n)
        phi_p, a_p, b_p = phi_c.data_ptr(), alpha_c.data_ptr(), bias_c.data_ptr()
        phi_dt, pdt = H.dtype_tag(phi_c), H.dtype_tag(alpha_c)
    out = torch.empty(M, C, dtype=x2.dtype, device=dev)
    inv = torch.empty(M, dtype=torch.float32, device=dev) if want_saved else None
    mix = torch.empty(M, n, dtype=torch.float32, device=dev) if (want_saved and n > 1) else None
    args = (x2.data_ptr(), H.dtype_tag(x2), phi_p, phi_dt, H.ptr(packed), a_p, b_p, pdt,
            out.data_ptr(), H.ptr(inv), H.ptr(mix), M, n, C, float(pre_eps), float(rms_eps))
    sp = _ssq_ptr(ssq, M, C) if n > 1 else None
    if norm is None:
        H.check(H.load().mhc_head_fwd(*args, sp, H.stream(dev)), "mhc_head_fwd")
    else:
        wp, wdt, weps, _keep = _norm_args(norm, C, dev)
        H.check(H.load().mhc_head_norm_fwd(*args, wp, wdt, weps, sp, H.stream(dev)),
                "mhc_head_norm_fwd")
    return out, inv, mix


def post(x_flat, h_res, h_post, f_out, n, C, ssq_out=None):
    """out = H_res . x + H_post (x) F; h_res None means identity (use_mhc = 2).
    ssq_out: an [M, C / 128] fp32 buffer that receives out's per-row partial
    sums of squares (for the next pre launch), or None."""
    dev = H.require_device(x_flat, h_res, h_post, f_out)
    NC = n * C
    x2 = _rows(x_flat, NC)
    M = x2.shape[0]
    hp = h_post.contiguous().view(M, n)
    f2 = f_out.contiguous().view(M, C)
    if hp.dtype != (h_res.dtype if h_res is not None else hp.dtype):
        raise TypeError("mhc_amd: h_res and h_post must share a dtype")
    out = torch.empty_like(x2)
    lib = H.load()
    sp = _ssq_ptr(ssq_out, M, C)
    if h_res is not None:
        hr = h_res.contiguous().view(M, n, n)
        rc = lib.mhc_post_fwd(x2.data_ptr(), H.dtype_tag(x2), hr.data_ptr(), hp.data_ptr(),
                              H.dtype_tag(hp), f2.data_ptr(), H.dtype_tag(f2), out.data_ptr(),
                              M, n, C, sp, H.stream(dev))
        H.check(rc, "mhc_post_fwd")
    else:
        rc = lib.mhc_post_nohres_fwd(x2.data_ptr(), H.dtype_tag(x2), hp.data_ptr(),
                                     H.dtype_tag(hp), f2.data_ptr(), H.dtype_tag(f2),
                                     out.data_ptr(), M, n, C, sp, H.stream(dev))
        H.check(rc, "mhc_post_nohres_fwd")
    return out


def sinkhorn(m: torch.Tensor, iters: int, eps: float) -> torch.Tensor:
    dev = H.require_device(m)
    N = m.shape[-1]
    if m.dim() < 2 or m.shape[-2] != N:
        raise ValueError(f"mhc_amd: last two dims must be square, got {tuple(m.shape)}")
    mc = m.contiguous()
    out = torch.empty_like(mc)
    batch = mc.numel() // (N * N) if N > 0 else 0
    rc = H.load().mhc_sinkhorn_fwd(mc.data_ptr(), out.data_ptr(), H.dtype_tag(mc), batch, N,
                                   int(iters), float(eps), H.stream(dev))
    H.check(rc, "mhc_sinkhorn_fwd")
    return out


def expand_norm(x: torch.Tensor, weight: torch.Tensor, eps: float, n: int,
                ssq_out=None) -> torch.Tensor:
    """RMSNorm over the last dim (gain weight) followed by StreamExpand to n
    copies, one launch: [B, L, C] -> [B, L, n*C].  ssq_out as in post."""
    dev = H.require_device(x, weight)
    B, L, C = x.shape
    xc = x.contiguous()
    wp, wdt, weps, _keep = _norm_args((weight, eps), C, dev)
    out = torch.empty(B, L, n * C, dtype=x.dtype, device=dev)
    rc = H.load().mhc_expand_norm_fwd(xc.data_ptr(), H.dtype_tag(xc), wp, wdt, out.data_ptr(),
                                      B * L, n, C, weps, _ssq_ptr(ssq_out, B * L, C),
                                      H.stream(dev))
    H.check(rc, "mhc_expand_norm_fwd")
    return out


def pre_token_threshold(max_tokens: int = -1) -> int:
    """Set (max_tokens >= 0) or query the batch size at or below which the
    pre-phase launches use the small-batch group kernel (bit-identical to the
    large-batch kernels); returns the previous value."""
    return int(H.load().mhc_pre_token_threshold(int(max_tokens)))


def pre_row_staging(on: int = -1) -> int:
    """Set (on >= 0) or query whether the persistent pre kernel loads x tiles
    as whole rows staged through LDS where the shape allows; returns the
    previous setting (0 or 1).  The two agree to rounding (the row sums of
    squares are added in another order)."""
    return int(H.load().mhc_pre_row_staging(int(on)))


def pre_group_split_tokens(max_tokens: int = -1) -> int:
    """Set (max_tokens >= 0) or query the batch size at or below which the
    n = 8 small-batch pre phase runs as two launches (the projection split
    over the output tiles; bit-identical); returns the previous value."""
    return int(H.load().mhc_pre_group_split_tokens(int(max_tokens)))


def stream_expand(x: torch.Tensor, n: int) -> torch.Tensor:
    dev = H.require_device(x)
    B, L, D = x.shape
    xc = x.contiguous()
    out = torch.empty(B, L, n * D, dtype=x.dtype, device=dev)
    rc = H.load().mhc_stream_expand_fwd(xc.data_ptr(), out.data_ptr(), xc.element_size(),
                                        B * L, n, D, H.stream(dev))
    H.check(rc, "mhc_stream_expand_fwd")
    return out


# ------------------------------------------------------------------ backward
# Gradients come back in the dtypes the reference's backward kernels store:
# the forward inputs' dtypes, with the per-token g_raw in fp32.

def post_bwd(x_flat, h_res, h_post, f_out, n, C, g_out):
    """(g_x, g_h_res, g_h_post, g_f) of out = H_res . x + H_post (x) F.  With
    h_res None (use_mhc = 2) g_x is g_out itself and g_h_res is None."""
    dev = H.require_device(g_out, h_post, f_out, h_res, x_flat if h_res is not None else None)
    NC = n * C
    M = g_out.numel() // NC
    hp = h_post.contiguous().view(M, n)
    f2 = f_out.contiguous().view(M, C)
    g_hp = torch.empty_like(hp)
    g_f = torch.empty_like(f2)
    lib = H.load()
    if h_res is None:
        g2 = _rows(g_out, NC)
        rc = lib.mhc_post_nohres_bwd(hp.data_ptr(), H.dtype_tag(hp), f2.data_ptr(), H.dtype_tag(f2),
                                     g2.data_ptr(), H.dtype_tag(g2), None, g_hp.data_ptr(),
                                     g_f.data_ptr(), M, n, C, H.stream(dev))
        H.check(rc, "mhc_post_nohres_bwd")
        return g2, None, g_hp, g_f
    x2 = _rows(x_flat, NC)
    g2 = _rows(g_out, NC)
    if g2.dtype != x2.dtype:
        g2 = g2.to(x2.dtype)
    hr = h_res.contiguous().view(M, n, n)
    if hr.dtype != hp.dtype:
        raise TypeError("mhc_amd: h_res and h_post must share a dtype")
    g_x = torch.empty_like(x2)
    g_hr = torch.empty_like(hr)
    rc = lib.mhc_post_bwd(x2.data_ptr(), H.dtype_tag(x2), hr.data_ptr(), hp.data_ptr(),
                          H.dtype_tag(hp), f2.data_ptr(), H.dtype_tag(f2), g2.data_ptr(),
                          g_x.data_ptr(), g_hr.data_ptr(), g_hp.data_ptr(), g_f.data_ptr(),
                          M, n, C, H.stream(dev))
    H.check(rc, "mhc_post_bwd")
    return g_x, g_hr, g_hp, g_f


def pre_bwd(x2, phi, alphas, biases, inv_rms, mixes, n, C, mode, post_mult, pre_eps,
            g_sub=None, g_hpre=None, g_hpost=None, g_hres=None):
    """Per-token pre-phase backward.  alphas / biases: (pre, post, res) with
    None for absent segments.  Returns (g_x [M, n*C] x dtype, g_raw [M, FD] fp32
    or None for mode RMS)."""
    grads = [g for g in (g_sub, g_hpre, g_hpost, g_hres) if g is not None]
    dev = H.require_device(x2, inv_rms, *grads)
    M = x2.shape[0]
    gdt = grads[0].dtype if grads else x2.dtype
    g_sub, g_hpre, g_hpost, g_hres = (None if g is None else g.to(gdt).contiguous()
                                      for g in (g_sub, g_hpre, g_hpost, g_hres))
    g_x = torch.empty_like(x2)
    if mode == H.MODE_RMS:
        phi_p = phi_dt = None
        ps = [None] * 5
        pdt = H.DTYPE_F32
        g_raw = None
    else:
        FD = {H.MODE_FULL: 2 * n + n * n, H.MODE_NOHRES: 2 * n, H.MODE_HEAD: n}[mode]
        phi_c = phi.detach().contiguous()
        phi_p, phi_dt = phi_c.data_ptr(), H.dtype_tag(phi_c)
        present = [p for p in (alphas[0], biases[0], alphas[1], biases[1], alphas[2]) if p is not None]
        conv = iter(H.params_like(x2, *present))
        ps = [None if p is None else next(conv)
              for p in (alphas[0], biases[0], alphas[1], biases[1], alphas[2])]
        pdt = H.dtype_tag(ps[0])
        g_raw = torch.empty(M, FD, dtype=torch.float32, device=dev)
    rc = H.load().mhc_pre_bwd(
        x2.data_ptr(), H.dtype_tag(x2), phi_p, phi_dt if phi_dt is not None else H.DTYPE_F32,
        *[H.ptr(p) for p in ps], pdt, inv_rms.data_ptr(), H.ptr(mixes),
        H.ptr(g_sub), H.ptr(g_hpre), H.ptr(g_hpost), H.ptr(g_hres),
        H.dtype_tag(g_sub if g_sub is not None else x2), g_x.data_ptr(), H.ptr(g_raw),
        M, n, C, mode, float(post_mult), float(pre_eps), H.stream(dev))
    H.check(rc, "mhc_pre_bwd")
    return g_x, g_raw


def pre_bwd_weights(x2, inv_rms, mixes, g_raw, phi, alphas, n, C, mode):
    """(g_phi, [g_alpha_seg], [g_bias_seg]) from pre_bwd's g_raw; alphas as in
    pre_bwd.  g_alpha_* are 0-dim, g_bias_* flat, all in the alphas' dtype."""
    dev = H.require_device(x2, inv_rms, mixes, g_raw, phi)
    M = x2.shape[0]
    present = [a for a in alphas if a is not None]
    conv = iter(H.params_like(x2, *present))
    al = [None if a is None else next(conv) for a in alphas]
    pdt = al[0].dtype
    lib = H.load()
    g_phi = torch.empty(phi.shape, dtype=phi.dtype, device=dev)
    sizes = (n, n, n * n)
    g_alpha = [None if a is None else torch.empty((), dtype=pdt, device=dev) for a in al]
    g_bias = [None if a is None else torch.empty(sizes[i], dtype=pdt, device=dev)
              for i, a in enumerate(al)]
    if M == 0:
        g_phi.zero_()
        for t in g_alpha + g_bias:
            if t is not None:
                t.zero_()
        return g_phi, g_alpha, g_bias
    nbytes = lib.mhc_pre_bwd_weights_workspace_bytes(M, n, C, mode)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    rc = lib.mhc_pre_bwd_weights(
        x2.data_ptr(), H.dtype_tag(x2), inv_rms.data_ptr(), mixes.data_ptr(), g_raw.data_ptr(),
        *[H.ptr(a) for a in al], H.dtype_tag(al[0]), g_phi.data_ptr(), H.dtype_tag(g_phi),
        H.ptr(g_alpha[0]), H.ptr(g_bias[0]), H.ptr(g_alpha[1]), H.ptr(g_bias[1]),
        H.ptr(g_alpha[2]), H.ptr(g_bias[2]), ws.data_ptr(), nbytes, M, n, C, mode,
        H.stream(dev))
    H.check(rc, "mhc_pre_bwd_weights")
    return g_phi, g_alpha, g_bias


def check_sinkhorn_bwd_iters(n: int, iters: int) -> None:
    """Raise, before a forward whose Sinkhorn will need a gradient, when the
    backward kernel cannot take `iters` iterations for n (it would otherwise
    fail only at backward)."""
    cap = int(H.load().mhc_sinkhorn_bwd_max_iters(int(n)))
    if iters > cap:
        raise ValueError(f"mhc_amd: sinkhorn_iters={iters} exceeds what the Sinkhorn backward "
                         f"takes for n={n} ({cap}); train with sinkhorn_iters <= {cap}")


def sinkhorn_bwd(m: torch.Tensor, g: torch.Tensor, iters: int, eps: float,
                 out_dtype=None) -> torch.Tensor:
    """d sinkhorn(m) / d m applied to g, stored in out_dtype (default m's)."""
    dev = H.require_device(m, g)
    N = m.shape[-1]
    mc = m.contiguous()
    gc = g.contiguous()
    out = torch.empty(mc.shape, dtype=out_dtype or mc.dtype, device=dev)
    batch = mc.numel() // (N * N) if N > 0 else 0
    rc = H.load().mhc_sinkhorn_bwd(mc.data_ptr(), H.dtype_tag(mc), gc.data_ptr(), H.dtype_tag(gc),
                                   out.data_ptr(), H.dtype_tag(out), batch, N, int(iters),
                                   float(eps), H.stream(dev))
    H.check(rc, "mhc_sinkhorn_bwd")
    return out
