"""The reference's autograd Functions called directly, the phi-pack cache
policy, and gradient flow into F when the mHC modules are frozen.

_PrePhaseFullFn.apply(x, W, a_pre, b_pre, a_post, b_post, a_res, b_res,
post_mult, pre_eps, rms_eps, n, c) -> (sublayer_in, h_pre, h_post, h_res_raw)
is the internal op boundary of the reference (model/mhc_fused.py:571-717);
reference-style code that calls it (with sinkhorn_normalize and
_PostPhaseFullFn, as MHCConnection_Fused.forward does at
model/mhc_fused.py:820-832) must land on the MFMA kernels.
"""
from __future__ import annotations

import pickle

import pytest
import torch
import torch.nn as nn

from oracle import mhc_ref as R
from tests._util import make_params, maxabs, maxrel, tol

pytestmark = pytest.mark.gpu

from model import _hip as H  # noqa: E402
from model import _ops  # noqa: E402
from model.mhc_common import MHCHead, _MHCHeadFn  # noqa: E402
from model.mhc_fused import (MHCConnection_Fused, _PostPhaseFullFn,  # noqa: E402
                             _PrePhaseFullFn, sinkhorn_normalize)
from model.mhc_fused_no_hres import MHCConnection_FusedNoHres, _PrePhaseFn  # noqa: E402

ARGS = ("alpha_pre", "bias_pre", "alpha_post", "bias_post", "alpha_res", "bias_res")


def _case(n, C, M, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(2, M // 2, n * C, generator=g).to(dtype)
    p = make_params("full", n, C, dtype, g)
    return x, p


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,C,M", [(4, 768, 256), (8, 768, 64), (2, 256, 34)])
def test_pre_phase_full_fn_forward(dev, dtype, n, C, M):
    x, p = _case(n, C, M, dtype, 5 + n)
    pd = {k: v.to(dev) for k, v in p.items()}
    xd = x.to(dev)
    print(f"_PrePhaseFullFn fwd n={n} C={C} M={M} {dtype}", flush=True)
    with torch.no_grad():
        sub, h_pre, h_post, h_raw = _PrePhaseFullFn.apply(
            xd, pd["phi_weight"], *[pd[k] for k in ARGS], 2.0, 1e-6, 1e-6, n, C)
    packed = _ops.PhiPack(H.MODE_FULL).get(pd["phi_weight"], n, C)
    # MFMA images: bf16 phi (any n), fp32 phi for n in {1, 2, 4} (the split
    # kernel) and n = 8 (the K-streamed kernel on hi / lo images)
    assert (packed is not None) == (dtype == torch.bfloat16 or n in (1, 2, 4, 8))
    o = _ops.pre_full(xd, pd["phi_weight"], packed, *[pd[k] for k in ARGS], n, C, 2.0, 1e-6,
                      1e-6, 0, 0.0, sinkhorn=False, want_h_pre=True, want_raw=True)
    # the same launch the modules make: bit for bit
    assert torch.equal(sub.reshape(M, C), o["sub_in"])
    assert torch.equal(h_pre.reshape(M, n), o["h_pre"])
    assert torch.equal(h_post.reshape(M, n), o["h_post"])
    assert torch.equal(h_raw.reshape(M, n, n), o["h_res_raw"])
    r_sub, r_pre, r_post, r_raw, _, _ = R.pre_full(x, p, n, C)
    bar = tol(dtype)
    assert maxrel(r_sub, sub) <= bar
    assert maxrel(r_pre, h_pre) <= bar
    assert maxrel(r_post, h_post) <= bar
    # h_res_raw = alpha_res * m + bias_res: the kernels round x_norm to bf16 as
    # the oracle does (model/mhc_fused.py:845) but keep m in fp32 where the
    # oracle rounds it to bf16 (:546); one bf16 step of the largest entry is 2**-8.
    assert maxrel(r_raw, h_raw) <= (8e-3 if dtype == torch.bfloat16 else 1e-5)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_pre_phase_full_fn_reference_composition_backward(dev, dtype):
    """The reference's fused forward spelled with its own Functions
    (model/mhc_fused.py:820-832), forward and backward, against autograd of the
    fp32 oracle on the same (exactly upcast) inputs."""
    n, C, M = 4, 768, 96
    x, p = _case(n, C, M, dtype, 11)
    g = torch.Generator().manual_seed(12)
    fw = (torch.randn(C, C, generator=g) * 0.03).to(dtype)
    gout = torch.randn(2, M // 2, n * C, generator=g).to(dtype)

    xr = x.float().clone().requires_grad_(True)
    pr = {k: v.float().clone().requires_grad_(True) for k, v in p.items()}
    ref = R.mhc_full_forward(xr, pr, lambda s: s @ fw.float().t(), n, C, sinkhorn_iters=20)["out"]
    (ref * gout.float()).sum().backward()

    xd = x.to(dev).requires_grad_(True)
    pd = {k: v.to(dev).requires_grad_(True) for k, v in p.items()}
    fwd_t = fw.t().contiguous().to(dev)
    sub, _h_pre, h_post, h_raw = _PrePhaseFullFn.apply(
        xd, pd["phi_weight"], *[pd[k] for k in ARGS], 2.0, 1e-6, 1e-6, n, C)
    h_res = sinkhorn_normalize(h_raw, iters=20, eps=1e-6).to(xd.dtype)
    out = _PostPhaseFullFn.apply(xd, h_res, h_post, sub @ fwd_t, n, C)
    (out.float() * gout.to(dev).float()).sum().backward()
    bar = 2e-2 if dtype == torch.bfloat16 else 1e-4
    assert maxrel(ref, out) <= (1e-2 if dtype == torch.bfloat16 else 1e-5)
    assert maxrel(xr.grad, xd.grad) <= bar
    assert maxrel(pr["phi_weight"].grad, pd["phi_weight"].grad) <= bar
    for k in ("bias_pre", "bias_post", "bias_res"):
        assert maxrel(pr[k].grad, pd[k].grad) <= bar, k


def test_nohres_and_head_functions_pack_phi(dev):
    """_PrePhaseFn / _MHCHeadFn called without a pack run the MFMA kernels:
    bit-identical to the modules' launches."""
    n, C, M = 4, 768, 64
    g = torch.Generator().manual_seed(2)
    x = torch.randn(1, M, n * C, generator=g).to(torch.bfloat16).to(dev)
    mod = MHCConnection_FusedNoHres(n, C).to(dev).to(torch.bfloat16)
    args = (mod.alpha_pre, mod.bias_pre, mod.alpha_post, mod.bias_post)
    with torch.no_grad():
        got = _PrePhaseFn.apply(x, mod.phi_weight, *args, 2.0, 1e-6, 1e-6, n, C)
        packed = mod._phi_pack.get(mod.phi_weight, n, C)
        assert packed is not None
        o = _ops.pre_nohres(x, mod.phi_weight, packed, *args, n, C, 2.0, 1e-6, 1e-6,
                            want_h_pre=True)
    assert torch.equal(got[0].reshape(M, C), o["sub_in"])
    assert torch.equal(got[2].reshape(M, n), o["h_post"])
    head = MHCHead(n, C).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        got = _MHCHeadFn.apply(x, head.phi_weight, head.alpha, head.bias, 1e-6, 1e-6, n, C)
        assert torch.equal(got, head(x))


def _fresh_out(mod, x, f):
    ref = MHCConnection_Fused(mod.n, mod.dim, sinkhorn_iters=mod.sinkhorn_iters)
    ref = ref.to(x.device).to(x.dtype)
    ref.load_state_dict(mod.state_dict())
    with torch.no_grad():
        return ref(x, f)


def test_phi_pack_follows_weight_updates(dev):
    """The cached MFMA image tracks optimizer steps and load_state_dict; a write
    through .data needs invalidate() in inference and is seen in training."""
    n, C, M = 4, 768, 64
    g = torch.Generator().manual_seed(8)
    x = torch.randn(1, M, n * C, generator=g).to(torch.bfloat16).to(dev)
    fw = (torch.randn(C, C, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    f = lambda z: z @ fw  # noqa: E731
    mod = MHCConnection_Fused(n, C, sinkhorn_iters=20).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        mod.alpha_pre.fill_(0.7)
        mod.alpha_post.fill_(0.7)
        mod.alpha_res.fill_(0.7)
        out0 = mod(x, f)                         # caches the image
    opt = torch.optim.SGD(mod.parameters(), lr=5.0)
    loss = mod(x.clone().requires_grad_(True), f).float().pow(2).mean()
    loss.backward()
    opt.step()
    with torch.no_grad():
        out1 = mod(x, f)
    assert not torch.equal(out0, out1)
    assert torch.equal(out1, _fresh_out(mod, x, f))

    other = MHCConnection_Fused(n, C, sinkhorn_iters=20).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        other.alpha_pre.fill_(0.5)
    mod.load_state_dict(other.state_dict())
    with torch.no_grad():
        assert torch.equal(mod(x, f), _fresh_out(mod, x, f))

    mod.phi_weight.data.normal_(0.0, 0.05)       # invisible to the version counter
    mod._phi_pack.invalidate()
    with torch.no_grad():
        assert torch.equal(mod(x, f), _fresh_out(mod, x, f))
    mod.phi_weight.data.normal_(0.0, 0.05)
    out_train = mod(x, f)                        # grad mode on: repacked every call
    assert torch.equal(out_train.detach(), _fresh_out(mod, x, f))


def test_module_pickles_after_forward(dev):
    mod = MHCConnection_Fused(4, 256).to(dev).to(torch.bfloat16)
    x = torch.randn(1, 16, 1024, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        out = mod(x, lambda z: z)
    assert mod._phi_pack._buf is not None
    copy = pickle.loads(pickle.dumps(mod))
    assert copy._phi_pack._buf is None
    with torch.no_grad():
        assert torch.equal(copy(x, lambda z: z), out)


@pytest.mark.parametrize("kind", ["full", "nohres"])
def test_frozen_connection_trainable_sublayer_gets_gradients(dev, kind):
    """in_norm hand-off with the connection and norms frozen and only F
    trainable: F's weight gradient equals autograd of the oracle."""
    n, C, M = 4, 64, 24
    g = torch.Generator().manual_seed(15)
    x = torch.randn(1, M, n * C, generator=g)
    p = make_params(kind, n, C, torch.float32, g)
    lin = nn.Linear(C, C, bias=False)
    norm = nn.RMSNorm(C, eps=1e-6)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(C, C, generator=g) * 0.1)
        norm.weight.copy_(1 + 0.1 * torch.randn(C, generator=g))
    gout = torch.randn(1, M, n * C, generator=g)

    lr = nn.Linear(C, C, bias=False)
    lr.load_state_dict(lin.state_dict())
    nr = nn.RMSNorm(C, eps=1e-6)
    nr.load_state_dict(norm.state_dict())
    fwd = R.mhc_full_forward if kind == "full" else R.mhc_nohres_forward
    kw = dict(sinkhorn_iters=20) if kind == "full" else {}
    ref = fwd(x, p, lambda z: lr(nr(z)), n, C, **kw)["out"]
    (ref * gout).sum().backward()

    mod = (MHCConnection_Fused(n, C, sinkhorn_iters=20) if kind == "full"
           else MHCConnection_FusedNoHres(n, C)).to(dev)
    with torch.no_grad():
        for k, v in p.items():
            getattr(mod, k).copy_(v)
    mod.requires_grad_(False)
    nd = nn.RMSNorm(C, eps=1e-6).to(dev)
    nd.load_state_dict(norm.state_dict())
    nd.requires_grad_(False)
    ld = nn.Linear(C, C, bias=False).to(dev)
    ld.load_state_dict(lin.state_dict())
    out = mod(x.to(dev), ld, nd)
    (out * gout.to(dev)).sum().backward()
    assert ld.weight.grad is not None
    assert maxrel(lr.weight.grad, ld.weight.grad) <= 1e-4
    assert maxabs(ref, out) <= 1e-5 * ref.abs().max().item()


def test_sinkhorn_iterations_beyond_backward_limit(dev):
    """A Sinkhorn count the backward kernel cannot take fails at the forward that
    would need it (a clear error instead of one at backward), and runs in
    inference."""
    n, C, M = 4, 64, 8
    cap = H.load().mhc_sinkhorn_bwd_max_iters(n)
    mod = MHCConnection_Fused(n, C, sinkhorn_iters=cap + 1).to(dev)
    x = torch.randn(1, M, n * C, device=dev)
    with torch.no_grad():
        out = mod(x, lambda z: z)
    assert torch.isfinite(out).all()
    with pytest.raises(ValueError, match="sinkhorn_iters"):
        mod(x, lambda z: z)
    m = torch.randn(3, n, n, device=dev, requires_grad=True)
    with pytest.raises(ValueError, match="sinkhorn_iters"):
        sinkhorn_normalize(m, cap + 1)
    ok = MHCConnection_Fused(n, C, sinkhorn_iters=cap).to(dev)
    ok(x, lambda z: z).sum().backward()
    assert ok.phi_weight.grad is not None
