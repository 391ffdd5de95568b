"""The fp32-stream pre kernel (pre_split_kernel: bf16 MFMA on hi / lo splits of
x and phi, 8-token tiles) against the fp32 VALU kernel (the same entry point
without a phi image) and against the CPU oracle, at the BASELINE fp32 bar
(1e-5 max-norm relative, model/mhc_fused.py:871-876).

This is the layout of the reference's trainers (fp32 model under bf16
autocast, trainer/train_pretrain.py:129-130): fp32 x, phi and gate
parameters.  Shapes: n in {1, 2, 4}, the three projection modes, C a multiple
of 256 and not (640, 200), C = 1024 (phi tiles from LDS and L2), batches with a
ragged last tile, fewer tiles than CUs and several tiles per CU, Sinkhorn 0 /
1 / 20 iterations, repeated launches."""
from __future__ import annotations

import pytest
import torch

from oracle import mhc_ref as R
from tests._util import make_params, maxrel

pytestmark = pytest.mark.gpu

from model import _hip as H  # noqa: E402
from model import _ops  # noqa: E402

F32 = torch.float32
BAR = 1e-5
_MODE = {"full": H.MODE_FULL, "nohres": H.MODE_NOHRES, "head": H.MODE_HEAD}


def _run(kind, xd, pd, packed, n, C, iters=20):
    if kind == "full":
        o = _ops.pre_full(xd, pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"],
                          pd["alpha_post"], pd["bias_post"], pd["alpha_res"], pd["bias_res"], n, C,
                          2.0, 1e-6, 1e-6, iters, 1e-6, want_h_pre=True, want_raw=True,
                          want_saved=True)
    elif kind == "nohres":
        o = _ops.pre_nohres(xd, pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"],
                            pd["alpha_post"], pd["bias_post"], n, C, 2.0, 1e-6, 1e-6,
                            want_h_pre=True, want_saved=True)
    else:
        out, inv, mix = _ops.head(xd, pd["phi_weight"], packed, pd["alpha"], pd["bias"], n, C,
                                  1e-6, 1e-6, want_saved=True)
        o = {"sub_in": out, "inv_rms": inv, "mixes_raw": mix}
    torch.cuda.synchronize()
    return {k: v.clone() for k, v in o.items() if v is not None}


def _case(kind, n, C, M, seed):
    g = torch.Generator().manual_seed(seed)
    p = make_params(kind, n, C, F32, g, stress=True)
    x = torch.randn(1, M, n * C, generator=g) * 2.0
    dev = torch.device("cuda:0")
    pd = {k: v.to(dev) for k, v in p.items()}
    packed = _ops.PhiPack(_MODE[kind]).get(pd["phi_weight"], n, C)
    assert packed is not None and packed.numel() == H.load().mhc_phi_split_bytes(n, C, _MODE[kind])
    return x, p, pd, packed, dev


@pytest.mark.parametrize("kind", ["full", "nohres", "head"])
@pytest.mark.parametrize("n,C", [(4, 768), (2, 768), (1, 768), (4, 256), (4, 1024), (2, 512),
                                 (4, 640), (2, 200), (1, 1024)])
@pytest.mark.parametrize("M", [1, 9, 4096 + 5])
def test_split_matches_fp32_valu_kernel(kind, n, C, M):
    if kind == "head" and n == 1:
        pytest.skip("MHCHead with n = 1 is an RMSNorm (no projection)")
    x, p, pd, packed, dev = _case(kind, n, C, M, seed=1000 * n + C + M)
    print(f"split {kind} n={n} C={C} M={M}", flush=True)
    xd = x.to(dev)
    got = _run(kind, xd, pd, packed, n, C)
    ref = _run(kind, xd, pd, None, n, C)
    assert got.keys() == ref.keys()
    for k in ref:
        assert maxrel(ref[k], got[k]) <= BAR, (k, maxrel(ref[k], got[k]))


@pytest.mark.parametrize("n,C", [(4, 768), (2, 512), (1, 256)])
def test_split_vs_oracle(n, C):
    M = 8 * 256 * 3 + 5  # several tiles per CU and a ragged last tile
    x, p, pd, packed, dev = _case("full", n, C, M, seed=3 + n)
    o = _run("full", x.to(dev), pd, packed, n, C)
    idx = torch.tensor([0, 1, 7, 8, 9, M // 2, M - 6, M - 1])
    sub, h_pre, h_post, h_raw, inv, mixes = R.pre_full(x[:, idx], p, n, C)
    h_res = R.sinkhorn(h_raw.float(), 20, 1e-6)
    d = idx.to(dev)
    for ref, key, shape in ((sub, "sub_in", (M, C)), (h_pre, "h_pre", (M, n)),
                            (h_post, "h_post", (M, n)), (h_raw, "h_res_raw", (M, n * n)),
                            (h_res, "h_res", (M, n * n)), (inv, "inv_rms", (M,)),
                            (mixes, "mixes_raw", (M, 2 * n + n * n))):
        got = o[key].reshape(shape)[d].cpu()
        assert maxrel(ref[0].reshape(got.shape), got) <= BAR, key


# fp32 on the K-streamed kernel (hi / lo operands of x_norm and of phi, three
# MFMA products): n = 8 at any C, n in {2, 4} past C = 1024; one tile, many
# tiles per CU, ragged tiles, C not a multiple of 32 (200)
KS32 = [(8, 768), (8, 512), (8, 200), (4, 2048), (2, 1536)]


@pytest.mark.parametrize("kind", ["full", "nohres", "head"])
@pytest.mark.parametrize("n,C", KS32)
@pytest.mark.parametrize("M", [1, 33, 8192 + 7])
def test_ks32_matches_fp32_valu_kernel(kind, n, C, M):
    if M > 4096 and C > 768:
        M = 3000  # the VALU reference takes one workgroup per token
    x, p, pd, packed, dev = _case(kind, n, C, M, seed=77 * n + C + M)
    print(f"ks32 {kind} n={n} C={C} M={M}", flush=True)
    xd = x.to(dev)
    got = _run(kind, xd, pd, packed, n, C)
    ref = _run(kind, xd, pd, None, n, C)
    assert got.keys() == ref.keys()
    for k in ref:
        assert maxrel(ref[k], got[k]) <= BAR, (k, maxrel(ref[k], got[k]))


@pytest.mark.parametrize("n,C", [(8, 768), (4, 2048)])
def test_ks32_vs_oracle(n, C):
    M = 32 * 256 + 11
    x, p, pd, packed, dev = _case("full", n, C, M, seed=5 + n)
    o = _run("full", x.to(dev), pd, packed, n, C)
    idx = torch.tensor([0, 1, 31, 32, 33, M // 2, M - 12, M - 1])
    sub, h_pre, h_post, h_raw, inv, mixes = R.pre_full(x[:, idx], p, n, C)
    h_res = R.sinkhorn(h_raw.float(), 20, 1e-6)
    d = idx.to(dev)
    for ref, key, shape in ((sub, "sub_in", (M, C)), (h_pre, "h_pre", (M, n)),
                            (h_post, "h_post", (M, n)), (h_raw, "h_res_raw", (M, n * n)),
                            (h_res, "h_res", (M, n * n)), (inv, "inv_rms", (M,)),
                            (mixes, "mixes_raw", (M, 2 * n + n * n))):
        got = o[key].reshape(shape)[d].cpu()
        assert maxrel(ref[0].reshape(got.shape), got) <= BAR, key


def test_ks32_norm_second_launch():
    """The fused-norm entry point at fp32 n = 8: the K-streamed launch and an
    in-place RMSNorm launch, against the plain launch normed by torch."""
    n, C, M = 8, 768, 100
    x, p, pd, packed, dev = _case("full", n, C, M, seed=9)
    xd = x.to(dev)
    w = (1 + 0.1 * torch.randn(C, generator=torch.Generator().manual_seed(1))).to(dev)
    args = (pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"], pd["alpha_post"],
            pd["bias_post"], pd["alpha_res"], pd["bias_res"], n, C, 2.0, 1e-6, 1e-6, 20, 1e-6)
    plain = _ops.pre_full(xd, *args)
    normed = _ops.pre_full(xd, *args, norm=(w, 1e-6))
    ref = torch.nn.functional.rms_norm(plain["sub_in"], (C,), w, 1e-6)
    assert maxrel(ref, normed["sub_in"]) <= 2e-6
    assert torch.equal(plain["h_res"], normed["h_res"])


@pytest.mark.parametrize("iters", [0, 1, 20])
def test_split_sinkhorn_iterations(iters):
    n, C, M = 4, 768, 300
    x, p, pd, packed, dev = _case("full", n, C, M, seed=iters)
    xd = x.to(dev)
    got = _run("full", xd, pd, packed, n, C, iters)
    ref = _run("full", xd, pd, None, n, C, iters)
    assert maxrel(ref["h_res"], got["h_res"]) <= BAR


def test_split_repeat_launches():
    """Many workgroups, repeated launches: bit-identical every time."""
    n, C, M = 4, 768, 8 * 256 * 4 + 3
    x, p, pd, packed, dev = _case("full", n, C, M, seed=11)
    xd = x.to(dev)
    first = _run("full", xd, pd, packed, n, C)
    for _ in range(4):
        again = _run("full", xd, pd, packed, n, C)
        for k in first:
            assert torch.equal(first[k], again[k]), k


# ---------------------------------------------------------------- backward

def _misaligned(t: torch.Tensor) -> torch.Tensor:
    """The same values at an address 4 bytes past a 16-byte boundary: the MFMA
    backward kernels need 16-byte aligned rows, so this copy takes the fp32
    VALU kernels (the comparison's reference)."""
    buf = torch.empty(t.numel() + 1, dtype=t.dtype, device=t.device)
    v = buf[1:].view(t.shape)
    v.copy_(t)
    return v


def _alpha_err(ref, got, g_raw, mixes, lo, hi):
    terms = (g_raw[:, lo:hi].float() * mixes[:, lo:hi].float()).abs().sum().item()
    return abs(ref.float().item() - got.float().item()) / max(abs(ref.float().item()), terms, 1e-30)


@pytest.mark.parametrize("kind", ["full", "nohres"])
@pytest.mark.parametrize("n,C,M", [(4, 768, 37), (4, 768, 1100), (2, 768, 300), (4, 256, 64),
                                   (4, 1024, 50), (2, 200, 33), (4, 640, 17)])
def test_split_backward_matches_fp32_valu_kernels(kind, n, C, M):
    """pre_bwd (g_x, g_raw) and pre_bwd_weights (g_phi, g_alpha, g_bias) of
    fp32 x / phi / gradients on MFMA against the fp32 VALU kernels."""
    x, p, pd, packed, dev = _case(kind, n, C, M, seed=77 * n + C + M)
    xd = x.to(dev).view(M, n * C)
    o = _run(kind, x.to(dev), pd, packed, n, C)
    inv, mixes = o["inv_rms"], o["mixes_raw"]
    g = torch.Generator().manual_seed(M)
    gsub = torch.randn(M, C, generator=g).to(dev)
    ghp = torch.randn(M, n, generator=g).to(dev)
    ghpost = torch.randn(M, n, generator=g).to(dev)
    ghres = torch.randn(M, n * n, generator=g).to(dev) if kind == "full" else None
    if kind == "full":
        alphas = (pd["alpha_pre"], pd["alpha_post"], pd["alpha_res"])
        biases = (pd["bias_pre"], pd["bias_post"], pd["bias_res"])
        mode = H.MODE_FULL
    else:
        alphas = (pd["alpha_pre"], pd["alpha_post"], None)
        biases = (pd["bias_pre"], pd["bias_post"], None)
        mode = H.MODE_NOHRES
    print(f"split bwd {kind} n={n} C={C} M={M}", flush=True)
    res = []
    for xin in (xd, _misaligned(xd)):
        g_x, g_raw = _ops.pre_bwd(xin, pd["phi_weight"], alphas, biases, inv, mixes, n, C, mode,
                                  2.0, 1e-6, gsub, ghp, ghpost, ghres)
        g_w, g_a, g_b = _ops.pre_bwd_weights(xin, inv, mixes, g_raw, pd["phi_weight"], alphas, n,
                                             C, mode)
        torch.cuda.synchronize()
        res.append((g_x.clone(), g_raw.clone(), g_w.clone(), g_a, g_b))
    (gx, graw, gw, ga, gb), (rx, rraw, rw, ra, rb) = res
    assert maxrel(rx, gx) <= BAR
    assert maxrel(rraw, graw) <= BAR
    assert maxrel(rw, gw) <= BAR
    fd = 2 * n + (n * n if kind == "full" else 0)
    bounds = ((0, n), (n, 2 * n), (2 * n, fd))
    for i in range(3 if kind == "full" else 2):
        assert _alpha_err(ra[i], ga[i], rraw, mixes, *bounds[i]) <= BAR, i
        assert maxrel(rb[i], gb[i]) <= BAR, i


def test_module_fp32_autocast_layout_training_step_matches_oracle():
    """MHCConnection_Fused in the reference trainers' layout: fp32 parameters
    and stream, F returning bf16 (autocast).  Forward and backward run the
    fp32 MFMA kernels; gradients of x, phi and the gate parameters against
    autograd of the fp32 oracle with the same bf16 F."""
    from model.mhc_fused import MHCConnection_Fused
    dev = torch.device("cuda:0")
    n, C, M = 4, 768, 96
    g = torch.Generator().manual_seed(23)
    x = torch.randn(1, M, n * C, generator=g)
    p = make_params("full", n, C, F32, g)
    fw = (torch.randn(C, C, generator=g) * 0.03).to(torch.bfloat16)
    gout = torch.randn(1, M, n * C, generator=g)

    def f_ref(s):  # bf16 matmul of the bf16-cast input, as autocast runs F
        return (s.to(torch.bfloat16).float() @ fw.float().t()).to(torch.bfloat16).float()

    xr = x.clone().requires_grad_(True)
    pr = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    ref = R.mhc_full_forward(xr, pr, f_ref, n, C, sinkhorn_iters=20)["out"]
    (ref * gout).sum().backward()

    mod = MHCConnection_Fused(n, C, sinkhorn_iters=20).to(dev)
    with torch.no_grad():
        for k, v in p.items():
            getattr(mod, k).copy_(v)
    fwd_t = fw.t().contiguous().to(dev)
    xd = x.to(dev).requires_grad_(True)
    out = mod(xd, lambda s: s.to(torch.bfloat16) @ fwd_t)
    assert out.dtype == F32
    (out * gout.to(dev)).sum().backward()
    # F's bf16 output and input cast bound the agreement to bf16 rounding of F.
    assert maxrel(ref, out) <= 1e-2
    assert maxrel(xr.grad, xd.grad) <= 1e-2
    assert maxrel(pr["phi_weight"].grad, mod.phi_weight.grad) <= 1e-2
    for k in ("bias_pre", "bias_post", "bias_res"):
        assert maxrel(pr[k].grad, getattr(mod, k).grad) <= 1e-2, k
