"""GPU parity of the backward kernels, through the C ABI, against autograd of
the CPU oracle.

The reference's backward kernels recompute in fp32 from the saved inv_rms /
mixes_raw (model/mhc_fused.py:271-413, :462-526, :644-717) and its Sinkhorn
backward is autograd of the fp32 recompute (model/mhc_fused.py:131-137), so
the truth here is autograd of the fp32 oracle at the same inputs (bf16 inputs
upcast exactly).  Bars: max|ref-got|/max|ref| <= 1e-4 for fp32 inputs, 1e-2
for bf16 (each gradient is stored once in bf16).
"""
from __future__ import annotations

import pytest
import torch

from oracle import mhc_ref as R
from tests._util import make_params, maxrel

pytestmark = pytest.mark.gpu

from model import _hip as H  # noqa: E402
from model import _ops  # noqa: E402


def _bar(dtype):
    return 1e-4 if dtype == torch.float32 else 1e-2


def _leaf(t):
    return t.detach().float().clone().requires_grad_(True)


def _alpha_err(ref, got, g_raw, mixes, lo, hi):
    """Error of a gate-alpha gradient, sum_t sum_f g_raw[t, f] * mixes[t, f] over
    the segment's features [lo, hi), relative to the sum of the terms'
    magnitudes: the sum can cancel to far below its terms, and then the
    last-ulp differences in mixes (a different fp32 summation order) dominate
    a plain relative error."""
    terms = (g_raw[:, lo:hi].float() * mixes[:, lo:hi].float()).abs().sum().item()
    return abs(ref.item() - got.float().item()) / max(abs(ref.item()), terms, 1e-30)


# ------------------------------------------------------------------ post phase

@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,C", [(1, 64), (2, 96), (4, 768), (4, 100), (8, 768), (16, 32)])
@pytest.mark.parametrize("res", [True, False])
def test_post_bwd_vs_oracle(dev, dtype, n, C, res):
    M = 37
    g = torch.Generator().manual_seed(100 + n + C)
    x = torch.randn(1, M, n * C, generator=g).to(dtype)
    h_res = torch.rand(1, M, n, n, generator=g).to(dtype)
    h_post = (torch.rand(1, M, n, generator=g) * 2).to(dtype)
    f = torch.randn(1, M, C, generator=g).to(dtype)
    gout = torch.randn(1, M, n * C, generator=g).to(dtype)
    xr, hr, hp, fr = _leaf(x), _leaf(h_res), _leaf(h_post), _leaf(f)
    ref = R.post_full(xr, hr, hp, fr, n, C) if res else \
        (xr.view(1, M, n, C) + hp.unsqueeze(-1) * fr.unsqueeze(-2)).reshape(1, M, n * C)
    (ref * gout.float()).sum().backward()
    g_x, g_hr, g_hp, g_f = _ops.post_bwd(x.to(dev), h_res.to(dev) if res else None,
                                         h_post.to(dev), f.to(dev), n, C, gout.to(dev))
    torch.cuda.synchronize()
    bar = _bar(dtype)
    assert g_x.dtype == dtype and g_f.dtype == dtype and g_hp.dtype == dtype
    assert maxrel(xr.grad.view(M, n * C), g_x) <= bar
    assert maxrel(hp.grad.view(M, n), g_hp) <= bar
    assert maxrel(fr.grad.view(M, C), g_f) <= bar
    if res:
        assert maxrel(hr.grad.view(M, n, n), g_hr) <= bar


def test_post_bwd_empty_and_errors(dev):
    n, C = 4, 64
    z = torch.empty(0, n * C, device=dev)
    g_x, g_hr, g_hp, g_f = _ops.post_bwd(z, torch.empty(0, n, n, device=dev),
                                         torch.empty(0, n, device=dev), torch.empty(0, C, device=dev),
                                         n, C, z)
    assert g_x.shape == (0, n * C) and g_f.shape == (0, C)
    lib = H.load()
    rc = lib.mhc_post_bwd(None, 0, None, None, 0, None, 0, None, None, None, None, None, 5, n, C,
                          H.stream(dev))
    assert rc != 0 and b"null pointer" in lib.mhc_last_error()


# ------------------------------------------------------------------- Sinkhorn

@pytest.mark.parametrize("n", [1, 2, 3, 4, 8, 16])
@pytest.mark.parametrize("iters", [0, 1, 2, 10, 20])
def test_sinkhorn_bwd_vs_autograd(dev, n, iters):
    batch = 70
    g = torch.Generator().manual_seed(7 * n + iters)
    m = torch.randn(batch, n, n, generator=g) * 1.5
    gy = torch.randn(batch, n, n, generator=g)
    mr = m.double().requires_grad_(True)
    R.sinkhorn(mr, iters, 1e-6).backward(gy.double())
    got = _ops.sinkhorn_bwd(m.to(dev), gy.to(dev), iters, 1e-6)
    torch.cuda.synchronize()
    assert got.dtype == torch.float32
    assert maxrel(mr.grad.float(), got) <= 1e-4


# (4, 64), (8, 40): the per-lane trajectory kernel at its longest; the rest
# take the checkpointed workgroup kernel (segments recomputed from every K-th
# iterate), up to the 256-iteration cap, n = 16 included.
@pytest.mark.parametrize("n,iters", [(4, 64), (8, 40), (3, 30), (16, 31), (16, 100), (4, 65),
                                     (2, 130), (8, 256), (1, 50), (5, 7)])
def test_sinkhorn_bwd_long_schedules(dev, n, iters):
    g = torch.Generator().manual_seed(n + iters)
    m = torch.randn(33, n, n, generator=g)
    gy = torch.randn(33, n, n, generator=g)
    mr = m.double().requires_grad_(True)
    R.sinkhorn(mr, iters, 1e-6).backward(gy.double())
    got = _ops.sinkhorn_bwd(m.to(dev), gy.to(dev), iters, 1e-6)
    assert maxrel(mr.grad.float(), got) <= 1e-4


def test_sinkhorn_bwd_iteration_limit(dev):
    cap = H.load().mhc_sinkhorn_bwd_max_iters(3)
    assert cap == 256
    with pytest.raises(RuntimeError, match="iters must be"):
        _ops.sinkhorn_bwd(torch.zeros(2, 3, 3, device=dev), torch.zeros(2, 3, 3, device=dev),
                          cap + 1, 1e-6)


# The 10- and 20-iteration kernels (2 x 2 blocks a lane) read both inputs
# through buffer descriptors, one load per tensor and row pair, whatever their
# dtypes; a base that is not 4-byte aligned (a 16-bit view starting one
# element into its buffer) takes the other kernels.  37 matrices: the last
# workgroup is part-filled.
@pytest.mark.parametrize("n", [2, 4, 8])
@pytest.mark.parametrize("in_dt,g_dt,out_dt", [
    (torch.bfloat16, torch.bfloat16, torch.bfloat16), (torch.float16, torch.float32, torch.float32),
    (torch.float32, torch.bfloat16, torch.float32), (torch.bfloat16, torch.float32, torch.float16)])
@pytest.mark.parametrize("offset", [0, 1])
@pytest.mark.parametrize("iters", [10, 20])
def test_sinkhorn_bwd_dtypes_and_offsets(dev, n, in_dt, g_dt, out_dt, offset, iters):
    batch = 37
    g = torch.Generator().manual_seed(100 * n + 10 * offset + int(in_dt == torch.float32) + iters)
    m = (torch.randn(batch, n, n, generator=g) * 1.5).to(in_dt)
    gy = torch.randn(batch, n, n, generator=g).to(g_dt)

    def place(t):  # t on the device, `offset` elements into a larger buffer
        buf = torch.zeros(t.numel() + offset, dtype=t.dtype, device=dev)
        v = buf[offset:].view(t.shape)
        v.copy_(t.to(dev))
        return v

    print(f"sinkhorn_bwd n={n} iters={iters} {in_dt} {g_dt} -> {out_dt} offset={offset}", flush=True)
    got = _ops.sinkhorn_bwd(place(m), place(gy), iters, 1e-6, out_dtype=out_dt)
    torch.cuda.synchronize()
    mr = m.double().requires_grad_(True)
    R.sinkhorn(mr, iters, 1e-6).backward(gy.double())
    assert got.dtype == out_dt
    bar = {torch.float32: 1e-4, torch.float16: 2e-3, torch.bfloat16: 1e-2}[out_dt]
    assert maxrel(mr.grad.float(), got.float()) <= bar


def test_sinkhorn_bwd_bf16_io(dev):
    g = torch.Generator().manual_seed(3)
    m = (torch.randn(300, 4, 4, generator=g) * 2).to(torch.bfloat16)
    gy = torch.randn(300, 4, 4, generator=g).to(torch.bfloat16)
    mr = m.double().requires_grad_(True)
    R.sinkhorn(mr, 20, 1e-6).backward(gy.double())
    got = _ops.sinkhorn_bwd(m.to(dev), gy.to(dev), 20, 1e-6)
    assert got.dtype == torch.bfloat16
    assert maxrel(mr.grad.float(), got) <= 1e-2


# ------------------------------------------------------------------ pre phase

def _pre_case(dev, kind, n, C, M, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, M, n * C, generator=g).to(dtype)
    p = make_params(kind, n, C, dtype, g)
    pd = {k: v.to(dev) for k, v in p.items()}
    if kind == "full":
        o = _ops.pre_full(x.to(dev), pd["phi_weight"], None, pd["alpha_pre"], pd["bias_pre"],
                          pd["alpha_post"], pd["bias_post"], pd["alpha_res"], pd["bias_res"], n, C,
                          2.0, 1e-6, 1e-6, 0, 0.0, sinkhorn=False, want_saved=True)
        inv, mixes = o["inv_rms"], o["mixes_raw"]
    elif kind == "nohres":
        o = _ops.pre_nohres(x.to(dev), pd["phi_weight"], None, pd["alpha_pre"], pd["bias_pre"],
                            pd["alpha_post"], pd["bias_post"], n, C, 2.0, 1e-6, 1e-6,
                            want_saved=True)
        inv, mixes = o["inv_rms"], o["mixes_raw"]
    else:
        _, inv, mixes = _ops.head(x.to(dev), pd.get("phi_weight"), None, pd.get("alpha"),
                                  pd.get("bias"), n, C, 1e-6, 1e-6, want_saved=True)
    return x, p, pd, inv, mixes, g


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
# n = 16: FD = 288 features, more than a 256-thread workgroup has threads;
# n = 8 fp32: the MFMA kernel with x streamed per chunk (C = 768, 1024);
# n = 8, C = 200: the weight kernel's 256-column slices with a partial last
# slice (n*C = 1600) and a ragged last token range; n = 6: FD = 48, three
# feature tiles (two column tiles a wave as well)
@pytest.mark.parametrize("n,C,M", [(4, 64, 24), (4, 768, 300), (2, 100, 17), (8, 768, 40),
                                   (1, 64, 9), (4, 256, 1100), (16, 64, 20), (16, 256, 300),
                                   (8, 1024, 70), (8, 200, 130), (6, 64, 77)])
def test_pre_full_bwd_vs_oracle(dev, dtype, n, C, M):
    """g_x, g_phi, alphas and biases of the full pre phase for given upstream
    gradients of (sublayer_in, h_pre, h_post, h_res_raw)."""
    x, p, pd, inv, mixes, g = _pre_case(dev, "full", n, C, M, dtype, 11 * n + C + M)
    ups = [torch.randn(1, M, C, generator=g), torch.randn(1, M, n, generator=g),
           torch.randn(1, M, n, generator=g), torch.randn(1, M, n, n, generator=g)]
    ups = [u.to(dtype) for u in ups]
    xr = _leaf(x)
    pr = {k: _leaf(v) for k, v in p.items()}
    outs = R.pre_full(xr, pr, n, C)[:4]
    sum((o * u.float()).sum() for o, u in zip(outs, ups)).backward()

    alphas = (pd["alpha_pre"], pd["alpha_post"], pd["alpha_res"])
    biases = (pd["bias_pre"], pd["bias_post"], pd["bias_res"])
    x2 = x.to(dev).view(M, n * C)
    g_x, g_raw = _ops.pre_bwd(x2, pd["phi_weight"], alphas, biases, inv, mixes, n, C, H.MODE_FULL,
                              2.0, 1e-6, *[u.to(dev) for u in ups])
    g_w, g_a, g_b = _ops.pre_bwd_weights(x2, inv, mixes, g_raw, pd["phi_weight"], alphas, n, C,
                                         H.MODE_FULL)
    torch.cuda.synchronize()
    bar = _bar(dtype)
    assert g_x.dtype == dtype and g_w.dtype == dtype
    assert maxrel(xr.grad.view(M, n * C), g_x) <= bar
    assert maxrel(pr["phi_weight"].grad, g_w) <= bar
    bounds = ((0, n), (n, 2 * n), (2 * n, 2 * n + n * n))
    for i, seg in enumerate(("pre", "post", "res")):
        assert _alpha_err(pr[f"alpha_{seg}"].grad, g_a[i], g_raw, mixes, *bounds[i]) <= bar, seg
        assert maxrel(pr[f"bias_{seg}"].grad.reshape(-1), g_b[i]) <= bar, seg


# n = 2: FD = 4 (one short phi operand on the MFMA kernel); n = 8 fp32: x
# streamed per chunk
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,C,M", [(4, 64, 24), (8, 768, 33), (2, 96, 700), (8, 512, 300)])
def test_pre_nohres_bwd_vs_oracle(dev, dtype, n, C, M):
    x, p, pd, inv, mixes, g = _pre_case(dev, "nohres", n, C, M, dtype, 5 * n + C + M)
    ups = [torch.randn(1, M, C, generator=g).to(dtype), None,
           torch.randn(1, M, n, generator=g).to(dtype)]
    xr = _leaf(x)
    pr = {k: _leaf(v) for k, v in p.items()}
    sub, _, h_post, _ = R.pre_nohres(xr, pr, n, C)[:4]
    ((sub * ups[0].float()).sum() + (h_post * ups[2].float()).sum()).backward()
    alphas = (pd["alpha_pre"], pd["alpha_post"], None)
    biases = (pd["bias_pre"], pd["bias_post"], None)
    x2 = x.to(dev).view(M, n * C)
    g_x, g_raw = _ops.pre_bwd(x2, pd["phi_weight"], alphas, biases, inv, mixes, n, C,
                              H.MODE_NOHRES, 2.0, 1e-6, ups[0].to(dev), None, ups[2].to(dev))
    g_w, g_a, g_b = _ops.pre_bwd_weights(x2, inv, mixes, g_raw, pd["phi_weight"], alphas, n, C,
                                         H.MODE_NOHRES)
    torch.cuda.synchronize()
    bar = _bar(dtype)
    assert maxrel(xr.grad.view(M, n * C), g_x) <= bar
    assert maxrel(pr["phi_weight"].grad, g_w) <= bar
    assert g_a[2] is None and g_b[2] is None
    for i, seg in enumerate(("pre", "post")):
        assert _alpha_err(pr[f"alpha_{seg}"].grad, g_a[i], g_raw, mixes, i * n, (i + 1) * n) <= bar, seg
        assert maxrel(pr[f"bias_{seg}"].grad, g_b[i]) <= bar, seg


# n = 4 / 2: FD = 4 / 2 (a short phi operand on the MFMA kernel)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("n,C,M", [(4, 64, 24), (1, 768, 50), (8, 768, 300), (4, 768, 300),
                                   (2, 256, 70), (4, 200, 33)])
def test_head_bwd_vs_oracle(dev, dtype, n, C, M):
    kind = "head"
    x, p, pd, inv, mixes, g = _pre_case(dev, kind, n, C, M, dtype, 3 * n + C + M)
    gout = torch.randn(1, M, C, generator=g).to(dtype)
    xr = _leaf(x)
    pr = {k: _leaf(v) for k, v in p.items()}
    (R.head(xr, pr, n, C).float() * gout.float()).sum().backward()
    x2 = x.to(dev).view(M, n * C)
    bar = _bar(dtype)
    if n == 1:
        g_x, g_raw = _ops.pre_bwd(x2, None, (None,) * 3, (None,) * 3, inv, None, 1, C, H.MODE_RMS,
                                  0.0, 0.0, g_sub=gout.to(dev))
        assert g_raw is None
        assert maxrel(xr.grad.view(M, C), g_x) <= bar
        return
    alphas, biases = (pd["alpha"], None, None), (pd["bias"], None, None)
    g_x, g_raw = _ops.pre_bwd(x2, pd["phi_weight"], alphas, biases, inv, mixes, n, C, H.MODE_HEAD,
                              0.0, 1e-6, g_sub=gout.to(dev))
    g_w, g_a, g_b = _ops.pre_bwd_weights(x2, inv, mixes, g_raw, pd["phi_weight"], alphas, n, C,
                                         H.MODE_HEAD)
    torch.cuda.synchronize()
    assert maxrel(xr.grad.view(M, n * C), g_x) <= bar
    assert maxrel(pr["phi_weight"].grad, g_w) <= bar
    assert _alpha_err(pr["alpha"].grad.reshape(()), g_a[0], g_raw, mixes, 0, n) <= bar
    assert maxrel(pr["bias"].grad, g_b[0]) <= bar


def test_pre_bwd_weights_workspace_checks(dev):
    lib = H.load()
    n, C, M = 4, 64, 10
    need = lib.mhc_pre_bwd_weights_workspace_bytes(M, n, C, H.MODE_FULL)
    assert need > 0
    t = torch.zeros(M, n * C, device=dev)
    f = torch.zeros(M, 24, device=dev)
    a = torch.zeros((), device=dev)
    w = torch.empty(n * C, 24, device=dev)
    ws = torch.empty(need - 4, dtype=torch.uint8, device=dev)
    rc = lib.mhc_pre_bwd_weights(t.data_ptr(), 0, f.data_ptr(), f.data_ptr(), f.data_ptr(),
                                 a.data_ptr(), a.data_ptr(), a.data_ptr(), 0, w.data_ptr(), 0,
                                 None, None, None, None, None, None, ws.data_ptr(), need - 4,
                                 M, n, C, H.MODE_FULL, H.stream(dev))
    assert rc != 0 and b"workspace" in lib.mhc_last_error()


def test_module_bf16_training_step_matches_oracle(dev):
    """End to end through autograd at the C2 shape family (bf16, n = 4, C = 768):
    gradients of x, phi and the gate parameters of MHCConnection_Fused."""
    from model.mhc_fused import MHCConnection_Fused
    n, C, M = 4, 768, 96
    g = torch.Generator().manual_seed(21)
    x = torch.randn(1, M, n * C, generator=g).to(torch.bfloat16)
    p = make_params("full", n, C, torch.bfloat16, g)
    fw = (torch.randn(C, C, generator=g) * 0.03).to(torch.bfloat16)
    gout = torch.randn(1, M, n * C, generator=g).to(torch.bfloat16)

    xr = _leaf(x)
    pr = {k: _leaf(v) for k, v in p.items()}
    d = R.mhc_full_forward(xr, pr, lambda s: s @ fw.float().t(), n, C, sinkhorn_iters=20)
    d["mixes"].retain_grad()
    (d["out"].float() * gout.float()).sum().backward()

    mod = MHCConnection_Fused(n, C, sinkhorn_iters=20).to(dev).to(torch.bfloat16)
    with torch.no_grad():
        for k, v in p.items():
            getattr(mod, k).copy_(v)
    xd = x.to(dev).requires_grad_(True)
    fwd_t = fw.t().contiguous().to(dev)  # a plain (non-transposed) right operand
    out = mod(xd, lambda s: s @ fwd_t)
    (out.float() * gout.to(dev).float()).sum().backward()
    assert maxrel(xr.grad, xd.grad) <= 2e-2
    assert maxrel(pr["phi_weight"].grad, mod.phi_weight.grad) <= 2e-2
    for k in ("bias_pre", "bias_post", "bias_res"):
        assert maxrel(pr[k].grad, getattr(mod, k).grad) <= 2e-2, k
    # alpha_seg's gradient is sum_t sum_f g_raw[t, f] * mixes[t, f] with
    # g_raw = d loss / d mixes / alpha_seg; it can cancel far below its terms,
    # so it is held to 2e-2 of the terms' magnitudes (the oracle's)
    mixes, g_mixes = d["mixes"].detach(), d["mixes"].grad
    for seg, (lo, hi) in (("pre", (0, n)), ("post", (n, 2 * n)), ("res", (2 * n, 2 * n + n * n))):
        ref_a = pr[f"alpha_{seg}"]
        terms = (g_mixes[..., lo:hi] / ref_a.detach() * mixes[..., lo:hi]).abs().sum().item()
        got = getattr(mod, f"alpha_{seg}").grad.float().item()
        err = abs(ref_a.grad.item() - got) / max(abs(ref_a.grad.item()), terms, 1e-30)
        assert err <= 2e-2, (seg, err)


@pytest.mark.parametrize("n,iters", [(16, 40), (4, 100), (16, 20)])
def test_module_training_long_sinkhorn_matches_oracle(dev, n, iters):
    """A training step with more Sinkhorn iterations than the per-lane backward
    kernels keep (n = 16 past 30, n = 4 past 64): the checkpointed backward,
    fp32, against autograd of the oracle."""
    from model.mhc_fused import MHCConnection_Fused
    C, M = 64, 24
    g = torch.Generator().manual_seed(40 + n)
    x = torch.randn(1, M, n * C, generator=g)
    p = make_params("full", n, C, torch.float32, g, stress=True)
    fw = torch.randn(C, C, generator=g) * 0.1
    gout = torch.randn(1, M, n * C, generator=g)
    xr = _leaf(x)
    pr = {k: _leaf(v) for k, v in p.items()}
    ref = R.mhc_full_forward(xr, pr, lambda s: s @ fw.t(), n, C, sinkhorn_iters=iters)["out"]
    (ref * gout).sum().backward()
    mod = MHCConnection_Fused(n, C, sinkhorn_iters=iters).to(dev)
    with torch.no_grad():
        for k, v in p.items():
            getattr(mod, k).copy_(v)
    xd = x.to(dev).requires_grad_(True)
    fwd_t = fw.t().contiguous().to(dev)
    out = mod(xd, lambda s: s @ fwd_t)
    (out * gout.to(dev)).sum().backward()
    assert maxrel(ref.detach(), out.detach().cpu()) <= 1e-5
    assert maxrel(xr.grad, xd.grad) <= 1e-4
    assert maxrel(pr["phi_weight"].grad, mod.phi_weight.grad) <= 1e-4
    assert maxrel(pr["bias_res"].grad, mod.bias_res.grad) <= 1e-4
