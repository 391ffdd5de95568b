"""Drop-in modules on the GPU against the reference's golden vectors and the oracle."""
from __future__ import annotations

import pytest
import torch
import torch.nn as nn

from oracle import mhc_ref as R
from tests._util import (golden_names, load_golden, make_params, maxabs, maxrel, seeded_names, t,
                         tol)

pytestmark = pytest.mark.gpu

from model.mhc_common import MHCHead, StreamExpand  # noqa: E402
from model.mhc_fused import MHCConnection_Fused, sinkhorn_normalize  # noqa: E402
from model.mhc_fused_no_hres import MHCConnection_FusedNoHres  # noqa: E402

DT = {"bf16": torch.bfloat16, "f32": torch.float32}


def _load_module(mod, p, dev, dtype):
    mod = mod.to(dtype)
    with torch.no_grad():
        for k, v in p.items():
            getattr(mod, k).copy_(v)
    return mod.to(dev)


@pytest.mark.parametrize("name", golden_names())
def test_module_matches_reference_golden(dev, name):
    """Reference _forward_ref outputs (tests/golden) reproduced by the HIP modules."""
    rec = load_golden(name)
    dtype = DT[str(rec["dtype"])]
    n, C = int(rec["n"]), int(rec["C"])
    x = t(rec["x"], dtype).to(dev)
    p = {k[2:]: t(v, dtype) for k, v in rec.items() if k.startswith("p_")}
    if name.startswith("full"):
        mod = _load_module(MHCConnection_Fused(n, C, sinkhorn_iters=int(rec["iters"])), p, dev, dtype)
    elif name.startswith("nohres"):
        mod = _load_module(MHCConnection_FusedNoHres(n, C), p, dev, dtype)
    else:
        mod = _load_module(MHCHead(n, C), p, dev, dtype)
    with torch.no_grad():
        if "f_weight" in rec:
            fw = t(rec["f_weight"], dtype).to(dev)
            out = mod(x, lambda z: z @ fw.t())
        else:
            out = mod(x)
    ref = torch.from_numpy(rec["out"])
    assert maxrel(ref, out) <= tol(dtype), f"{name}: {maxrel(ref, out):.3e}"


@pytest.mark.parametrize("iters", [10, 20])
def test_config1_fp32_parity(dev, iters):
    """x [1, 256, 4*768] fp32, phi N(0, 0.02), alpha 0.01,
    biases 0 / I, F = Linear(768, 768) N(0, 0.02); bar 1e-5."""
    n, C = 4, 768
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 256, n * C, generator=g)
    p = make_params("full", n, C, torch.float32, g, stress=False)
    fw = torch.randn(C, C, generator=g) * 0.02
    mod = _load_module(MHCConnection_Fused(n, C, sinkhorn_iters=iters), p, dev, torch.float32)
    with torch.no_grad():
        out = mod(x.to(dev), lambda z: z @ fw.to(dev).t())
    ref = R.mhc_full_forward(x, p, lambda z: z @ fw.t(), n, C, sinkhorn_iters=iters)["out"]
    assert maxrel(ref, out) <= 1e-5


def test_config2_full_size_bf16(dev):
    """BASELINE config 2 shape (16384 tokens, n=4, C=768, bf16, F a fixed N(0,1)
    tensor): a random subset of tokens against the oracle (mHC is per-token), and
    size-independent properties over all tokens."""
    from model import _hip as H, _ops
    n, C, M = 4, 768, 16384
    g = torch.Generator().manual_seed(2)
    x = torch.randn(M, n * C, generator=g).to(torch.bfloat16)
    f = torch.randn(M, C, generator=g).to(torch.bfloat16)
    p = make_params("full", n, C, torch.bfloat16, g, stress=False)
    pd = {k: v.to(dev) for k, v in p.items()}
    packed = _ops.PhiPack(H.MODE_FULL).get(pd["phi_weight"], n, C)
    assert packed is not None
    xd = x.to(dev).view(1, M, n * C)
    o = _ops.pre_full(xd, pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"], pd["alpha_post"],
                      pd["bias_post"], pd["alpha_res"], pd["bias_res"], n, C, 2.0, 1e-6, 1e-6, 20, 1e-6)
    out = _ops.post(xd, o["h_res"], o["h_post"], f.to(dev), n, C)
    hr = o["h_res"].float()
    assert torch.isfinite(out.float()).all()
    assert (hr >= 0).all()
    # bf16 storage of a doubly-stochastic matrix: sums are 1 up to n half-ulps.
    assert (hr.sum(-1) - 1).abs().max().item() <= n * 2 ** -9
    assert (hr.sum(-2) - 1).abs().max().item() <= n * 2 ** -9
    idx = torch.randperm(M, generator=g)[:256]
    xs = x[idx].view(1, -1, n * C)
    fs = f[idx].view(1, -1, C)
    ref = R.mhc_full_forward(xs, p, lambda z: fs, n, C, sinkhorn_iters=20)
    assert maxrel(ref["out"][0], out[idx.to(dev)]) <= 1e-2
    assert maxrel(ref["sub_in"][0], o["sub_in"][idx.to(dev)]) <= 1e-2


def test_config5_n8_bf16(dev):
    """BASELINE config 5 mHC shape: n=8, C=768, phi [6144, 80], 8x8 Sinkhorn."""
    n, C, M = 8, 768, 512
    g = torch.Generator().manual_seed(5)
    x = torch.randn(1, M, n * C, generator=g).to(torch.bfloat16)
    p = make_params("full", n, C, torch.bfloat16, g, stress=False)
    fw = (torch.randn(C, C, generator=g) * 0.02).to(torch.bfloat16)
    mod = _load_module(MHCConnection_Fused(n, C, sinkhorn_iters=20), p, dev, torch.bfloat16)
    with torch.no_grad():
        out = mod(x.to(dev), lambda z: z @ fw.to(dev).t())
    ref = R.mhc_full_forward(x, p, lambda z: z @ fw.t(), n, C, sinkhorn_iters=20)["out"]
    assert maxrel(ref, out) <= 1e-2


def test_sinkhorn_normalize_api(dev):
    M = torch.randn(2, 3, 4, 4)
    got = sinkhorn_normalize(M.to(dev))           # reference default iters=10, eps=1e-6
    assert maxabs(R.sinkhorn(M, 10, 1e-6), got) <= 1e-5


def test_stream_expand_module(dev):
    x = torch.randn(2, 5, 64, device=dev)
    assert torch.equal(StreamExpand(4, 64)(x).cpu(), R.stream_expand(x.cpu(), 4))
    assert StreamExpand(1, 64)(x) is x


def _leaves(p, dev, dtype):
    return {k: v.to(dtype).to(dev).requires_grad_(True) for k, v in p.items()}


@pytest.mark.parametrize("kind", ["full", "nohres"])
def test_backward_vs_oracle_autograd(dev, kind):
    """Gradients to x, phi, alphas, biases and through F against autograd of the
    oracle (fp32, CPU)."""
    n, C, M = 4, 64, 24
    g = torch.Generator().manual_seed(9)
    x = torch.randn(1, M, n * C, generator=g)
    p = make_params(kind, n, C, torch.float32, g)
    lin = nn.Linear(C, C, bias=False)
    with torch.no_grad():
        lin.weight.copy_(torch.randn(C, C, generator=g) * 0.1)
    gout = torch.randn(1, M, n * C, generator=g)

    # oracle on CPU
    xr = x.clone().requires_grad_(True)
    pr = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    lr = nn.Linear(C, C, bias=False)
    lr.load_state_dict(lin.state_dict())
    if kind == "full":
        ref = R.mhc_full_forward(xr, pr, lr, n, C, sinkhorn_iters=20)["out"]
        mod = MHCConnection_Fused(n, C, sinkhorn_iters=20)
    else:
        ref = R.mhc_nohres_forward(xr, pr, lr, n, C)["out"]
        mod = MHCConnection_FusedNoHres(n, C)
    (ref * gout).sum().backward()

    mod = _load_module(mod, p, dev, torch.float32)
    ld = nn.Linear(C, C, bias=False).to(dev)
    ld.load_state_dict(lin.state_dict())
    xd = x.to(dev).requires_grad_(True)
    out = mod(xd, ld)
    (out * gout.to(dev)).sum().backward()
    assert maxrel(ref, out) <= 1e-5
    assert maxrel(xr.grad, xd.grad) <= 1e-4
    assert maxrel(lr.weight.grad, ld.weight.grad) <= 1e-4
    for k in p:
        assert maxrel(pr[k].grad, getattr(mod, k).grad) <= 1e-4, k


def test_head_backward_vs_oracle_autograd(dev):
    n, C, M = 4, 64, 24
    g = torch.Generator().manual_seed(4)
    x = torch.randn(1, M, n * C, generator=g)
    p = make_params("head", n, C, torch.float32, g, phi_std=0.05)
    gout = torch.randn(1, M, C, generator=g)
    xr = x.clone().requires_grad_(True)
    pr = {k: v.clone().requires_grad_(True) for k, v in p.items()}
    (R.head(xr, pr, n, C) * gout).sum().backward()
    mod = _load_module(MHCHead(n, C), p, dev, torch.float32)
    xd = x.to(dev).requires_grad_(True)
    (mod(xd) * gout.to(dev)).sum().backward()
    assert maxrel(xr.grad, xd.grad) <= 1e-4
    for k in p:
        assert maxrel(pr[k].grad, getattr(mod, k).grad) <= 1e-4, k


def test_integration_ctypes_stub(dev, monkeypatch):
    """The ctypes binding shown in INTEGRATION.md, executed as written, gives
    the same outputs as the package's own ops (it calls the same C ABI)."""
    import re
    from pathlib import Path

    from model import _hip as H, _ops

    text = (Path(__file__).resolve().parent.parent / "INTEGRATION.md").read_text()
    sec = text[text.index("## 2."):]
    code = re.search(r"```python\n(.*?)```", sec, re.S).group(1)
    monkeypatch.setenv("MHC_AMD_LIB", str(H.LIB_PATH))
    ns = {}
    exec(compile(code, "INTEGRATION.md", "exec"), ns)

    n, C, M = 4, 768, 80
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, M // 2, n * C, generator=g).to(torch.bfloat16).to(dev)
    f = torch.randn(2, M // 2, C, generator=g).to(torch.bfloat16).to(dev)
    p = {k: v.to(dev) for k, v in make_params("full", n, C, torch.bfloat16, g).items()}
    packed = _ops.PhiPack(H.MODE_FULL).get(p["phi_weight"], n, C)
    args = (p["alpha_pre"], p["bias_pre"], p["alpha_post"], p["bias_post"], p["alpha_res"],
            p["bias_res"])
    sub, h_post, h_res = ns["mhc_pre_sinkhorn"](x, p["phi_weight"], *args, 2.0, 1e-6, 1e-6, n, C,
                                               20, 1e-6, packed=packed)
    o = _ops.pre_full(x, p["phi_weight"], packed, *args, n, C, 2.0, 1e-6, 1e-6, 20, 1e-6)
    assert torch.equal(sub.reshape(M, C), o["sub_in"])
    assert torch.equal(h_post.reshape(M, n), o["h_post"])
    assert torch.equal(h_res.reshape(M, n, n), o["h_res"])
    out = ns["mhc_post"](x, h_res, h_post, f, n, C)
    ref = _ops.post(x, o["h_res"], o["h_post"], f.reshape(M, C), n, C)
    assert torch.equal(out.reshape(M, n * C), ref.reshape(M, n * C))


@pytest.mark.parametrize("name", [
    "c1_full_n4_c768_it20_f32", "c1_full_n4_c768_it10_f32",
    "c2_full_n4_c768_it20_stress_bf16", "c5_full_n8_c768_it20_stress_bf16"])
def test_module_matches_reference_c768(dev, name):
    """Reference _forward_ref rows at C = 768 (tests/golden/cases.py): config 1
    itself (fp32, T = 256) at the 1e-5 bar, and bf16 rows of the config-2
    (n = 4) and config-5 (n = 8) shapes with stress gates (alphas 0.6 / 0.4 /
    0.8, random biases, so every gate follows the projection) at the 1e-2 bar.
    Every bf16 kernel (n = 4 and n = 8) rounds x_norm to bf16 before the
    projection, as _forward_ref does (:845), not fp32 as the reference's fused
    kernel keeps it (model/mhc_fused.py:209-229).  Many more seeds:
    tests/test_gpu_parity_seeds.py."""
    from tests.golden import cases as K
    case, inp, ref = K.load(name)
    assert name in seeded_names("full")
    dtype = inp["x"].dtype
    n, C = case["n"], case["C"]
    p = {k: inp[k] for k in ("phi_weight", "alpha_pre", "bias_pre", "alpha_post", "bias_post",
                             "alpha_res", "bias_res")}
    mod = _load_module(MHCConnection_Fused(n, C, sinkhorn_iters=case["iters"]), p, dev, dtype)
    fw = inp["f_weight"].t().contiguous().to(dev)
    print(f"c768 module {name}", flush=True)
    with torch.no_grad():
        out = mod(inp["x"].to(dev), lambda z: z @ fw)
    err = maxrel(ref["out"], out)
    assert err <= tol(dtype), f"{name}: {err:.3e}"


@pytest.mark.parametrize("n,C,M", [(4, 768, 16384), (8, 768, 8192), (16, 768, 4096)])
def test_full_size_stress_gates_bf16(dev, n, C, M):
    """Full-size launches with projection-driven (stress) gates on every large-batch
    kernel: the persistent kernel at config 2's shape, the K-streamed kernel at
    config 5's (n = 8, with the packed n = 8 post kernel) and at n = 16.  All
    tokens: finite outputs, a non-negative H_res whose bf16 row and column sums
    are 1 up to n half-ulps, 0 <= h_post <= 2; 256 random tokens against the
    oracle at the bf16 bar (mHC is per-token)."""
    from model import _hip as H, _ops
    g = torch.Generator().manual_seed(11 + n)
    x = torch.randn(M, n * C, generator=g).to(torch.bfloat16)
    f = torch.randn(M, C, generator=g).to(torch.bfloat16)
    p = make_params("full", n, C, torch.bfloat16, g, stress=True)
    pd = {k: v.to(dev) for k, v in p.items()}
    packed = _ops.PhiPack(H.MODE_FULL).get(pd["phi_weight"], n, C)
    assert packed is not None
    xd = x.to(dev).view(1, M, n * C)
    print(f"full-size stress n={n} C={C} M={M}", flush=True)
    o = _ops.pre_full(xd, pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"], pd["alpha_post"],
                      pd["bias_post"], pd["alpha_res"], pd["bias_res"], n, C, 2.0, 1e-6, 1e-6, 20, 1e-6)
    out = _ops.post(xd, o["h_res"], o["h_post"], f.to(dev), n, C)
    hr = o["h_res"].float()
    hp = o["h_post"].float()
    assert torch.isfinite(out.float()).all() and torch.isfinite(o["sub_in"].float()).all()
    assert (hr >= 0).all()
    assert (hr.sum(-1) - 1).abs().max().item() <= n * 2 ** -9
    assert (hr.sum(-2) - 1).abs().max().item() <= n * 2 ** -9
    assert (hp >= 0).all() and (hp <= 2).all()
    idx = torch.randperm(M, generator=g)[:256]
    xs = x[idx].view(1, -1, n * C)
    fs = f[idx].view(1, -1, C)
    ref = R.mhc_full_forward(xs, p, lambda z: fs, n, C, sinkhorn_iters=20)
    assert maxrel(ref["out"][0], out[idx.to(dev)]) <= 1e-2
    assert maxrel(ref["sub_in"][0], o["sub_in"][idx.to(dev)]) <= 1e-2
