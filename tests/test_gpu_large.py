"""Maximum sizes: batches whose tensors pass 2^31 and 2^32 bytes (x alone is
4.9 GB at 800,000 tokens, n = 4, C = 768), where any 32-bit byte or element
offset would wrap.

Every mHC output is per token except the weight gradients, so these checks
are size-independent:
  * sampled tokens (the first, the last, the middle and a seeded random set)
    of the big launch equal, bit for bit, the same kernel run on just those
    tokens (which the other GPU tests pin against the oracle; at n = 8 to
    rounding, see below), and are checked against the CPU oracle as well at
    the BASELINE bars;
  * the weight gradients are linear in the tokens: the gradient over all
    tokens equals the sum of the gradients over two halves (fp32 outputs,
    only the summation order differs).
"""
from __future__ import annotations

import pytest
import torch

from oracle import mhc_ref as R
from tests._util import make_params, maxabs, maxrel, tol

pytestmark = pytest.mark.gpu

from model import _hip as H  # noqa: E402
from model import _ops  # noqa: E402

BF = torch.bfloat16


def _sample(M: int, k: int = 24, seed: int = 0) -> torch.Tensor:
    g = torch.Generator().manual_seed(seed)
    fixed = torch.tensor([0, 1, 2, 15, 16, M // 2, M // 2 + 1, M - 17, M - 3, M - 2, M - 1])
    return torch.unique(torch.cat([fixed, torch.randint(0, M, (k,), generator=g)]))


def _pre(x, pd, packed, n, C, **kw):
    return _ops.pre_full(x, pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"],
                         pd["alpha_post"], pd["bias_post"], pd["alpha_res"], pd["bias_res"], n, C,
                         2.0, 1e-6, 1e-6, 20, 1e-6, want_h_pre=True, want_raw=True,
                         want_saved=True, **kw)


@pytest.mark.parametrize("n,M", [(4, 800_000), (8, 400_000)])
def test_forward_past_4gb(dev, n, M):
    C = 768
    NC = n * C
    gen = torch.Generator(device=dev).manual_seed(11)
    x = torch.randn(1, M, NC, generator=gen, device=dev, dtype=BF)
    f = torch.randn(1, M, C, generator=gen, device=dev, dtype=BF)
    p = make_params("full", n, C, BF, torch.Generator().manual_seed(12))
    pd = {k: v.to(dev) for k, v in p.items()}
    packed = _ops.PhiPack(H.MODE_FULL).get(pd["phi_weight"], n, C)
    assert x.numel() * 2 > 2 ** 32
    print(f"large forward n={n} M={M}", flush=True)
    big = _pre(x, pd, packed, n, C)
    out = _ops.post(x, big["h_res"], big["h_post"], f, n, C).view(M, NC)
    normed = _pre(x, pd, packed, n, C, norm=(pd["bias_pre"].new_ones(C), 1e-6))["sub_in"]
    torch.cuda.synchronize()

    idx = _sample(M)
    S = idx.numel()
    xs = x[0, idx.to(dev)].unsqueeze(0).contiguous()
    fs = f[0, idx.to(dev)].unsqueeze(0).contiguous()
    small = _pre(xs, pd, packed, n, C)
    small_out = _ops.post(xs, small["h_res"], small["h_post"], fs, n, C).view(S, NC)
    small_norm = _pre(xs, pd, packed, n, C, norm=(pd["bias_pre"].new_ones(C), 1e-6))["sub_in"]
    torch.cuda.synchronize()
    d = idx.to(dev)
    if n <= 4:  # per-token arithmetic in a fixed order: bit for bit
        for k in ("sub_in", "h_pre", "h_post", "h_res_raw", "h_res", "inv_rms", "mixes_raw"):
            assert torch.equal(big[k][d], small[k]), k
        assert torch.equal(out[d], small_out)
        assert torch.equal(normed[d], small_norm)
    else:
        # the n = 8 kernel starts each workgroup's K walk at a different chunk
        # (spreading L2 reads), so a token's fp32 sums run in an order that
        # depends on its workgroup: rounding-level agreement
        for k in ("inv_rms", "mixes_raw"):
            assert maxrel(small[k], big[k][d]) <= 1e-5, k
        for k in ("sub_in", "h_pre", "h_post", "h_res"):
            assert maxrel(small[k], big[k][d]) <= 1e-2, k
        assert maxrel(small_out, out[d]) <= 1e-2
        assert maxrel(small_norm, normed[d]) <= 1e-2

    # and the sampled tokens against the oracle
    xc = xs.cpu()
    sub, h_pre, h_post, h_raw, inv, mixes = R.pre_full(xc, p, n, C)
    bar = tol(BF)
    assert maxrel(h_pre[0], small["h_pre"]) <= bar
    assert maxrel(h_post[0], small["h_post"]) <= bar
    assert maxrel(inv[0], small["inv_rms"]) <= 1e-5
    h_res = R.sinkhorn(h_raw.float(), 20, 1e-6).to(BF)
    assert maxabs(h_res[0], small["h_res"]) <= 1e-2
    ref_out = R.post_full(xc, small["h_res"].cpu().view(1, S, n, n), small["h_post"].cpu().view(1, S, n),
                          fs.cpu(), n, C)
    assert maxrel(ref_out[0], small_out) <= bar


def test_backward_past_4gb(dev):
    n, C, M = 4, 768, 800_000
    NC = n * C
    gen = torch.Generator(device=dev).manual_seed(21)
    x = torch.randn(1, M, NC, generator=gen, device=dev, dtype=BF)
    p = make_params("full", n, C, BF, torch.Generator().manual_seed(22))
    pd = {k: v.to(dev) for k, v in p.items()}
    packed = _ops.PhiPack(H.MODE_FULL).get(pd["phi_weight"], n, C)
    o = _pre(x, pd, packed, n, C)
    f = torch.randn(M, C, generator=gen, device=dev, dtype=BF)
    gout = torch.randn(M, NC, generator=gen, device=dev, dtype=BF)
    gsub = torch.randn(M, C, generator=gen, device=dev, dtype=BF)
    x2 = x.view(M, NC)
    alphas = (pd["alpha_pre"], pd["alpha_post"], pd["alpha_res"])
    biases = (pd["bias_pre"], pd["bias_post"], pd["bias_res"])
    print(f"large backward n={n} M={M}", flush=True)

    def bwd(rows):
        xr = x2 if rows is None else x2[rows].contiguous()
        sel = (lambda t: t) if rows is None else (lambda t: t[rows].contiguous())
        g_x, g_hr, g_hp, g_f = _ops.post_bwd(xr, sel(o["h_res"]), sel(o["h_post"]), sel(f), n, C,
                                             sel(gout))
        g_raw_res = _ops.sinkhorn_bwd(sel(o["h_res_raw"]), g_hr, 20, 1e-6, out_dtype=BF)
        g_xp, g_raw = _ops.pre_bwd(xr, pd["phi_weight"], alphas, biases, sel(o["inv_rms"]),
                                   sel(o["mixes_raw"]), n, C, H.MODE_FULL, 2.0, 1e-6, sel(gsub),
                                   None, g_hp, g_raw_res)
        return dict(g_x=g_x, g_hr=g_hr, g_hp=g_hp, g_f=g_f, g_raw_res=g_raw_res, g_xp=g_xp,
                    g_raw=g_raw)

    big = bwd(None)
    idx = _sample(M, seed=1).to(dev)
    small = bwd(idx)
    torch.cuda.synchronize()
    for k, v in small.items():
        assert torch.equal(big[k][idx], v), k

    # weight gradients: linear in the tokens (fp32 outputs: only the order of the sums differs)
    phi32 = pd["phi_weight"].float()
    h = M // 2
    inv, mix, g_raw = o["inv_rms"], o["mixes_raw"], big["g_raw"]
    full = _ops.pre_bwd_weights(x2, inv, mix, g_raw, phi32, alphas, n, C, H.MODE_FULL)
    lo = _ops.pre_bwd_weights(x2[:h], inv[:h], mix[:h], g_raw[:h], phi32, alphas, n, C, H.MODE_FULL)
    hi = _ops.pre_bwd_weights(x2[h:], inv[h:], mix[h:], g_raw[h:], phi32, alphas, n, C, H.MODE_FULL)
    torch.cuda.synchronize()
    assert full[0].dtype == torch.float32
    assert maxrel(lo[0] + hi[0], full[0]) <= 1e-4
    for s_ in range(3):
        assert maxrel(lo[2][s_].float() + hi[2][s_].float(), full[2][s_].float()) <= 1e-2
