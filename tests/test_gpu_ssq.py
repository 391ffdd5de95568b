"""Per-row sums of squares handed from the launch that writes a stream to the
pre launch that reads it (out_ssq of mhc_post_fwd / mhc_expand_norm_fwd,
x_ssq of the pre-phase entry points; _ops.StreamChain in the modules).

* the post kernels (n = 1 ... 16, with and without H_res, ragged batches) and
  the entry RMSNorm + StreamExpand write the sums of the squares of what they
  store, against float64 sums of the stored tensor; their main outputs are
  bit-identical to the launches without the sums;
* the pre kernels that use them (n = 8, n = 16, C > 1024; large-batch and
  small-batch kernels) take inv_rms from the given sums and agree with the
  launch that forms them itself to the layer bars; n <= 4 at C <= 1024
  ignores them (bit-identical outputs);
* the small-batch and K-streamed kernels stay bit-identical given the sums.
"""
from __future__ import annotations

import pytest
import torch

from tests._util import make_params, maxrel

pytestmark = pytest.mark.gpu

from model import _hip as H  # noqa: E402
from model import _ops  # noqa: E402

ARGS = ("alpha_pre", "bias_pre", "alpha_post", "bias_post", "alpha_res", "bias_res")


def _ref_ssq(t: torch.Tensor, n: int, C: int) -> torch.Tensor:
    M = t.numel() // (n * C)
    return t.detach().cpu().reshape(M, n, C // 128, 128).double().pow(2).sum(dim=(1, 3))


def _given_total(ssq: torch.Tensor) -> torch.Tensor:
    """Row totals as the kernels form them: fp32 sums of the partials in order."""
    s = ssq[:, 0].clone()
    for j in range(1, ssq.shape[1]):
        s = s + ssq[:, j]
    return s


@pytest.mark.parametrize("n", [1, 2, 4, 8, 16])
@pytest.mark.parametrize("C", [128, 768, 2048])
@pytest.mark.parametrize("res", [True, False])
def test_post_writes_row_sums_of_squares(dev, n, C, res):
    M = 37
    g = torch.Generator().manual_seed(n * 7 + C + res)
    bf = torch.bfloat16
    x = torch.randn(M, n * C, generator=g).to(bf).to(dev)
    h_res = (torch.rand(M, n, n, generator=g) / n).to(bf).to(dev) if res else None
    h_post = (torch.rand(M, n, generator=g) * 2).to(bf).to(dev)
    f = torch.randn(M, C, generator=g).to(bf).to(dev)
    print(f"post ssq n={n} C={C} res={res}", flush=True)
    ssq = torch.full((M, C // 128), float("nan"), device=dev)
    out = _ops.post(x, h_res, h_post, f, n, C, ssq_out=ssq)
    plain = _ops.post(x, h_res, h_post, f, n, C)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    ref = _ref_ssq(out, n, C)
    if n == 16:  # one wave per token: the total in slot 0
        assert (ssq[:, 1:] == 0).all()
        assert maxrel(ref.sum(1).float(), ssq[:, 0].cpu()) <= 2e-6
    else:
        assert ((ssq.cpu().double() - ref).abs() / ref).max() <= 2e-6


@pytest.mark.parametrize("n,C", [(4, 768), (8, 768), (8, 256), (16, 1024)])
def test_expand_norm_writes_row_sums_of_squares(dev, n, C):
    M = 19
    g = torch.Generator().manual_seed(n + C)
    x = torch.randn(1, M, C, generator=g).to(torch.bfloat16).to(dev)
    w = (1 + 0.1 * torch.randn(C, generator=g)).to(torch.bfloat16).to(dev)
    ssq = torch.full((M, C // 128), float("nan"), device=dev)
    out = _ops.expand_norm(x, w, 1e-6, n, ssq_out=ssq)
    plain = _ops.expand_norm(x, w, 1e-6, n)
    torch.cuda.synchronize()
    assert torch.equal(out, plain)
    assert (ssq[:, 1:] == 0).all()
    assert maxrel(_ref_ssq(out, n, C).sum(1).float(), ssq[:, 0].cpu()) <= 2e-6


def _pre(x, p, packed, n, C, ssq=None, norm=None):
    return _ops.pre_full(x, p["phi_weight"], packed, *[p[k] for k in ARGS], n, C, 2.0, 1e-6, 1e-6,
                         20, 1e-6, want_h_pre=True, want_raw=True, want_saved=True, ssq=ssq,
                         norm=norm)


# (n, C, M): K-streamed at n = 8 (one tile, many tiles, ragged), the n = 8
# small-batch kernel (M <= 1024), n = 16, and n <= 4 past C = 1024
CASES = [(8, 768, 8192), (8, 768, 1000), (8, 512, 1500), (8, 768, 64), (8, 256, 17),
         (16, 256, 600), (4, 2048, 700), (2, 1536, 300)]


@pytest.mark.parametrize("n,C,M", CASES)
def test_pre_takes_inv_rms_from_given_sums(dev, n, C, M):
    g = torch.Generator().manual_seed(n + C + M)
    bf = torch.bfloat16
    x = torch.randn(1, M, n * C, generator=g).to(bf).to(dev)
    p = {k: v.to(dev) for k, v in make_params("full", n, C, bf, g).items()}
    packed = _ops.PhiPack(H.MODE_FULL).get(p["phi_weight"], n, C)
    ssq = _ref_ssq(x, n, C).float().to(dev)
    print(f"pre given sums n={n} C={C} M={M}", flush=True)
    own = _pre(x, p, packed, n, C)
    given = _pre(x, p, packed, n, C, ssq=ssq)
    torch.cuda.synchronize()
    want = 1.0 / torch.sqrt(_given_total(ssq) / (n * C) + 1e-6)
    assert maxrel(want, given["inv_rms"]) <= 1e-6
    assert maxrel(own["inv_rms"], given["inv_rms"]) <= 1e-6
    # the same token through a different sum order: rounding-level agreement
    for k in ("sub_in", "h_pre", "h_post", "h_res"):
        assert maxrel(own[k].float(), given[k].float()) <= 1e-2, k
    # the kernel reads the given sums: four times the sums halve inv_rms
    quad = _pre(x, p, packed, n, C, ssq=ssq * 4)
    assert maxrel(given["inv_rms"] * 0.5, quad["inv_rms"]) <= 1e-5


@pytest.mark.parametrize("n,C,M", [(4, 768, 4096), (4, 768, 64), (2, 1024, 300)])
def test_pre_ignores_sums_where_it_forms_them_in_registers(dev, n, C, M):
    g = torch.Generator().manual_seed(5 + n + M)
    bf = torch.bfloat16
    x = torch.randn(1, M, n * C, generator=g).to(bf).to(dev)
    p = {k: v.to(dev) for k, v in make_params("full", n, C, bf, g).items()}
    packed = _ops.PhiPack(H.MODE_FULL).get(p["phi_weight"], n, C)
    bogus = torch.full((M, C // 128), 3.0, device=dev)
    own = _pre(x, p, packed, n, C)
    given = _pre(x, p, packed, n, C, ssq=bogus)
    for k in own:
        if own[k] is not None:
            assert torch.equal(own[k], given[k]), k


@pytest.mark.parametrize("M", [64, 200, 1024])
@pytest.mark.parametrize("norm", [False, True])
def test_group_and_kstream_kernels_bit_identical_given_sums(dev, M, norm):
    n, C = 8, 768
    g = torch.Generator().manual_seed(M + norm)
    bf = torch.bfloat16
    x = torch.randn(1, M, n * C, generator=g).to(bf).to(dev)
    p = {k: v.to(dev) for k, v in make_params("full", n, C, bf, g).items()}
    packed = _ops.PhiPack(H.MODE_FULL).get(p["phi_weight"], n, C)
    ssq = _ref_ssq(x, n, C).float().to(dev)
    nw = ((1 + 0.1 * torch.randn(C, generator=g)).to(bf).to(dev), 1e-6) if norm else None
    prev = _ops.pre_token_threshold(1024)
    try:
        small = _pre(x, p, packed, n, C, ssq=ssq, norm=nw)
        _ops.pre_token_threshold(0)
        large = _pre(x, p, packed, n, C, ssq=ssq, norm=nw)
    finally:
        _ops.pre_token_threshold(prev)
    for k in small:
        if small[k] is not None:
            assert torch.equal(small[k], large[k]), k


def test_chain_through_modules_matches_unchained(dev):
    """Two n = 8 connections and an MHCHead, bf16: with a StreamChain (the post
    launch hands its sums to the next pre launch) against the same calls
    without one, to the bf16 layer bar; the chain's sums equal float64 sums
    of the stream it recorded."""
    from model.mhc_common import MHCHead
    from model.mhc_fused import MHCConnection_Fused
    n, C, M = 8, 768, 512
    g = torch.Generator().manual_seed(3)
    bf = torch.bfloat16
    mods = [MHCConnection_Fused(n, C, sinkhorn_iters=20) for _ in range(2)]
    head = MHCHead(n, C)
    for m in mods + [head]:
        with torch.no_grad():
            m.phi_weight.normal_(0.0, 0.05, generator=g)
    mods = [m.to(dev).to(bf) for m in mods]
    head = head.to(dev).to(bf)
    fw = (torch.randn(C, C, generator=g) * 0.05).to(bf).to(dev)
    x = torch.randn(1, M, n * C, generator=g).to(bf).to(dev)
    f = lambda z: z @ fw  # noqa: E731
    with torch.no_grad():
        chain = _ops.StreamChain()
        h = x
        for m in mods:
            h = m(h, f, chain=chain)
            assert chain.src is h and chain.ssq is not None
            assert maxrel(_ref_ssq(h, n, C).float(), chain.ssq.cpu()) <= 2e-6
        out_c = head(h, chain=chain)
        h = x
        for m in mods:
            h = m(h, f)
        out_p = head(h)
    assert maxrel(out_p.float(), out_c.float()) <= 1e-2
