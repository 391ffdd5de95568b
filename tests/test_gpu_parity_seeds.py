"""Layer-output parity on many random seeds with stress gates.

The bf16 bar, max|out - ref| / max|ref| <= 1e-2 (the reference's comparator,
model/mhc_fused.py:871-876), is under two bf16 steps of the largest output
element, so any intermediate that differs from the PyTorch path in its last
bit can cost that much.  With the projection run on x_norm rounded to bf16 as
the PyTorch path rounds it (model/mhc_fused.py:845), every MFMA kernel (the
persistent and K-streamed large-batch kernels and the small-batch group
kernel) reproduces its mixes, gates and pre-aggregate, and the layer output
stays inside the bar on every seed; most outputs are bit-identical.  (Kept in
fp32, as the reference's fused kernel keeps it, model/mhc_fused.py:209-229,
x_norm put the n = 8 layer output above the bar on 2 of 24 seeds, up to
~1.5e-2.)
"""
from __future__ import annotations

import pytest
import torch

from oracle import mhc_ref as R
from tests._util import make_params, maxrel, tol

pytestmark = pytest.mark.gpu

from model import _ops  # noqa: E402
from model.mhc_fused import MHCConnection_Fused  # noqa: E402

BF = torch.bfloat16


@pytest.fixture
def threshold():
    old = _ops.pre_token_threshold(-1)
    yield _ops.pre_token_threshold
    _ops.pre_token_threshold(old)


def _case(n, seed, dev):
    C = 768
    g = torch.Generator().manual_seed(1000 + seed)
    p = make_params("full", n, C, BF, g, stress=True)
    x = torch.randn(2, 32, n * C, generator=g).to(BF)
    fw = (torch.randn(C, C, generator=g) * 0.03).to(BF)
    mod = MHCConnection_Fused(n, C, sinkhorn_iters=20).to(BF)
    with torch.no_grad():
        for k, v in p.items():
            getattr(mod, k).copy_(v)
    mod = mod.to(dev)
    ref = R.mhc_full_forward(x, p, lambda z: z @ fw.t(), n, C, sinkhorn_iters=20)["out"]
    fwd = fw.t().contiguous().to(dev)
    return mod, x.to(dev), (lambda z: z @ fwd), ref


@pytest.mark.parametrize("path", ["group", "persistent"])
@pytest.mark.parametrize("n", [2, 4])
@pytest.mark.parametrize("seed", range(12))
def test_layer_output_random_seeds_bf16(dev, threshold, n, seed, path):
    threshold(1 << 40 if path == "group" else 0)
    mod, x, f, ref = _case(n, seed, dev)
    print(f"seeds n={n} seed={seed} path={path}", flush=True)
    with torch.no_grad():
        out = mod(x, f).cpu()
    err = maxrel(ref, out)
    differ = (out.float() != ref.float()).float().mean().item()
    assert err <= tol(BF), f"seed {seed}: {err:.3e}"
    assert differ <= 1e-2, f"seed {seed}: {differ:.2%} of outputs differ"


@pytest.mark.parametrize("path", ["group", "kstream"])
@pytest.mark.parametrize("seed", range(12))
def test_layer_output_random_seeds_bf16_n8(dev, threshold, seed, path):
    threshold(1 << 40 if path == "group" else 0)
    mod, x, f, ref = _case(8, seed, dev)
    print(f"seeds n=8 seed={seed} path={path}", flush=True)
    with torch.no_grad():
        out = mod(x, f).cpu()
    err = maxrel(ref, out)
    differ = (out.float() != ref.float()).float().mean().item()
    assert err <= tol(BF), f"seed {seed}: {err:.3e}"
    assert differ <= 1e-2, f"seed {seed}: {differ:.2%} of outputs differ"


@pytest.mark.parametrize("n,C", [(4, 2048), (2, 1536), (16, 256), (8, 2048)])
@pytest.mark.parametrize("seed", range(4))
def test_layer_output_random_seeds_wide_bf16(dev, n, C, seed):
    """The shapes only the K-streamed kernel serves (C > 1024, n = 16), at the
    batch of the seeds above with stress gates, at the 1e-2 bar."""
    bar = tol(BF)
    g = torch.Generator().manual_seed(2000 + seed)
    p = make_params("full", n, C, BF, g, stress=True)
    x = torch.randn(2, 32, n * C, generator=g).to(BF)
    fw = (torch.randn(C, C, generator=g) * 0.03).to(BF)
    mod = MHCConnection_Fused(n, C, sinkhorn_iters=20).to(BF)
    with torch.no_grad():
        for k, v in p.items():
            getattr(mod, k).copy_(v)
    mod = mod.to(dev)
    ref = R.mhc_full_forward(x, p, lambda z: z @ fw.t(), n, C, sinkhorn_iters=20)["out"]
    fwd = fw.t().contiguous().to(dev)
    print(f"wide seeds n={n} C={C} seed={seed}", flush=True)
    with torch.no_grad():
        out = mod(x.to(dev), lambda z: z @ fwd).cpu()
    assert maxrel(ref, out) <= bar, f"seed {seed}: {maxrel(ref, out):.3e}"
