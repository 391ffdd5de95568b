"""The persistent pre kernel with row-staged x tiles (whole-row loads through an
LDS transpose, mhc_pre_row_staging on) against the same kernel loading the
MFMA operand layout directly (off).  Both feed the same operands to the same
MFMA and pre-aggregate sequence; the row-staged kernel sums each row's squares
from its whole-row registers, in row order, where the operand-layout kernel
sums per-wave partials.  So inv_rms may differ in its last bit, and through
x_norm's rounding a token's mixes and gates by a rounding step: every output
agrees at rounding level, and tokens whose mixes are bit-identical agree bit
for bit.  The operand-layout path is itself pinned against the oracle by the
other GPU tests; here the sampled outputs are also checked against the oracle
at the BASELINE bars.  Shapes: C a multiple of 256 (the shapes row staging
takes: n in {2, 4} with C in {256, 512, 768, 1024}, n = 1 with C in {512,
1024}, modes full / no-H_res / head), batches with a ragged last tile, fewer
tiles than CUs, several tiles per CU and the C2 size, plus shapes it does not
take (C % 256 != 0, n * C / 256 odd, fused norm), which must be unaffected by
the setting, bit for bit."""
from __future__ import annotations

import pytest
import torch

from oracle import mhc_ref as R
from tests._util import make_params, maxrel, tol

pytestmark = pytest.mark.gpu

from model import _hip as H  # noqa: E402
from model import _ops  # noqa: E402

BF = torch.bfloat16
_MODE = {"full": H.MODE_FULL, "nohres": H.MODE_NOHRES, "head": H.MODE_HEAD}


@pytest.fixture
def staging():
    """Restore the row-staging and token-kernel settings after each test."""
    old_row = _ops.pre_row_staging(-1)
    old_tok = _ops.pre_token_threshold(-1)
    _ops.pre_token_threshold(0)  # persistent kernel at every size
    yield _ops.pre_row_staging
    _ops.pre_row_staging(old_row)
    _ops.pre_token_threshold(old_tok)


def _run(kind, xd, pd, packed, n, C, norm=None):
    if kind == "full":
        o = _ops.pre_full(xd, pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"],
                          pd["alpha_post"], pd["bias_post"], pd["alpha_res"], pd["bias_res"], n, C,
                          2.0, 1e-6, 1e-6, 20, 1e-6, want_h_pre=True, want_raw=True,
                          want_saved=True, norm=norm)
    elif kind == "nohres":
        o = _ops.pre_nohres(xd, pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"],
                            pd["alpha_post"], pd["bias_post"], n, C, 2.0, 1e-6, 1e-6,
                            want_h_pre=True, want_saved=True, norm=norm)
    else:
        out, inv, mix = _ops.head(xd, pd["phi_weight"], packed, pd["alpha"], pd["bias"], n, C,
                                  1e-6, 1e-6, want_saved=True, norm=norm)
        o = {"sub_in": out, "inv_rms": inv, "mixes_raw": mix}
    torch.cuda.synchronize()
    return {k: v.clone() for k, v in o.items() if v is not None}


def _both(staging, kind, n, C, M, seed, norm=None, exact=False):
    g = torch.Generator().manual_seed(seed)
    p = make_params(kind, n, C, BF, g, stress=True)
    x = (torch.randn(1, M, n * C, generator=g) * 2.0).to(BF)
    dev = torch.device("cuda:0")
    pd = {k: v.to(dev) for k, v in p.items()}
    packed = _ops.PhiPack(_MODE[kind]).get(pd["phi_weight"], n, C)
    xd = x.to(dev)
    if norm is not None:
        norm = (norm.to(dev), 1e-6)
    print(f"row staging {kind} n={n} C={C} M={M}", flush=True)
    staging(0)
    ref = _run(kind, xd, pd, packed, n, C, norm)
    staging(1)
    row = _run(kind, xd, pd, packed, n, C, norm)
    assert ref.keys() == row.keys()
    if exact:
        for k in ref:
            assert torch.equal(ref[k], row[k]), k
        return x, p, row
    same = torch.ones(M, dtype=torch.bool, device=dev)  # tokens with bit-identical mixes
    for k in ref:
        if k != "sub_in":  # inv_rms: its last bit; a flipped x_norm element: a bf16 step
            assert maxrel(ref[k], row[k]) <= (1e-6 if k == "inv_rms" else 8e-3), k
        if k not in ("inv_rms", "sub_in"):  # equal mixes: equal gates and pre-aggregate
            same &= (ref[k] == row[k]).reshape(M, -1).all(-1)
    assert maxrel(ref["sub_in"], row["sub_in"]) <= tol(BF)
    assert same.float().mean().item() >= 0.5
    for k in ref:
        if k != "inv_rms":
            assert torch.equal(ref[k].reshape(M, -1)[same], row[k].reshape(M, -1)[same]), k
    return x, p, row


@pytest.mark.parametrize("kind", ["full", "nohres", "head"])
@pytest.mark.parametrize("n,C", [(4, 768), (4, 512), (4, 256), (2, 768), (2, 1024), (1, 512),
                                 (1, 256)])
@pytest.mark.parametrize("M", [1, 37, 4096 + 5, 16384])
def test_row_staging_matches_operand_layout(staging, kind, n, C, M):
    if kind == "head" and n == 1:
        pytest.skip("MHCHead with n = 1 is an RMSNorm (no projection)")
    _both(staging, kind, n, C, M, seed=1000 * n + C + M)


@pytest.mark.parametrize("n,C", [(4, 768), (2, 512)])
def test_row_staging_vs_oracle(staging, n, C):
    M = 16 * 256 * 2 + 11
    x, p, o = _both(staging, "full", n, C, M, seed=7)
    idx = torch.tensor([0, 1, 15, 16, M // 2, M - 12, M - 1])
    sub, h_pre, h_post, h_raw, inv, mixes = R.pre_full(x[:, idx], p, n, C)
    d = idx.to(o["sub_in"].device)
    bar = tol(BF)
    assert maxrel(sub[0], o["sub_in"].view(M, C)[d].cpu()) <= bar
    assert maxrel(h_pre[0], o["h_pre"].view(M, n)[d].cpu()) <= bar
    assert maxrel(h_post[0], o["h_post"].view(M, n)[d].cpu()) <= bar
    assert maxrel(inv[0], o["inv_rms"].view(M)[d].cpu()) <= 1e-5


@pytest.mark.parametrize("n,C,norm", [(4, 640, False), (2, 200, False), (4, 768, True),
                                      (1, 768, False)])
def test_shapes_without_row_staging_unaffected(staging, n, C, norm):
    w = torch.rand(C, generator=torch.Generator().manual_seed(3)).to(BF) + 0.5 if norm else None
    _both(staging, "full", n, C, 4096 + 9, seed=11, norm=w, exact=True)


def test_row_staging_repeat_launches(staging):
    """Many workgroups, repeated launches of the row-staged kernel: bit-identical
    every time (guards the LDS hand-off between steps)."""
    n, C, M = 4, 768, 16 * 256 * 6 + 3
    x, p, first = _both(staging, "full", n, C, M, seed=5)
    dev = torch.device("cuda:0")
    pd = {k: v.to(dev) for k, v in p.items()}
    packed = _ops.PhiPack(H.MODE_FULL).get(pd["phi_weight"], n, C)
    xd = x.to(dev)
    staging(1)
    for _ in range(5):
        again = _run("full", xd, pd, packed, n, C)
        for k in first:
            assert torch.equal(first[k], again[k]), k
