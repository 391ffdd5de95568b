"""The small-batch pre kernel (pre_group_kernel: one workgroup per group of up
to 16 tokens, phi streamed from L2) against the large-batch kernels on the
same inputs: pre_persist_kernel for n <= 4 and pre_kstream_kernel for n = 8.
Each is forced through mhc_pre_token_threshold.  The group kernel walks the
same MFMA blocks in the same order and sums in the same order, so every output
must match bit for bit: the layer's result does not depend on the batch size
or on which side of the threshold it falls.  Both sides are pinned against the
oracle by tests/test_gpu_fused.py and tests/test_gpu_ops.py.

Shapes: group sizes 1, 2, 4 and 8 (M = 1, 37, 300, 700, 1100 on a 256-CU
MI355X), a ragged last group, C a multiple of 256 and not (640, 200), n in
{1, 2, 4, 8}, the three projection modes, with and without the fused RMSNorm,
Sinkhorn iteration counts 20, 1 and 0.  At n = 8 up to
mhc_pre_group_split_tokens (128) the small-batch side is the split form (two
launches); test_group_split_matches_one_launch pins it against the one-launch
kernel directly, with and without handed-over sums of squares."""
from __future__ import annotations

import pytest
import torch

from tests._util import make_params

pytestmark = pytest.mark.gpu

from model import _hip as H  # noqa: E402
from model import _ops  # noqa: E402

BF = torch.bfloat16
_MODE = {"full": H.MODE_FULL, "nohres": H.MODE_NOHRES, "head": H.MODE_HEAD}


@pytest.fixture
def threshold():
    old = _ops.pre_token_threshold(-1)
    yield _ops.pre_token_threshold
    _ops.pre_token_threshold(old)


def _run(kind, xd, pd, packed, n, C, norm, iters):
    if kind == "full":
        o = _ops.pre_full(xd, pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"],
                          pd["alpha_post"], pd["bias_post"], pd["alpha_res"], pd["bias_res"], n, C,
                          2.0, 1e-6, 1e-6, iters, 1e-6, want_h_pre=True, want_raw=True,
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


def _both(threshold, kind, n, C, M, seed, use_norm=False, iters=20):
    g = torch.Generator().manual_seed(seed)
    p = make_params(kind, n, C, BF, g, stress=True)
    x = (torch.randn(1, M, n * C, generator=g) * 2.0).to(BF)
    dev = torch.device("cuda:0")
    pd = {k: v.to(dev) for k, v in p.items()}
    packed = _ops.PhiPack(_MODE[kind]).get(pd["phi_weight"], n, C)
    xd = x.to(dev)
    norm = None
    if use_norm:
        w = (torch.rand(C, generator=g) + 0.5).to(BF)
        norm = (w.to(dev), 1e-6)
    print(f"group {kind} n={n} C={C} M={M} norm={use_norm} iters={iters}", flush=True)
    threshold(0)
    big = _run(kind, xd, pd, packed, n, C, norm, iters)
    threshold(1 << 40)
    small = _run(kind, xd, pd, packed, n, C, norm, iters)
    assert big.keys() == small.keys()
    for k in big:
        assert torch.equal(big[k], small[k]), k


@pytest.mark.parametrize("kind", ["full", "nohres", "head"])
@pytest.mark.parametrize("n,C", [(4, 768), (8, 768), (2, 768), (1, 768), (4, 256), (2, 1024),
                                 (8, 512), (8, 520)])
@pytest.mark.parametrize("M", [1, 37, 300, 1100])
def test_group_matches_large_batch_kernel(threshold, kind, n, C, M):
    # n = 8: C % 64 == 0 walks chunk pairs in both kernels, C = 520 single chunks
    if kind == "head" and n == 1:
        pytest.skip("MHCHead with n = 1 is an RMSNorm (no projection)")
    _both(threshold, kind, n, C, M, seed=100 * n + C + M)


@pytest.mark.parametrize("kind", ["full", "nohres", "head"])
@pytest.mark.parametrize("n,C", [(4, 768), (8, 768), (2, 512)])
@pytest.mark.parametrize("M", [1, 64, 700])
def test_group_matches_large_batch_kernel_with_norm(threshold, kind, n, C, M):
    _both(threshold, kind, n, C, M, seed=7 * n + C + M, use_norm=True)


@pytest.mark.parametrize("n,C", [(4, 640), (2, 200), (8, 640), (1, 200)])
@pytest.mark.parametrize("M", [5, 300])
def test_group_partial_column_blocks(threshold, n, C, M):
    """C not a multiple of 256 (640) or of 32 (200): blocks past C read zeros."""
    _both(threshold, "full", n, C, M, seed=n + C + M)


@pytest.mark.parametrize("iters", [0, 1, 7])
@pytest.mark.parametrize("n", [2, 4, 8])
def test_group_sinkhorn_iteration_counts(threshold, n, iters):
    _both(threshold, "full", n, 768, 21, seed=n + iters, iters=iters)


def test_group_repeat_launches(threshold):
    """Back-to-back launches of the group kernel give the same bits each time."""
    n, C, M = 4, 768, 64
    g = torch.Generator().manual_seed(9)
    p = make_params("full", n, C, BF, g, stress=True)
    x = torch.randn(1, M, n * C, generator=g).to(BF)
    dev = torch.device("cuda:0")
    pd = {k: v.to(dev) for k, v in p.items()}
    packed = _ops.PhiPack(H.MODE_FULL).get(pd["phi_weight"], n, C)
    threshold(1 << 40)
    first = _run("full", x.to(dev), pd, packed, n, C, None, 20)
    for _ in range(5):
        again = _run("full", x.to(dev), pd, packed, n, C, None, 20)
        for k in first:
            assert torch.equal(first[k], again[k]), k


@pytest.mark.parametrize("n,C", [(4, 768), (2, 768), (1, 1024), (8, 768)])
@pytest.mark.parametrize("M", [16 * 256 * 2 + 16 * 37 + 5, 16 * 256 * 4])
def test_group_matches_large_batch_kernel_several_tiles_per_workgroup(threshold, n, C, M):
    """Token counts that give the large-batch kernels two to four tiles a
    workgroup on a 256-CU part: the persistent kernel's steady steps, its last
    step (whose Sinkhorn of the tile before it runs after the loop, on the gate
    waves) and ragged last tiles, bit for bit against the group kernel."""
    _both(threshold, "full", n, C, M, seed=3 * n + C + M)


@pytest.fixture
def split():
    old = _ops.pre_group_split_tokens(-1)
    yield _ops.pre_group_split_tokens
    _ops.pre_group_split_tokens(old)


@pytest.mark.parametrize("kind", ["full", "nohres", "head"])
@pytest.mark.parametrize("M", [1, 16, 37, 64, 128, 300])
@pytest.mark.parametrize("use_norm,use_ssq", [(False, False), (True, False), (False, True),
                                               (True, True)])
def test_group_split_matches_one_launch(threshold, split, kind, M, use_norm, use_ssq):
    """n = 8: the split form (projection per 16-column output tile on its own
    workgroups, mixes parked in the sublayer-input rows, then the rest) against
    the one-launch small-batch kernel, bit for bit, every output."""
    n, C = 8, 768
    g = torch.Generator().manual_seed(11 * M + (kind == "head") + 2 * use_norm + 4 * use_ssq)
    p = make_params(kind, n, C, BF, g, stress=True)
    x = (torch.randn(1, M, n * C, generator=g) * 2.0).to(BF)
    dev = torch.device("cuda:0")
    pd = {k: v.to(dev) for k, v in p.items()}
    packed = _ops.PhiPack(_MODE[kind]).get(pd["phi_weight"], n, C)
    xd = x.to(dev)
    norm = ((torch.rand(C, generator=g) + 0.5).to(BF).to(dev), 1e-6) if use_norm else None
    ssq = None
    if use_ssq:  # per-row partials per 128 columns (any values: both sides read the same)
        ssq = (x.float().view(M, n, C // 128, 128) ** 2).sum(dim=(1, 3)).to(dev).contiguous()
    print(f"group split {kind} M={M} norm={use_norm} ssq={use_ssq}", flush=True)
    threshold(1 << 40)

    def run():
        if kind == "full":
            o = _ops.pre_full(xd, pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"],
                              pd["alpha_post"], pd["bias_post"], pd["alpha_res"], pd["bias_res"],
                              n, C, 2.0, 1e-6, 1e-6, 20, 1e-6, want_h_pre=True, want_raw=True,
                              want_saved=True, norm=norm, ssq=ssq)
        elif kind == "nohres":
            o = _ops.pre_nohres(xd, pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"],
                                pd["alpha_post"], pd["bias_post"], n, C, 2.0, 1e-6, 1e-6,
                                want_h_pre=True, want_saved=True, norm=norm, ssq=ssq)
        else:
            out, inv, mix = _ops.head(xd, pd["phi_weight"], packed, pd["alpha"], pd["bias"], n, C,
                                      1e-6, 1e-6, want_saved=True, norm=norm, ssq=ssq)
            o = {"sub_in": out, "inv_rms": inv, "mixes_raw": mix}
        torch.cuda.synchronize()
        return {k: v.clone() for k, v in o.items() if v is not None}

    split(0)
    one = run()
    split(1 << 40)
    two = run()
    assert one.keys() == two.keys()
    for k in one:
        assert torch.equal(one[k], two[k]), k
