"""GPU parity of every HIP kernel against the CPU oracle, through the C ABI.

Bars (BASELINE): max|ref-got|/max|ref| <= 1e-2 in bf16 and <= 1e-5 in fp32
(the reference's comparator, model/mhc_fused.py:871-876); Sinkhorn H_res row
and column sums within 1e-5 of the oracle's in fp32.
"""
from __future__ import annotations

import pytest
import torch

from oracle import mhc_ref as R
from tests._util import make_params, maxabs, maxrel, seeded_names, tol

pytestmark = pytest.mark.gpu

from model import _hip as H  # noqa: E402
from model import _ops  # noqa: E402


def _to(p, dev):
    return {k: v.to(dev) for k, v in p.items()}


def _pre_case(dev, n, C, M, dtype, stress, iters, use_pack, seed=0):
    g = torch.Generator().manual_seed(seed + 31 * n + C + M)
    x = torch.randn(1, M, n * C, generator=g).to(dtype)
    p = make_params("full", n, C, dtype, g, stress)
    pd = _to(p, dev)
    packed = _ops.PhiPack(H.MODE_FULL).get(pd["phi_weight"], n, C) if use_pack else None
    o = _ops.pre_full(x.to(dev), pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"],
                      pd["alpha_post"], pd["bias_post"], pd["alpha_res"], pd["bias_res"], n, C,
                      2.0, 1e-6, 1e-6, iters, 1e-6, sinkhorn=True, want_h_pre=True,
                      want_raw=True, want_saved=True)
    torch.cuda.synchronize()
    sub, h_pre, h_post, h_raw, inv, mixes = R.pre_full(x, p, n, C)
    h_res = R.sinkhorn(h_raw.float(), iters, 1e-6).to(dtype)
    return o, dict(sub=sub[0], h_pre=h_pre[0], h_post=h_post[0], h_raw=h_raw[0],
                   h_res=h_res[0], inv=inv[0], mixes=mixes[0]), packed


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,C", [(4, 768), (4, 64), (8, 768), (2, 256), (1, 128), (16, 64),
                                 (4, 104), (4, 100), (4, 2048), (2, 1536), (8, 2048), (16, 256)])
@pytest.mark.parametrize("M", [1, 17, 64])
def test_pre_full_vs_oracle(dev, dtype, n, C, M):
    o, r, packed = _pre_case(dev, n, C, M, dtype, stress=True, iters=20, use_pack=True)
    mfma = packed is not None
    print(f"pre n={n} C={C} M={M} {dtype} mfma={mfma}", flush=True)
    bar = tol(dtype)
    assert maxrel(r["sub"], o["sub_in"]) <= bar
    assert maxrel(r["h_pre"], o["h_pre"]) <= bar
    assert maxrel(r["h_post"], o["h_post"]) <= bar
    # The kernels project x_norm rounded to bf16, as the oracle does
    # (model/mhc_fused.py:845): mixes_raw (fp32) lands within half a bf16 step of
    # the oracle's bf16 mixes and h_res_raw within one step (8e-3 of the largest
    # entry).
    raw_bar = 1e-5 if dtype == torch.float32 else 8e-3
    assert maxrel(r["h_raw"], o["h_res_raw"]) <= raw_bar
    assert maxrel(r["inv"], o["inv_rms"]) <= 1e-5
    assert maxrel(r["mixes"], o["mixes_raw"]) <= raw_bar
    assert maxabs(r["h_res"], o["h_res"]) <= (1e-2 if dtype == torch.bfloat16 else 1e-5)
    if dtype == torch.float32:
        for dim in (-1, -2):
            assert maxabs(r["h_res"].sum(dim), o["h_res"].sum(dim)) <= 1e-5


@pytest.mark.parametrize("n,C", [(4, 768), (8, 768), (2, 512), (4, 2048), (2, 1536), (16, 128),
                                 (8, 1152)])
def test_pre_mfma_matches_generic(dev, n, C):
    """The MFMA kernel and the generic VALU kernel agree on the same bf16 input.
    Both project x_norm rounded to bf16 (model/mhc_fused.py:845), so their fp32
    mixes differ only in the order of the fp32 sums (and an x_norm element
    whose rounding an inv_rms one ulp apart flips)."""
    a, _, packed = _pre_case(dev, n, C, 48, torch.bfloat16, True, 20, use_pack=True, seed=5)
    b, _, _ = _pre_case(dev, n, C, 48, torch.bfloat16, True, 20, use_pack=False, seed=5)
    assert packed is not None
    print(f"mfma vs generic n={n} C={C}", flush=True)
    assert maxrel(b["mixes_raw"], a["mixes_raw"]) <= 1e-5
    assert maxrel(b["inv_rms"], a["inv_rms"]) <= 1e-6
    for k in ("sub_in", "h_post", "h_res"):
        assert maxrel(b[k], a[k]) <= 1e-2, k


@pytest.mark.parametrize("n,C,M", [(4, 768, 4096), (2, 512, 4096), (4, 768, 20000),
                                   (8, 768, 8192), (8, 768, 8200), (4, 2048, 2100),
                                   (2, 1536, 4100), (16, 256, 3000), (16, 768, 1030),
                                   (4, 1064, 2100), (2, 1032, 4100), (8, 520, 4100)])
def test_pre_mfma_many_workgroups_repeat(dev, n, C, M):
    """Every CU busy, one or more tiles per workgroup, several launches: the
    persistent kernel's output must equal the generic kernel's within bf16
    rounding on every launch and be bit-identical between launches.  C % 64 != 0
    (1064, 1032, 520) keeps the K-streamed kernel on single 32-column chunks
    instead of chunk pairs.  (A store
    whose data registers were overwritten before the store read them left
    zeros in a few lanes only under this kind of load.)"""
    print(f"many workgroups n={n} C={C} M={M}", flush=True)
    bar = 1e-2
    g = torch.Generator().manual_seed(7 + n + M)
    x = torch.randn(M, n * C, generator=g).to(torch.bfloat16).to(dev)
    p = _to(make_params("full", n, C, torch.bfloat16, g), dev)
    packed = _ops.PhiPack(H.MODE_FULL).get(p["phi_weight"], n, C)
    assert packed is not None
    args = (p["alpha_pre"], p["bias_pre"], p["alpha_post"], p["bias_post"], p["alpha_res"],
            p["bias_res"], n, C, 2.0, 1e-6, 1e-6, 20, 1e-6)
    ref = _ops.pre_full(x, p["phi_weight"], None, *args)
    first = None
    for rep in range(4):
        o = _ops.pre_full(x, p["phi_weight"], packed, *args)
        torch.cuda.synchronize()
        for k in ("sub_in", "h_post", "h_res"):
            assert maxrel(ref[k], o[k]) <= bar, (rep, k)
            if first is not None:
                assert torch.equal(first[k], o[k]), (rep, k)
        first = first or o


@pytest.mark.parametrize("iters", [0, 1, 10, 20])
def test_pre_sinkhorn_iteration_counts(dev, iters):
    o, r, _ = _pre_case(dev, 4, 768, 32, torch.float32, True, iters, use_pack=True)
    assert maxabs(r["h_res"], o["h_res"]) <= 1e-5


@pytest.mark.parametrize("iters", [0, 1, 2, 7, 20])
@pytest.mark.parametrize("n,C,M", [(8, 768, 32), (8, 768, 45), (16, 128, 16), (16, 64, 21),
                                   (4, 1536, 40), (2, 2048, 33)])
def test_pre_kstream_sinkhorn_iteration_counts(dev, iters, n, C, M):
    """bf16, K-streamed kernel (n = 8, n = 16, and n <= 4 at C > 1024): the
    Sinkhorn iterations are spread over the pre-aggregate rounds; every count
    (including 0 and 1) must give the reference schedule."""
    print(f"kstream sinkhorn n={n} C={C} M={M} iters={iters}", flush=True)
    o, r, packed = _pre_case(dev, n, C, M, torch.bfloat16, True, iters, use_pack=True)
    assert packed is not None
    assert maxabs(r["h_res"], o["h_res"]) <= 1e-2
    assert maxrel(r["sub"], o["sub_in"]) <= 1e-2
    if iters >= 1:  # the schedule ends on a column normalisation (bf16 store)
        assert maxabs(o["h_res"].float().cpu().sum(-2), torch.ones(())) <= n * 2.0 ** -8


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,C", [(4, 768), (8, 768), (2, 64), (1, 96), (4, 100), (16, 32),
                                 (16, 128), (4, 2048)])
def test_pre_nohres_vs_oracle(dev, dtype, n, C):
    g = torch.Generator().manual_seed(11 + n + C)
    M = 40
    x = torch.randn(1, M, n * C, generator=g).to(dtype)
    p = make_params("nohres", n, C, dtype, g)
    pd = _to(p, dev)
    packed = _ops.PhiPack(H.MODE_NOHRES).get(pd["phi_weight"], n, C)
    o = _ops.pre_nohres(x.to(dev), pd["phi_weight"], packed, pd["alpha_pre"], pd["bias_pre"],
                        pd["alpha_post"], pd["bias_post"], n, C, 2.0, 1e-6, 1e-6, want_h_pre=True,
                        want_saved=True)
    sub, h_pre, h_post, inv, mixes = R.pre_nohres(x, p, n, C)
    bar = tol(dtype)
    assert maxrel(sub[0], o["sub_in"]) <= bar
    assert maxrel(h_pre[0], o["h_pre"]) <= bar
    assert maxrel(h_post[0], o["h_post"]) <= bar


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,C", [(4, 768), (8, 768), (2, 64), (1, 768), (4, 100), (16, 32),
                                 (16, 128), (2, 2048)])
def test_head_vs_oracle(dev, dtype, n, C):
    g = torch.Generator().manual_seed(17 + n + C)
    M = 33
    x = torch.randn(1, M, n * C, generator=g).to(dtype)
    p = make_params("head", n, C, dtype, g, phi_std=0.05)
    pd = _to(p, dev)
    packed = _ops.PhiPack(H.MODE_HEAD).get(pd["phi_weight"], n, C) if n > 1 else None
    out, inv, mix = _ops.head(x.to(dev), pd["phi_weight"], packed, pd["alpha"], pd["bias"], n, C,
                              1e-6, 1e-6, want_saved=True)
    ref = R.head(x, p, n, C)
    assert maxrel(ref[0], out) <= tol(dtype)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,C", [(4, 768), (8, 768), (2, 64), (1, 64), (4, 100), (16, 32),
                                 (16, 768), (16, 100), (16, 30), (4, 2048)])
@pytest.mark.parametrize("res", [True, False])
def test_post_vs_oracle(dev, dtype, n, C, res):
    g = torch.Generator().manual_seed(23 + n + C)
    M = 70
    x = torch.randn(1, M, n * C, generator=g).to(dtype)
    h_res = R.sinkhorn(torch.randn(1, M, n, n, generator=g), 10, 1e-6).to(dtype)
    h_post = (torch.rand(1, M, n, generator=g) * 2).to(dtype)
    f = torch.randn(1, M, C, generator=g).to(dtype)
    got = _ops.post(x.to(dev), h_res.to(dev) if res else None, h_post.to(dev), f.to(dev), n, C)
    ref = R.post_full(x, h_res, h_post, f, n, C) if res else R.post_nohres(x, h_post, f, n, C)
    assert maxrel(ref[0], got) <= tol(dtype)


def test_post_mixed_dtypes(dev):
    """Autocast training keeps the stream fp32 while F returns bf16
    (model/mhc_fused.py:733, :441): the generic kernel casts on load."""
    n, C, M = 4, 64, 20
    g = torch.Generator().manual_seed(3)
    x = torch.randn(1, M, n * C, generator=g)
    h_res = R.sinkhorn(torch.randn(1, M, n, n, generator=g), 10, 1e-6)
    h_post = torch.rand(1, M, n, generator=g) * 2
    f = torch.randn(1, M, C, generator=g).to(torch.bfloat16)
    got = _ops.post(x.to(dev), h_res.to(dev), h_post.to(dev), f.to(dev), n, C)
    ref = R.post_full(x, h_res, h_post, f.float(), n, C)
    assert got.dtype == torch.float32
    assert maxrel(ref[0], got) <= 1e-5


@pytest.mark.parametrize("n", [1, 2, 3, 4, 5, 8, 16])
@pytest.mark.parametrize("iters", [0, 1, 10, 20])
def test_sinkhorn_vs_oracle(dev, n, iters):
    g = torch.Generator().manual_seed(n * 7 + iters)
    M = torch.randn(3, 37, n, n, generator=g)
    got = _ops.sinkhorn(M.to(dev), iters, 1e-6)
    ref = R.sinkhorn(M, iters, 1e-6)
    assert maxabs(ref, got) <= 1e-5
    for dim in (-1, -2):
        assert maxabs(ref.sum(dim), got.sum(dim)) <= 1e-5


def test_sinkhorn_bf16_io(dev):
    g = torch.Generator().manual_seed(1)
    M = torch.randn(100, 4, 4, generator=g).to(torch.bfloat16)
    got = _ops.sinkhorn(M.to(dev), 20, 1e-6)
    assert got.dtype == torch.bfloat16
    ref = R.sinkhorn(M.float(), 20, 1e-6).to(torch.bfloat16)  # fp32 math, bf16 store
    assert maxabs(ref, got) <= 2 ** -8


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("n,C", [(4, 768), (8, 100), (2, 3)])
def test_stream_expand_exact(dev, dtype, n, C):
    x = torch.randn(2, 9, C).to(dtype)
    got = _ops.stream_expand(x.to(dev), n)
    assert torch.equal(got.cpu(), R.stream_expand(x, n))


def test_empty_batch(dev):
    n, C = 4, 768
    g = torch.Generator().manual_seed(0)
    p = _to(make_params("full", n, C, torch.bfloat16, g), dev)
    x = torch.empty(1, 0, n * C, dtype=torch.bfloat16, device=dev)
    o = _ops.pre_full(x, p["phi_weight"], None, p["alpha_pre"], p["bias_pre"], p["alpha_post"],
                      p["bias_post"], p["alpha_res"], p["bias_res"], n, C, 2.0, 1e-6, 1e-6, 20, 1e-6)
    assert o["sub_in"].shape == (0, C)
    out = _ops.post(x, o["h_res"].view(1, 0, n, n), o["h_post"].view(1, 0, n),
                    torch.empty(1, 0, C, dtype=torch.bfloat16, device=dev), n, C)
    assert out.shape == (0, n * C)


def test_bad_arguments_raise(dev):
    x = torch.randn(1, 4, 4 * 64, device=dev)
    with pytest.raises(ValueError):
        _ops.post(x, None, torch.rand(1, 4, 4, device=dev), torch.randn(1, 4, 64, device=dev), 4, 32)
    with pytest.raises(RuntimeError, match="n must be"):
        _ops.sinkhorn(torch.randn(2, 40, 40, device=dev), 3, 1e-6)


# ------------------------------------------------ reference function vectors

def _fixture(name):
    from tests.golden import cases as K
    case, inp, ref = K.load(name)
    return case, {k: v for k, v in inp.items()}, ref


@pytest.mark.parametrize("name", seeded_names("pre_full") + seeded_names("pre_nohres"))
def test_pre_vs_reference_vectors(dev, name):
    """HIP pre phase (MFMA kernels for bf16) against _pre_phase_full_ref /
    _pre_phase_ref outputs (model/mhc_fused.py:533-559,
    model/mhc_fused_no_hres.py:364-386) on the same inputs."""
    case, inp, ref = _fixture(name)
    n, C = case["n"], case["C"]
    d = {k: v.to(dev) for k, v in inp.items()}
    dtype = inp["x"].dtype
    full = case["kind"] == "pre_full"
    mode = H.MODE_FULL if full else H.MODE_NOHRES
    packed = _ops.PhiPack(mode).get(d["phi_weight"], n, C)
    print(f"pre vectors {name} mfma={packed is not None}", flush=True)
    if full:
        o = _ops.pre_full(d["x"], d["phi_weight"], packed, d["alpha_pre"], d["bias_pre"],
                          d["alpha_post"], d["bias_post"], d["alpha_res"], d["bias_res"], n, C,
                          2.0, 1e-6, 1e-6, 0, 0.0, sinkhorn=False, want_h_pre=True,
                          want_raw=True, want_saved=True)
    else:
        o = _ops.pre_nohres(d["x"], d["phi_weight"], packed, d["alpha_pre"], d["bias_pre"],
                            d["alpha_post"], d["bias_post"], n, C, 2.0, 1e-6, 1e-6,
                            want_h_pre=True, want_saved=True)
    ref = {k: v.reshape(o[k].shape) for k, v in ref.items()}
    bar = tol(dtype)
    # The kernels round x_norm to bf16 before the projection, as
    # _pre_phase_full_ref does (:541-546), and keep the projection's sum in
    # fp32 where the reference rounds it to bf16: the raw projection and
    # h_res_raw carry at most a bf16 step of their largest entry.
    raw_bar = 1e-5 if dtype != torch.bfloat16 else 8e-3
    assert maxrel(ref["sub_in"], o["sub_in"]) <= bar
    assert maxrel(ref["h_pre"], o["h_pre"]) <= bar
    assert maxrel(ref["h_post"], o["h_post"]) <= bar
    assert maxrel(ref["inv_rms"], o["inv_rms"]) <= 1e-5
    assert maxrel(ref["mixes_raw"], o["mixes_raw"]) <= raw_bar
    if full:
        assert maxrel(ref["h_res_raw"], o["h_res_raw"]) <= raw_bar


@pytest.mark.parametrize("name", seeded_names("post_full") + seeded_names("post_nohres"))
def test_post_vs_reference_vectors(dev, name):
    """HIP post phase against _post_phase_full_ref / _post_phase_ref outputs
    (model/mhc_fused.py:562-568, model/mhc_fused_no_hres.py:389-394)."""
    case, inp, ref = _fixture(name)
    n, C = case["n"], case["C"]
    d = {k: v.to(dev) for k, v in inp.items()}
    out = _ops.post(d["x"], d.get("h_res"), d["h_post"], d["f_out"], n, C)
    assert maxrel(ref["out"].reshape(out.shape), out) <= tol(inp["x"].dtype)


@pytest.mark.parametrize("name", seeded_names("sinkhorn"))
def test_sinkhorn_vs_reference_vectors(dev, name):
    """mhc_sinkhorn_fwd against _sinkhorn_ref (model/mhc_fused.py:47-56):
    entries and row / column sums within 1e-5 in fp32."""
    case, inp, ref = _fixture(name)
    y = _ops.sinkhorn(inp["M"].to(dev), case["iters"], 1e-6).cpu()
    r = ref["y"]
    assert maxabs(r, y) <= 1e-5
    for dim in (-1, -2):
        assert maxabs(r.sum(dim), y.sum(dim)) <= 1e-5
