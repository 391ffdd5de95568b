"""Pin the oracle (oracle/mhc_ref.py) before trusting it.  CPU only.

How each oracle function is pinned:
  mhc_full_forward, mhc_nohres_forward, head (bf16 and fp32)
      -> golden vectors written by the reference's own _forward_ref /
         _mhc_head_ref (tests/golden/make_golden.py), compared bit-exactly,
         at small C and, for mhc_full_forward, at C = 768 (config 1 itself,
         and config-2 / config-5 rows with stress gates);
      -> float64 scalar-loop brute force (oracle/brute.py) on tiny inputs.
  sinkhorn      -> reference vectors of _sinkhorn_ref (n 2..16, iters 1, 10,
                   20), bit-exact; brute force; closed forms (final column
                   sums = s/(s+eps), non-negativity, circulant fixed point).
  pre_full / post_full / pre_nohres / post_nohres
      -> reference vectors of _pre_phase_full_ref / _post_phase_full_ref /
         _pre_phase_ref / _post_phase_ref in bf16 and fp32, every output
         bit-exact (C up to 768); closed forms (phi = 0 gates, identical
         streams under a row-stochastic H_res, H_post = 0 leaves the einsum,
         uniform h_pre gives the stream mean).
  stream_expand -> definition (every copy equals the input).
Planted-mistake tests show that a transposed H_res, a dropped eps or a
swapped pre/post segment in the oracle fails these checks.
"""
from __future__ import annotations

import math

import pytest
import torch

from oracle import brute
from oracle import mhc_ref as R
from tests._util import golden_names, load_golden, maxrel, seeded_names, t
from tests.golden import cases as K

DT = {"bf16": torch.bfloat16, "f32": torch.float32}


def _golden_case(name):
    rec = load_golden(name)
    dt = DT[str(rec["dtype"])]
    n, C = int(rec["n"]), int(rec["C"])
    x = t(rec["x"], dt)
    p = {k[2:]: t(v, dt) for k, v in rec.items() if k.startswith("p_")}
    fn = None
    if "f_weight" in rec:
        fw = t(rec["f_weight"], dt)
        fn = lambda z: z @ fw.t()  # noqa: E731
    return rec, dt, n, C, x, p, fn


def _oracle_out(name, mod=R):
    rec, dt, n, C, x, p, fn = _golden_case(name)
    if name.startswith("full"):
        return mod.mhc_full_forward(x, p, fn, n, C, sinkhorn_iters=int(rec["iters"]))["out"]
    if name.startswith("nohres"):
        return mod.mhc_nohres_forward(x, p, fn, n, C)["out"]
    return mod.head(x, p, n, C)


@pytest.mark.parametrize("name", golden_names())
def test_oracle_matches_reference_golden(name):
    """The restatement reproduces the reference's own outputs bit for bit."""
    rec = load_golden(name)
    got = _oracle_out(name)
    ref = torch.from_numpy(rec["out"])
    assert torch.equal(got.float(), ref), f"{name}: maxrel {maxrel(ref, got):.3e}"


def _tiny_full(n, C, iters, seed, stress=True):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(1, 3, n * C, generator=g, dtype=torch.float64)
    p = {"phi_weight": torch.randn(n * C, 2 * n + n * n, generator=g, dtype=torch.float64) * 0.2,
         "alpha_pre": torch.tensor(0.7, dtype=torch.float64),
         "alpha_post": torch.tensor(0.5, dtype=torch.float64),
         "alpha_res": torch.tensor(0.9, dtype=torch.float64),
         "bias_pre": torch.randn(n, generator=g, dtype=torch.float64) * 0.3,
         "bias_post": torch.randn(n, generator=g, dtype=torch.float64) * 0.3,
         "bias_res": torch.eye(n, dtype=torch.float64) + torch.randn(n, n, generator=g, dtype=torch.float64) * 0.3}
    fw = torch.randn(C, C, generator=g, dtype=torch.float64) * 0.3
    return x, p, fw


@pytest.mark.parametrize("n,C,iters", [(4, 8, 20), (4, 8, 10), (2, 6, 3), (8, 4, 20), (1, 5, 20), (3, 4, 7)])
def test_oracle_full_vs_brute_f64(n, C, iters):
    """The oracle keeps the reference's fp32 RMS (x.float(), model/mhc_fused.py:843),
    so agreement with the float64 loops is at fp32 precision."""
    x, p, fw = _tiny_full(n, C, iters, seed=n * 100 + C)
    o = R.mhc_full_forward(x, p, lambda z: z @ fw.t(), n, C, sinkhorn_iters=iters)
    f_of = brute.linear(fw.tolist())
    for tok in range(x.shape[1]):
        b = brute.mhc_full_token(
            x[0, tok].tolist(), p["phi_weight"].tolist(), p["alpha_pre"].item(),
            p["bias_pre"].tolist(), p["alpha_post"].item(), p["bias_post"].tolist(),
            p["alpha_res"].item(), p["bias_res"].tolist(), f_of, n, C, iters=iters)
        for k in ("out", "h_res", "sub_in", "h_pre", "h_post"):
            ref = torch.tensor(b[k], dtype=torch.float64).reshape(o[k][0, tok].shape)
            assert torch.allclose(o[k][0, tok], ref, rtol=2e-6, atol=2e-6), k


@pytest.mark.parametrize("n,C", [(4, 8), (2, 5), (8, 3)])
def test_oracle_nohres_and_head_vs_brute_f64(n, C):
    x, p, fw = _tiny_full(n, C, 1, seed=7 + n)
    pn = {"phi_weight": p["phi_weight"][:, :2 * n].contiguous(), "alpha_pre": p["alpha_pre"],
          "alpha_post": p["alpha_post"], "bias_pre": p["bias_pre"], "bias_post": p["bias_post"]}
    o = R.mhc_nohres_forward(x, pn, lambda z: z @ fw.t(), n, C)
    ph = {"phi_weight": p["phi_weight"][:, :n].contiguous(), "alpha": torch.full((1,), 0.8, dtype=torch.float64),
          "bias": p["bias_pre"]}
    oh = R.head(x, ph, n, C)
    for tok in range(x.shape[1]):
        row = x[0, tok].tolist()
        b = brute.mhc_nohres_token(row, pn["phi_weight"].tolist(), pn["alpha_pre"].item(),
                                   pn["bias_pre"].tolist(), pn["alpha_post"].item(),
                                   pn["bias_post"].tolist(), brute.linear(fw.tolist()), n, C)
        assert torch.allclose(o["out"][0, tok], torch.tensor(b["out"], dtype=torch.float64), rtol=2e-6, atol=2e-6)
        bh = brute.head_token(row, ph["phi_weight"].tolist(), 0.8, ph["bias"].tolist(), n, C)
        assert torch.allclose(oh[0, tok], torch.tensor(bh, dtype=torch.float64), rtol=2e-6, atol=2e-6)
    o1 = R.head(x[..., :C].contiguous(), {}, 1, C)
    b1 = brute.head_token(x[0, 0, :C].tolist(), None, None, None, 1, C)
    assert torch.allclose(o1[0, 0], torch.tensor(b1, dtype=torch.float64), rtol=2e-6)


# ------------------------------------------------------------- closed forms

@pytest.mark.parametrize("n,iters", [(4, 20), (4, 10), (8, 20), (2, 1), (16, 20), (3, 5)])
def test_sinkhorn_closed_forms(n, iters):
    eps = 1e-6
    g = torch.Generator().manual_seed(n + iters)
    M = torch.randn(64, n, n, generator=g, dtype=torch.float64) * 2
    P = R.sinkhorn(M, iters, eps)
    assert (P >= 0).all()
    # The last pass divides columns by (s + eps): column sums are s/(s+eps) < 1
    # (the exact identity is test_sinkhorn_exact_column_identity).
    colsum = P.sum(dim=-2)
    assert (colsum <= 1.0).all() and (colsum > 1.0 - 1e-3).all()
    # On mHC-shaped inputs (h_res_raw = I + small mixes) rows converge to 1 too.
    if iters >= 10:
        Mr = torch.eye(n, dtype=torch.float64) + 0.1 * torch.randn(64, n, n, generator=g, dtype=torch.float64)
        rows = R.sinkhorn(Mr, iters, eps).sum(dim=-1)
        assert torch.allclose(rows, torch.ones_like(rows), atol=1e-5)
    # float64 brute force on a few matrices
    for b in range(3):
        ref = torch.tensor(brute.sinkhorn(M[b].tolist(), iters, eps), dtype=torch.float64)
        assert torch.allclose(P[b], ref, rtol=1e-13, atol=1e-15)


def test_sinkhorn_exact_column_identity():
    """After the final column pass each column sum equals s/(s+eps) where s is the
    column sum before it (model/mhc_fused.py:53-55)."""
    eps = 1e-3
    M = torch.randn(5, 4, 4, dtype=torch.float64)
    P_prev = R.sinkhorn(M, 3, eps)
    P_prev = P_prev / (P_prev.sum(dim=-1, keepdim=True) + eps)  # one more row pass
    s = P_prev.sum(dim=-2)
    P = R.sinkhorn(M, 4, eps)
    assert torch.allclose(P.sum(dim=-2), s / (s + eps), rtol=1e-14)


def test_sinkhorn_circulant_fixed_point():
    """bias_res = c*I with alpha = 0: the first softmax is already doubly
    stochastic; the diagonal stays e^c / (e^c + n - 1) up to eps."""
    n, c = 4, 1.0
    M = (torch.eye(n, dtype=torch.float64) * c).expand(3, n, n).contiguous()
    P = R.sinkhorn(M, 20, 1e-12)
    d = math.exp(c) / (math.exp(c) + n - 1)
    assert torch.allclose(torch.diagonal(P, dim1=-2, dim2=-1), torch.full((3, n), d, dtype=torch.float64), rtol=1e-9)


def test_pre_closed_form_zero_phi():
    """phi = 0: mixes = 0, so h_pre = sigmoid(b_pre) + eps, h_post = 2 sigmoid(b_post),
    h_res_raw = b_res, independent of x."""
    n, C = 4, 16
    x = torch.randn(2, 5, n * C, dtype=torch.float64)
    b_pre = torch.randn(n, dtype=torch.float64)
    b_post = torch.randn(n, dtype=torch.float64)
    b_res = torch.randn(n, n, dtype=torch.float64)
    p = {"phi_weight": torch.zeros(n * C, 2 * n + n * n, dtype=torch.float64),
         "alpha_pre": torch.tensor(0.3, dtype=torch.float64), "bias_pre": b_pre,
         "alpha_post": torch.tensor(0.3, dtype=torch.float64), "bias_post": b_post,
         "alpha_res": torch.tensor(0.3, dtype=torch.float64), "bias_res": b_res}
    sub, h_pre, h_post, h_raw, inv, mixes = R.pre_full(x, p, n, C)
    assert torch.allclose(h_pre, (torch.sigmoid(b_pre) + 1e-6).expand_as(h_pre))
    assert torch.allclose(h_post, (2 * torch.sigmoid(b_post)).expand_as(h_post))
    assert torch.allclose(h_raw, b_res.expand_as(h_raw))
    # uniform-in-stream h_pre: sublayer_in = sum_i h_i x_i
    ref = sum(h_pre[..., i:i + 1] * x[..., i * C:(i + 1) * C] for i in range(n))
    assert torch.allclose(sub, ref)
    # inv_rms against the textbook RMSNorm without gain
    xn = torch.nn.functional.rms_norm(x, (n * C,), eps=1e-6)
    assert torch.allclose(x * inv.unsqueeze(-1), xn, rtol=1e-6)


def test_projection_is_rmsnorm_then_matmul():
    n, C = 4, 8
    x = torch.randn(3, 2, n * C, dtype=torch.float64)
    phi = torch.randn(n * C, 2 * n + n * n, dtype=torch.float64)
    p = {"phi_weight": phi, "alpha_pre": torch.tensor(1.0, dtype=torch.float64),
         "alpha_post": torch.tensor(1.0, dtype=torch.float64), "alpha_res": torch.tensor(1.0, dtype=torch.float64),
         "bias_pre": torch.zeros(n, dtype=torch.float64), "bias_post": torch.zeros(n, dtype=torch.float64),
         "bias_res": torch.zeros(n, n, dtype=torch.float64)}
    *_, mixes = R.pre_full(x, p, n, C)
    ref = torch.nn.functional.rms_norm(x, (n * C,), eps=1e-6) @ phi
    assert torch.allclose(mixes.double(), ref, rtol=1e-6, atol=1e-6)


def test_post_closed_forms():
    n, C = 4, 12
    g = torch.Generator().manual_seed(3)
    base = torch.randn(2, 3, C, generator=g, dtype=torch.float64)
    x = R.stream_expand(base, n)
    # every copy equals the input
    for i in range(n):
        assert torch.equal(x[..., i * C:(i + 1) * C], base)
    H = R.sinkhorn(torch.randn(2, 3, n, n, generator=g, dtype=torch.float64), 30, 0.0)
    H = H / H.sum(dim=-1, keepdim=True)  # exactly row-stochastic
    zero = torch.zeros(2, 3, n, dtype=torch.float64)
    f = torch.randn(2, 3, C, generator=g, dtype=torch.float64)
    out = R.post_full(x, H, zero, f, n, C)
    assert torch.allclose(out, x, rtol=1e-12)  # identical streams are a fixed point
    hp = torch.rand(2, 3, n, generator=g, dtype=torch.float64)
    out2 = R.post_full(x, H, hp, f, n, C)
    for i in range(n):
        assert torch.allclose(out2[..., i * C:(i + 1) * C], base + hp[..., i:i + 1] * f, rtol=1e-12)
    out3 = R.post_nohres(x, hp, f, n, C)
    assert torch.allclose(out3, out2, rtol=1e-12)  # H_res = I on identical streams


def test_head_n1_is_rmsnorm():
    x = torch.randn(2, 3, 16, dtype=torch.float64)
    assert torch.allclose(R.head(x, {}, 1, 16), torch.nn.functional.rms_norm(x, (16,), eps=1e-6), rtol=1e-6)


# ------------------------------------------------------- planted mistakes

class _Mutant:
    """The oracle with one planted mistake (tests only)."""

    def __init__(self, kind):
        self.kind = kind

    def sinkhorn(self, M, iters, eps):
        if self.kind == "drop_eps":
            return R.sinkhorn(M, iters, 0.0)
        return R.sinkhorn(M, iters, eps)

    def mhc_full_forward(self, x, p, fn, n, C, sinkhorn_iters=10):
        q = dict(p)
        if self.kind == "swap_pre_post":
            w = q["phi_weight"].clone()
            w[:, :n], w[:, n:2 * n] = p["phi_weight"][:, n:2 * n], p["phi_weight"][:, :n]
            q["phi_weight"] = w
        o = R.mhc_full_forward(x, q, fn, n, C, sinkhorn_iters=sinkhorn_iters)
        if self.kind == "transpose_hres":
            B, L, _ = x.shape
            mixed = torch.einsum("blji,bljc->blic", o["h_res"], x.view(B, L, n, C))
            o["out"] = (mixed + o["h_post"].unsqueeze(-1) * o["f_out"].unsqueeze(-2)).reshape(B, L, n * C)
        return o

    def mhc_nohres_forward(self, *a, **k):
        return R.mhc_nohres_forward(*a, **k)

    def head(self, *a, **k):
        return R.head(*a, **k)


@pytest.mark.parametrize("kind", ["transpose_hres", "swap_pre_post"])
def test_planted_mistakes_fail_golden(kind):
    name = "full_n4_c64_it10_stress_f32.npz"
    rec = load_golden(name)
    got = _oracle_out(name, _Mutant(kind))
    assert maxrel(torch.from_numpy(rec["out"]), got) > 1e-3


def test_planted_dropped_eps_fails_brute():
    M = torch.randn(4, 4, dtype=torch.float64)
    ref = torch.tensor(brute.sinkhorn(M.tolist(), 5, 1e-2), dtype=torch.float64)
    assert (R.sinkhorn(M, 5, 1e-2) - ref).abs().max() < 1e-14
    assert (_Mutant("drop_eps").sinkhorn(M, 5, 1e-2) - ref).abs().max() > 1e-4


# ------------------------------------------- reference vectors (seeded fixtures)

@pytest.fixture
def one_thread():
    """torch's CPU fp32 GEMM splits long reductions (K = n*C = 3072) by thread
    count, so its last bit depends on it; make_golden.py runs the reference at
    one thread, and these checks run the oracle the same way."""
    prev = torch.get_num_threads()
    torch.set_num_threads(1)
    yield
    torch.set_num_threads(prev)


_FN_OUTS = {"pre_full": ("sub_in", "h_pre", "h_post", "h_res_raw", "inv_rms", "mixes_raw"),
            "pre_nohres": ("sub_in", "h_pre", "h_post", "inv_rms", "mixes_raw")}


def oracle_function_outputs(case, inp, mod=R):
    """The oracle function a seeded function-level case pins, on its inputs."""
    kind, n = case["kind"], case["n"]
    if kind == "sinkhorn":
        return {"y": mod.sinkhorn(inp["M"], case["iters"], 1e-6)}
    C = case["C"]
    if kind == "pre_full":
        return dict(zip(_FN_OUTS[kind], mod.pre_full(inp["x"], inp, n, C)))
    if kind == "pre_nohres":
        return dict(zip(_FN_OUTS[kind], mod.pre_nohres(inp["x"], inp, n, C)))
    if kind == "post_full":
        return {"out": mod.post_full(inp["x"], inp["h_res"], inp["h_post"], inp["f_out"], n, C)}
    if kind == "post_nohres":
        return {"out": mod.post_nohres(inp["x"], inp["h_post"], inp["f_out"], n, C)}
    raise ValueError(kind)


@pytest.mark.parametrize("name", [k for k in seeded_names() if k.startswith("fn_")])
def test_oracle_function_matches_reference_vectors(name, one_thread):
    """Each per-phase oracle function reproduces the reference function's
    outputs (every output, its dtype and its bits) on the same inputs."""
    case, inp, ref = K.load(name)
    got = oracle_function_outputs(case, inp)
    assert set(got) == set(ref)
    for k in ref:
        assert got[k].dtype == ref[k].dtype, k
        assert torch.equal(got[k], ref[k].view(got[k].shape)), f"{name}:{k} {maxrel(ref[k], got[k]):.3e}"


@pytest.mark.parametrize("name", seeded_names("full"))
def test_oracle_matches_reference_c768_rows(name, one_thread):
    """mhc_full_forward at C = 768: config 1 itself (fp32, T = 256, alpha 0.01,
    biases 0 / I, F = Linear ~ N(0, 0.02)) and bf16 rows with stress gates."""
    case, inp, ref = K.load(name)
    fw = inp["f_weight"]
    got = R.mhc_full_forward(inp["x"], inp, lambda z: z @ fw.t(), case["n"], case["C"],
                             sinkhorn_iters=case["iters"])["out"]
    assert got.dtype == ref["out"].dtype
    assert torch.equal(got, ref["out"]), f"{name}: {maxrel(ref['out'], got):.3e}"


class _PhaseMutant:
    """Per-phase oracle functions with one planted mistake (tests only)."""

    def __init__(self, kind):
        self.kind = kind

    def pre_full(self, x, p, n, C):
        q = dict(p)
        if self.kind == "swap_pre_post":
            w = p["phi_weight"].clone()
            w[:, :n], w[:, n:2 * n] = p["phi_weight"][:, n:2 * n], p["phi_weight"][:, :n]
            q["phi_weight"] = w
        if self.kind == "skip_xnorm_rounding":
            inv = R._inv_rms(x, 1e-6)
            mixes = (x.float() * inv) @ p["phi_weight"].float()
            q["phi_weight"] = p["phi_weight"]
            out = list(R.pre_full(x, q, n, C))
            out[5] = mixes
            return tuple(out)
        return R.pre_full(x, q, n, C)

    def post_full(self, x, h_res, h_post, f, n, C):
        if self.kind == "transpose_hres":
            h_res = h_res.transpose(-1, -2)
        return R.post_full(x, h_res, h_post, f, n, C)

    def sinkhorn(self, M, iters, eps):
        return R.sinkhorn(M, iters, 0.0 if self.kind == "drop_eps" else eps)


@pytest.mark.parametrize("kind,name", [
    ("swap_pre_post", "fn_pre_full_n4_c64_stress_f32"),
    ("skip_xnorm_rounding", "fn_pre_full_n4_c768_stress_bf16"),
    ("transpose_hres", "fn_post_full_n4_c64_f32"),
    ("drop_eps", "fn_sinkhorn_n4_it1_f32"),
])
def test_planted_mistakes_fail_function_vectors(kind, name, one_thread):
    case, inp, ref = K.load(name)
    got = oracle_function_outputs(case, inp, _PhaseMutant(kind))
    assert any(not torch.equal(got[k], ref[k].view(got[k].shape)) for k in ref)
