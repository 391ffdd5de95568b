"""Shared helpers for the test suite."""
from __future__ import annotations

from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def maxrel(ref: torch.Tensor, got: torch.Tensor) -> float:
    """The reference's comparator metric: max|ref - got| / max|ref|
    (model/mhc_fused.py:871-876)."""
    ref = ref.detach().float().cpu()
    got = got.detach().float().cpu()
    diff = (ref - got).abs().max().item()
    return diff / max(ref.abs().max().item(), 1e-8)


def maxabs(ref: torch.Tensor, got: torch.Tensor) -> float:
    return (ref.detach().float().cpu() - got.detach().float().cpu()).abs().max().item()


def load_golden(name: str):
    with np.load(GOLDEN / name, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def golden_names():
    """The fixtures that store their inputs (module forwards at small C); the
    seeded ones of tests/golden/cases.py are listed by `seeded_names`."""
    return sorted(p.name for p in GOLDEN.glob("*.npz")
                  if p.name.startswith(("full_", "nohres_", "head_")))


def seeded_names(kind=None):
    """Names of the seeded fixtures (tests/golden/cases.py), optionally of one kind."""
    from tests.golden import cases
    return sorted(k for k, c in cases.CASES.items() if kind is None or c["kind"] == kind)


def t(a, dtype) -> torch.Tensor:
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(dtype)


def make_params(kind: str, n: int, C: int, dtype, g: torch.Generator, stress: bool = True,
                phi_std: float = 0.02):
    """Seeded mHC parameters named like the reference module's parameters.

    stress=True uses large alphas and random biases so that the projection
    visibly drives every gate (the reference init, alpha = 0.01, hides most
    projection errors behind the biases)."""
    NC = n * C
    fd = {"full": 2 * n + n * n, "nohres": 2 * n, "head": n}[kind]
    p = {"phi_weight": torch.randn(NC, fd, generator=g) * phi_std}
    if kind == "head":
        p["alpha"] = torch.full((1,), 0.7 if stress else 0.01)
        p["bias"] = torch.randn(n, generator=g) * 0.3 if stress else torch.zeros(n)
    else:
        a = (0.6, 0.4, 0.8) if stress else (0.01, 0.01, 0.01)
        p["alpha_pre"] = torch.tensor(a[0])
        p["alpha_post"] = torch.tensor(a[1])
        p["bias_pre"] = torch.randn(n, generator=g) * 0.3 if stress else torch.zeros(n)
        p["bias_post"] = torch.randn(n, generator=g) * 0.3 if stress else torch.zeros(n)
        if kind == "full":
            p["alpha_res"] = torch.tensor(a[2])
            p["bias_res"] = (torch.eye(n) + torch.randn(n, n, generator=g) * 0.3) if stress else torch.eye(n)
    return {k: v.to(dtype) for k, v in p.items()}


def tol(dtype) -> float:
    """BASELINE parity bars (max-norm relative): 1e-2 in bf16, 1e-5 in fp32."""
    return {torch.bfloat16: 1e-2, torch.float16: 2e-3, torch.float32: 1e-5}[dtype]
