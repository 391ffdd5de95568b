"""Seeded golden-vector cases whose inputs are not stored.

The larger fixtures (C = 768 rows, function-level vectors) keep only the
reference's outputs plus a SHA-256 digest of the inputs.  The inputs are drawn
again here from a torch.Generator in a fixed order; `load` checks the digest,
so a change in torch's generator fails loudly instead of comparing against
the wrong inputs.  tests/golden/make_golden.py draws the same inputs through
`build_inputs` before calling the reference functions.

Outputs are stored in their own dtype: fp32 as float32, bf16 as its raw
16-bit patterns (uint16), so a bit-exact comparison needs no conversion.
"""
from __future__ import annotations

import hashlib
from pathlib import Path
from typing import Dict, Tuple

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent
DT = {"bf16": torch.bfloat16, "f32": torch.float32}

# name -> case.  kind: pre_full / post_full / pre_nohres / post_nohres /
# sinkhorn (function-level, the reference's *_ref functions) or full (the
# MHCConnection_Fused._forward_ref module forward with F = Linear(C, C)).
# params: "stress" (alphas 0.6 / 0.4 / 0.8, random biases) or "init"
# (alpha 0.01, biases 0 / I, the reference initialisation values).
CASES: Dict[str, dict] = {}


def _add(name, **kw):
    CASES[name] = kw


for _tag in ("bf16", "f32"):
    _add(f"fn_pre_full_n4_c64_stress_{_tag}", kind="pre_full", n=4, C=64, B=2, L=8, dtype=_tag,
         params="stress", seed=101)
    _add(f"fn_pre_full_n8_c32_stress_{_tag}", kind="pre_full", n=8, C=32, B=1, L=12, dtype=_tag,
         params="stress", seed=102)
    _add(f"fn_pre_full_n4_c768_stress_{_tag}", kind="pre_full", n=4, C=768, B=1, L=16,
         dtype=_tag, params="stress", seed=103)
    _add(f"fn_post_full_n4_c64_{_tag}", kind="post_full", n=4, C=64, B=2, L=8, dtype=_tag, seed=104)
    _add(f"fn_post_full_n8_c32_{_tag}", kind="post_full", n=8, C=32, B=1, L=12, dtype=_tag,
         seed=105)
    _add(f"fn_post_full_n4_c768_{_tag}", kind="post_full", n=4, C=768, B=1, L=16, dtype=_tag,
         seed=106)
    _add(f"fn_pre_nohres_n4_c64_stress_{_tag}", kind="pre_nohres", n=4, C=64, B=2, L=8,
         dtype=_tag, params="stress", seed=107)
    _add(f"fn_pre_nohres_n4_c768_stress_{_tag}", kind="pre_nohres", n=4, C=768, B=1, L=16,
         dtype=_tag, params="stress", seed=108)
    _add(f"fn_post_nohres_n4_c64_{_tag}", kind="post_nohres", n=4, C=64, B=2, L=8, dtype=_tag,
         seed=109)
for _n in (2, 4, 8, 16):
    for _it in (1, 10, 20):
        _add(f"fn_sinkhorn_n{_n}_it{_it}_f32", kind="sinkhorn", n=_n, K=64, iters=_it,
             dtype="f32", seed=200 + 10 * _n + _it)
# Module forwards at C = 768.  Config 1 exactly (T = 256, fp32, init params,
# F = Linear(768, 768) ~ N(0, 0.02), 20 Sinkhorn iterations); a shorter
# config-1 row at the reference default of 10 iterations; config-2 / config-5
# distributions (bf16) with stress gates, so the projection drives every gate.
_add("c1_full_n4_c768_it20_f32", kind="full", n=4, C=768, B=1, L=256, dtype="f32",
     params="init", iters=20, f_std=0.02, seed=0)
_add("c1_full_n4_c768_it10_f32", kind="full", n=4, C=768, B=1, L=32, dtype="f32",
     params="init", iters=10, f_std=0.02, seed=1)
_add("c2_full_n4_c768_it20_stress_bf16", kind="full", n=4, C=768, B=2, L=32, dtype="bf16",
     params="stress", iters=20, f_std=0.03, seed=2)
_add("c5_full_n8_c768_it20_stress_bf16", kind="full", n=8, C=768, B=1, L=24, dtype="bf16",
     params="stress", iters=20, f_std=0.03, seed=3)


def _params(n, C, FD, params, g):
    p = {"phi_weight": torch.randn(n * C, FD, generator=g) * 0.02}
    if params == "stress":
        p.update(alpha_pre=torch.tensor(0.6), alpha_post=torch.tensor(0.4),
                 alpha_res=torch.tensor(0.8),
                 bias_pre=torch.randn(n, generator=g) * 0.3,
                 bias_post=torch.randn(n, generator=g) * 0.3,
                 bias_res=torch.eye(n) + torch.randn(n, n, generator=g) * 0.3)
    else:
        p.update(alpha_pre=torch.tensor(0.01), alpha_post=torch.tensor(0.01),
                 alpha_res=torch.tensor(0.01), bias_pre=torch.zeros(n),
                 bias_post=torch.zeros(n), bias_res=torch.eye(n))
    return p


def build_inputs(name: str) -> Dict[str, torch.Tensor]:
    """The case's inputs, drawn in a fixed order from torch.Generator(seed)."""
    c = CASES[name]
    g = torch.Generator().manual_seed(c["seed"])
    dt = DT[c["dtype"]]
    n = c["n"]
    if c["kind"] == "sinkhorn":
        m = torch.randn(c["K"], n, n, generator=g) * 2.0 + torch.eye(n) * 1.5
        return {"M": m.to(dt)}
    C, B, L = c["C"], c["B"], c["L"]
    x = torch.randn(B, L, n * C, generator=g)
    out = {"x": x}
    kind = c["kind"]
    if kind in ("pre_full", "full"):
        out.update(_params(n, C, 2 * n + n * n, c["params"], g))
    elif kind == "pre_nohres":
        p = _params(n, C, 2 * n, c["params"], g)
        out.update({k: p[k] for k in ("phi_weight", "alpha_pre", "bias_pre", "alpha_post",
                                      "bias_post")})
    if kind == "full":
        out["f_weight"] = torch.randn(C, C, generator=g) * c["f_std"]
    if kind in ("post_full", "post_nohres"):
        # gates as the pre phase would hand them over: H_res doubly stochastic,
        # H_post = 2 * sigmoid(.), F an N(0, 1) sublayer output
        logits = torch.randn(B, L, n, n, generator=g) * 0.8 + torch.eye(n)
        h = logits.softmax(-1)
        for _ in range(20):
            h = h / h.sum(-2, keepdim=True)
            h = h / h.sum(-1, keepdim=True)
        out["h_post"] = 2.0 * torch.sigmoid(torch.randn(B, L, n, generator=g) * 0.5)
        out["f_out"] = torch.randn(B, L, C, generator=g)
        if kind == "post_full":
            out["h_res"] = h
    return {k: v.to(dt) for k, v in out.items()}


def digest(tensors: Dict[str, torch.Tensor]) -> str:
    """SHA-256 over (name, dtype, shape, raw bytes) of each tensor, sorted by name."""
    h = hashlib.sha256()
    for k in sorted(tensors):
        t = tensors[k].detach().contiguous()
        h.update(f"{k}|{t.dtype}|{tuple(t.shape)}|".encode())
        raw = t.view(torch.int16) if t.dtype == torch.bfloat16 else t
        h.update(raw.numpy().tobytes())
    return h.hexdigest()


def to_store(t: torch.Tensor) -> np.ndarray:
    """An output in its own dtype: float32, or bf16 bit patterns as uint16."""
    t = t.detach().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype != torch.float32:
        raise TypeError(f"unexpected output dtype {t.dtype}")
    return t.numpy()


def from_store(a: np.ndarray) -> torch.Tensor:
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.int16).copy()).view(torch.bfloat16)
    return torch.from_numpy(a.copy())


def load(name: str) -> Tuple[dict, Dict[str, torch.Tensor], Dict[str, torch.Tensor]]:
    """(case, inputs, reference outputs) of a seeded fixture; raises if the
    regenerated inputs' digest differs from the one stored with the outputs."""
    case = CASES[name]
    inputs = build_inputs(name)
    with np.load(GOLDEN / f"{name}.npz", allow_pickle=False) as z:
        stored = str(z["input_sha256"])
        outs = {k[4:]: from_store(z[k]) for k in z.files if k.startswith("out_")}
    got = digest(inputs)
    if got != stored:
        raise RuntimeError(f"{name}: regenerated inputs differ from the fixture's "
                           f"(sha256 {got[:12]} != {stored[:12]}); torch's generator changed")
    return case, inputs, outs
