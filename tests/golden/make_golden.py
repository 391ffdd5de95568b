"""Write golden input/output vectors of the reference's PyTorch mHC path.

Why an import: no reference test, fixture or closed form pins the exact bf16
rounding trajectory of MHCConnection_Fused._forward_ref
(model/mhc_fused.py:836-864), MHCConnection_FusedNoHres._forward_ref
(model/mhc_fused_no_hres.py:635-659) or _mhc_head_ref
(model/mhc_common.py:298-308).  This script runs those reference functions on
the CPU (their PyTorch branch; no GPU, no Triton launch), in this container
only, and stores small seeded cases as .npz fixtures (inputs and outputs,
no reference code).  fp32 cases are stored alongside as a cross-check.

The reference checkout is never needed at test time: tests read the .npz
files.  Re-run with:  python tests/golden/make_golden.py [/root/reference]
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import torch

OUT_DIR = Path(__file__).resolve().parent


def _arr(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def _params_full(n, C, dtype, g, stress):
    NC, FD = n * C, 2 * n + n * n
    p = {"phi_weight": torch.randn(NC, FD, generator=g) * 0.02}
    if stress:
        p.update(alpha_pre=torch.tensor(0.6), alpha_post=torch.tensor(0.4),
                 alpha_res=torch.tensor(0.8),
                 bias_pre=torch.randn(n, generator=g) * 0.3,
                 bias_post=torch.randn(n, generator=g) * 0.3,
                 bias_res=torch.eye(n) + torch.randn(n, n, generator=g) * 0.3)
    else:
        p.update(alpha_pre=torch.tensor(0.01), alpha_post=torch.tensor(0.01),
                 alpha_res=torch.tensor(0.01), bias_pre=torch.zeros(n),
                 bias_post=torch.zeros(n), bias_res=torch.eye(n))
    return {k: v.to(dtype) for k, v in p.items()}


def main(ref_root: str) -> None:
    sys.path.insert(0, ref_root)
    from model.mhc_fused import MHCConnection_Fused            # noqa: E402
    from model.mhc_fused_no_hres import MHCConnection_FusedNoHres  # noqa: E402
    from model.mhc_common import MHCHead                        # noqa: E402

    torch.set_num_threads(1)
    cases = []
    # (name, kind, n, C, B, L, dtype, iters, stress)
    for dt in (torch.bfloat16, torch.float32):
        tag = "bf16" if dt == torch.bfloat16 else "f32"
        cases += [
            (f"full_n4_c64_it20_{tag}", "full", 4, 64, 2, 8, dt, 20, False),
            (f"full_n4_c64_it10_stress_{tag}", "full", 4, 64, 2, 8, dt, 10, True),
            (f"full_n8_c32_it20_stress_{tag}", "full", 8, 32, 1, 12, dt, 20, True),
            (f"full_n2_c96_it20_stress_{tag}", "full", 2, 96, 1, 10, dt, 20, True),
            (f"nohres_n4_c64_stress_{tag}", "nohres", 4, 64, 2, 8, dt, 0, True),
            (f"head_n4_c64_stress_{tag}", "head", 4, 64, 2, 8, dt, 0, True),
            (f"head_n1_c64_{tag}", "head", 1, 64, 2, 8, dt, 0, False),
        ]
    for name, kind, n, C, B, L, dt, iters, stress in cases:
        g = torch.Generator().manual_seed(1234 + len(name))
        x = torch.randn(B, L, n * C, generator=g).to(dt)
        rec = {"x": _arr(x), "n": np.int64(n), "C": np.int64(C),
               "dtype": np.array("bf16" if dt == torch.bfloat16 else "f32")}
        if kind in ("full", "nohres"):
            fw = (torch.randn(C, C, generator=g) * 0.05).to(dt)
            fn = lambda z, fw=fw: z @ fw.t()  # F = Linear(C, C, bias=False)
            rec["f_weight"] = _arr(fw)
        if kind == "full":
            p = _params_full(n, C, dt, g, stress)
            mod = MHCConnection_Fused(n, C, sinkhorn_iters=iters).to(dt)
            with torch.no_grad():
                for k, v in p.items():
                    getattr(mod, k).copy_(v)
                out = mod._forward_ref(x, fn)
            rec["iters"] = np.int64(iters)
        elif kind == "nohres":
            p = _params_full(n, C, dt, g, stress)
            p = {k: p[k] for k in ("alpha_pre", "alpha_post", "bias_pre", "bias_post")}
            p["phi_weight"] = (torch.randn(n * C, 2 * n, generator=g) * 0.02).to(dt)
            mod = MHCConnection_FusedNoHres(n, C).to(dt)
            with torch.no_grad():
                for k, v in p.items():
                    getattr(mod, k).copy_(v)
                out = mod._forward_ref(x, fn)
        else:
            mod = MHCHead(n, C).to(dt)
            p = {}
            if n > 1:
                p = {"phi_weight": (torch.randn(n * C, n, generator=g) * 0.05).to(dt),
                     "alpha": torch.full((1,), 0.7).to(dt),
                     "bias": (torch.randn(n, generator=g) * 0.3).to(dt)}
            with torch.no_grad():
                for k, v in p.items():
                    getattr(mod, k).copy_(v)
                out = mod(x)
        for k, v in p.items():
            rec["p_" + k] = _arr(v)
        rec["out"] = _arr(out)
        np.savez_compressed(OUT_DIR / f"{name}.npz", **rec)
        print(f"wrote {name}.npz  out{tuple(out.shape)}")


if __name__ == "__main__":
    main(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
