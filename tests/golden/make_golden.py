"""Write golden input/output vectors of the reference's PyTorch mHC path.

Why an import: no reference test, fixture or closed form pins the exact bf16
rounding trajectory of MHCConnection_Fused._forward_ref
(model/mhc_fused.py:836-864), MHCConnection_FusedNoHres._forward_ref
(model/mhc_fused_no_hres.py:635-659), _mhc_head_ref
(model/mhc_common.py:298-308), or of the per-phase functions the oracle
restates one by one: _pre_phase_full_ref / _post_phase_full_ref
(model/mhc_fused.py:533-568), _sinkhorn_ref (:47-56), _pre_phase_ref /
_post_phase_ref (model/mhc_fused_no_hres.py:364-394).  Closed forms and
float64 loops pin their mathematics, not where torch rounds to bf16.  This
script runs those reference functions on the CPU (their PyTorch branch; no
GPU, no Triton launch), in this container only, and stores seeded cases as
.npz fixtures (inputs and outputs, no reference code).

Two formats:
  * the small module cases below store their inputs and outputs;
  * the cases of tests/golden/cases.py (function-level vectors and C = 768
    module rows) store the outputs in their own dtype plus a digest of the
    inputs, which cases.build_inputs draws again at test time.

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


def main_seeded(ref_root: str) -> None:
    """The cases of tests/golden/cases.py, through the reference's functions."""
    sys.path.insert(0, ref_root)
    sys.path.insert(0, str(OUT_DIR))
    import cases as K                                           # noqa: E402
    from model import mhc_fused as RF                           # noqa: E402
    from model import mhc_fused_no_hres as RN                   # noqa: E402

    torch.set_num_threads(1)
    for name, c in K.CASES.items():
        inp = K.build_inputs(name)
        kind, n = c["kind"], c["n"]
        outs = {}
        with torch.no_grad():
            if kind == "sinkhorn":
                outs["y"] = RF._sinkhorn_ref(inp["M"], c["iters"], 1e-6)
            elif kind == "pre_full":
                r = RF._pre_phase_full_ref(inp["x"], inp["phi_weight"], inp["alpha_pre"],
                                           inp["bias_pre"], inp["alpha_post"], inp["bias_post"],
                                           inp["alpha_res"], inp["bias_res"], 2.0, 1e-6, 1e-6,
                                           n, c["C"])
                outs.update(zip(("sub_in", "h_pre", "h_post", "h_res_raw", "inv_rms",
                                 "mixes_raw"), r))
            elif kind == "post_full":
                outs["out"] = RF._post_phase_full_ref(inp["x"], inp["h_res"], inp["h_post"],
                                                      inp["f_out"], n, c["C"])
            elif kind == "pre_nohres":
                r = RN._pre_phase_ref(inp["x"], inp["phi_weight"], inp["alpha_pre"],
                                      inp["bias_pre"], inp["alpha_post"], inp["bias_post"], 2.0,
                                      1e-6, 1e-6, n, c["C"])
                outs.update(zip(("sub_in", "h_pre", "h_post", "inv_rms", "mixes_raw"), r))
            elif kind == "post_nohres":
                outs["out"] = RN._post_phase_ref(inp["x"], inp["h_post"], inp["f_out"], n,
                                                 c["C"])
            elif kind == "full":
                mod = RF.MHCConnection_Fused(n, c["C"], sinkhorn_iters=c["iters"])
                mod = mod.to(inp["x"].dtype)
                for k in ("phi_weight", "alpha_pre", "bias_pre", "alpha_post", "bias_post",
                          "alpha_res", "bias_res"):
                    getattr(mod, k).copy_(inp[k])
                fw = inp["f_weight"]
                outs["out"] = mod._forward_ref(inp["x"], lambda z: z @ fw.t())
            else:
                raise ValueError(kind)
        rec = {"input_sha256": np.array(K.digest(inp))}
        rec.update({"out_" + k: K.to_store(v) for k, v in outs.items()})
        np.savez_compressed(OUT_DIR / f"{name}.npz", **rec)
        print(f"wrote {name}.npz  " + " ".join(f"{k}{tuple(v.shape)}" for k, v in outs.items()))


if __name__ == "__main__":
    root = next((a for a in sys.argv[1:] if not a.startswith("--")), "/root/reference")
    if "--seeded-only" not in sys.argv:
        main(root)
    main_seeded(root)
