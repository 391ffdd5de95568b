"""Float64 pure-Python restatement of the mHC forward -- TEST INFRASTRUCTURE ONLY.

Independent of torch: scalar loops over explicit indices, used on tiny inputs
to pin oracle/mhc_ref.py (a transposed operand, a wrong segment offset or a
dropped eps shows up as a mismatch).  Follows the same reference functions:
model/mhc_fused.py:47-56 (Sinkhorn), :533-568 (pre/post), :836-864 (module);
model/mhc_fused_no_hres.py:364-394; model/mhc_common.py:298-308.
Only tests/ import this module.
"""
from __future__ import annotations

import math
from typing import List, Sequence

Mat = List[List[float]]


def sigmoid(z: float) -> float:
    return 1.0 / (1.0 + math.exp(-z))


def sinkhorn(m: Sequence[Sequence[float]], iters: int, eps: float) -> Mat:
    n = len(m)
    x: Mat = []
    for i in range(n):
        mx = max(m[i])
        e = [math.exp(v - mx) for v in m[i]]
        s = sum(e)
        x.append([v / s + eps for v in e])

    def col_pass(x: Mat) -> Mat:
        sums = [sum(x[i][j] for i in range(n)) for j in range(n)]
        return [[x[i][j] / (sums[j] + eps) for j in range(n)] for i in range(n)]

    def row_pass(x: Mat) -> Mat:
        return [[v / (sum(row) + eps) for v in row] for row in x]

    x = col_pass(x)
    for _ in range(iters - 1):
        x = col_pass(row_pass(x))
    return x


def rms_inv(row: Sequence[float], eps: float) -> float:
    return 1.0 / math.sqrt(sum(v * v for v in row) / len(row) + eps)


def project(row: Sequence[float], inv: float, phi: Sequence[Sequence[float]]) -> List[float]:
    """mixes[f] = sum_k (row[k] * inv) * phi[k][f]."""
    fd = len(phi[0])
    return [sum(row[k] * inv * phi[k][f] for k in range(len(row))) for f in range(fd)]


def mhc_full_token(row: Sequence[float], phi, a_pre, b_pre, a_post, b_post, a_res, b_res,
                   f_of, n: int, C: int, eps=1e-6, pre_eps=1e-6, post_mult=2.0, iters=10,
                   sk_eps=1e-6):
    """One token of MHCConnection_Fused: returns dict(sub_in, h_pre, h_post, h_res_raw,
    h_res, f_out, out).  f_of maps the C-vector sublayer_in to the C-vector F output."""
    inv = rms_inv(row, eps)
    m = project(row, inv, phi)
    h_pre = [sigmoid(m[i] * a_pre + b_pre[i]) + pre_eps for i in range(n)]
    h_post = [sigmoid(m[n + i] * a_post + b_post[i]) * post_mult for i in range(n)]
    raw = [[m[2 * n + i * n + j] * a_res + b_res[i][j] for j in range(n)] for i in range(n)]
    h_res = sinkhorn(raw, iters, sk_eps)
    sub = [sum(h_pre[i] * row[i * C + c] for i in range(n)) for c in range(C)]
    f = f_of(sub)
    out = [sum(h_res[i][j] * row[j * C + c] for j in range(n)) + h_post[i] * f[c]
           for i in range(n) for c in range(C)]
    return dict(sub_in=sub, h_pre=h_pre, h_post=h_post, h_res_raw=raw, h_res=h_res, f_out=f,
                out=out, inv_rms=inv, mixes=m)


def mhc_nohres_token(row, phi, a_pre, b_pre, a_post, b_post, f_of, n, C, eps=1e-6,
                     pre_eps=1e-6, post_mult=2.0):
    inv = rms_inv(row, eps)
    m = project(row, inv, phi)
    h_pre = [sigmoid(m[i] * a_pre + b_pre[i]) + pre_eps for i in range(n)]
    h_post = [sigmoid(m[n + i] * a_post + b_post[i]) * post_mult for i in range(n)]
    sub = [sum(h_pre[i] * row[i * C + c] for i in range(n)) for c in range(C)]
    f = f_of(sub)
    out = [row[i * C + c] + h_post[i] * f[c] for i in range(n) for c in range(C)]
    return dict(sub_in=sub, h_pre=h_pre, h_post=h_post, f_out=f, out=out)


def head_token(row, phi, alpha, bias, n, C, pre_eps=1e-6, rms_eps=1e-6):
    inv = rms_inv(row, rms_eps)
    if n == 1:
        return [v * inv for v in row]
    m = project(row, inv, phi)
    mix = [sigmoid(m[i] * alpha + bias[i]) + pre_eps for i in range(n)]
    return [sum(mix[i] * row[i * C + c] for i in range(n)) for c in range(C)]


def linear(w: Sequence[Sequence[float]]):
    """F(z) = z @ w.T for a [C_out, C_in] weight (torch.nn.Linear without bias)."""
    def f(z):
        return [sum(w[o][k] * z[k] for k in range(len(z))) for o in range(len(w))]
    return f
