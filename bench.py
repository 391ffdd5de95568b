"""Benchmark of the fused mHC forward on one MI355X.

Workload: 16384 tokens (B=16, T=1024), n=4 streams,
C=768, bf16 streams with fp32 accumulation, phi [3072, 24] ~ N(0, 0.02),
alpha 0.01, biases 0 / I, Sinkhorn 20 iterations, F replaced by a fixed
seeded N(0, 1) tensor [16384, 768].  One step = the two kernels of one mHC
connection: the fused pre phase (RMS + projection + gates + Sinkhorn +
pre-aggregate) and the post phase (res-mix + post-expand).

Timing: W untimed warmup steps, then K timed steps bracketed by
torch.cuda.synchronize().  A step runs the pre kernel on 8 distinct input
sets, then the post kernel on the same 8 sets (see bench_mhc for why); each
group of 8 back-to-back launches of one kernel is bracketed by HIP events on
the stream it runs on; value = tokens / (mean pre + mean post launch time).
After the synchronize and before the first timed step, ~25 ms more of the
same steps run untimed, so the timed ones meet settled clocks.  A cold-cache measurement (read-only
flush before each kernel) and plain torch copy / sum kernels over 1 GiB
(`hbm_calibration`) are reported beside it.

Also printed in the JSON line: `roofline`, the step (pre + post launch, the
two kernels of one connection) against 8 TB/s, with each kernel's own
(`pre_roofline`, `post_roofline`) beside it; the CPU oracle baseline (the
config-2 shape in bf16 on the host cores, with fp32 and config 1 beside it);
`backward`: the four backward launches of one
connection at config 2 (post, Sinkhorn, per-token pre phase, weight
gradients), each against its algorithmic bytes, plus the fwd + bwd tokens/s of
the connection (F excluded); `fp32_layout`: the forward and backward launches
at the config-2 shape in the reference trainers' layout (fp32 stream, phi and
gates, bf16 F under autocast); `other_configs`: the same kernel pair at config
5's n = 8 shape, config 4's 64-token shape, and the widest shapes the
reference's module accepts (dim 2048 at n = 4, n = 16 at dim 768); and the end-to-end model
figures: `e2e_prefill` (config 3), `e2e_decode` (config 4, eager and
HIP-graph replay) and `e2e_prefill_moe` (config 5); `reference_bench_shapes`:
the reference's own fwd + bwd speed workloads (its `_bench` shapes, one
connection around an MLP sublayer).

`*roofline.traffic` is the measured HBM traffic per launch (per step for `roofline`):
FETCH_SIZE + WRITE_SIZE from two rocprofv3 --pmc passes over `--traffic`
(a 1 GiB copy of known size, then one pre and one post launch at config 2),
each scaled by the copy kernel's bytes / counter ratio.  The figures are read
from profiles/traffic_mhc_fwd_c2.txt (the rocprofv3 summary committed beside
the kernel-trace summary); traffic is null when that file is absent.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-e2e] [--no-cpu]
       python bench.py --section fp32-layout|other-configs|reference-shapes|backward
                                                           (one section only)
       python bench.py --traffic     (counter passes only; prints nothing)
       python bench.py --e2e-only [prefill|decode|moe]   (end-to-end model figures only)
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "minimind-mhc_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

METRIC = "mHC fwd tokens/s + % HBM roofline (16k tok, n=4, C=768); e2e prefill tok/s"
HBM_PEAK_GBS = 8000.0
N_STREAMS, C_DIM, TOKENS, ITERS = 4, 768, 16384, 20


def algorithmic_bytes(n: int, C: int, M: int, s: int = 2):
    """Compulsory HBM bytes per launch (each byte of each operand once).

    pre : read x (n*C) + phi once, write sublayer_in (C), h_post (n), h_res (n*n)
    post: read x (n*C), F (C), h_post (n), h_res (n*n), write out (n*C)
    Sum per token: 3*n*C*s + 2*C*s + 2*(n + n*n)*s  (+ phi once).
    """
    fd = 2 * n + n * n
    pre = M * (n * C + C + n + n * n) * s + n * C * fd * s
    post = M * (2 * n * C + C + n + n * n) * s
    return pre, post


def _sync():
    import torch
    torch.cuda.synchronize()


_BUSY = {}


def _queue_ahead(ms: float = 25.0):
    """Keep every CU busy for about `ms` while the host enqueues the timed
    launches behind that work: HIP events then bracket back-to-back kernels,
    not host enqueue gaps.  The work is bf16 GEMMs (torch.matmul on
    contiguous 4096 x 4096 operands), heavy enough to hold the clocks at their
    loaded level: after an idle spell the GPU needs ~15 ms of sustained load
    before its clocks settle (measured on MI355X: the config-2 pre launch runs
    at 31-36 us over the first ~15 ms of back-to-back launches and at
    28.4-28.7 us after; a single-wave spin here left the timed launches inside
    that ramp).  A training loop runs these kernels at the settled level."""
    import torch
    if "a" not in _BUSY:
        a = torch.randn(4096, 4096, device="cuda").to(torch.bfloat16)
        o = torch.empty_like(a)
        for _ in range(3):
            torch.matmul(a, a, out=o)
        _sync()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(20):
            torch.matmul(a, a, out=o)
        e1.record()
        _sync()
        _BUSY.update(a=a, o=o, per_ms=max(e0.elapsed_time(e1) / 20, 1e-3))
    a, o = _BUSY["a"], _BUSY["o"]
    for _ in range(int(ms / _BUSY["per_ms"]) + 1):
        torch.matmul(a, a, out=o)


def bench_mhc(steps: int, warmup: int, sets: int = 8, n: int = N_STREAMS, C: int = C_DIM,
              M: int = TOKENS, cold: bool = True, chain: bool = True):
    """Steady-state kernel times over `sets` distinct input sets.

    Each step runs the pre kernel on every set, then the post kernel on every
    set, so at config 2 (8 sets) a set's x is touched again only after 7 other
    sets' traffic (>= 875 MB, more than the 256 MB Infinity Cache): every
    launch reads cold data and evicts the dirty lines earlier launches left,
    i.e. pays for its own reads and (in steady state) its own writes.  One
    event pair brackets all `sets` launches of a kernel, so the event packets'
    own cost is spread over them (at config 2, 4 sets measured ~0.3 us a
    launch more than 8; 16 sets made the post launch slower, 36.7 us).  Also returns a cold-cache
    measurement (1 GiB read-only flush before each kernel, which leaves clean
    lines, so writes are absorbed by the cache).

    chain: where the shape carries per-row sums of squares from the launch
    that writes the stream to the pre launch that reads it (n >= 8 or
    C > 1024, as inside a model, where each connection's post launch writes
    the next one's input), the post launch writes them for its output and the
    pre launch takes those of its input (for the rotating inputs, formed once
    in the set-up, as a previous post launch would have).  chain=False times
    the pre launch forming them itself."""
    import torch
    from model import _hip as H, _ops

    dev = torch.device("cuda:0")
    g = torch.Generator().manual_seed(0)
    xs = [torch.randn(1, M, n * C, generator=g).to(torch.bfloat16).to(dev) for _ in range(sets)]
    fs = [torch.randn(M, C, generator=g).to(torch.bfloat16).to(dev) for _ in range(sets)]
    phi = (torch.randn(n * C, 2 * n + n * n, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    a = torch.tensor(0.01, dtype=torch.bfloat16, device=dev)
    b0 = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    br = torch.eye(n, dtype=torch.bfloat16, device=dev)
    packed = _ops.PhiPack(H.MODE_FULL).get(phi, n, C)
    assert packed is not None, "configs 2, 4 and 5 take the MFMA kernels"
    use_ssq = chain and _ops.ssq_wanted(torch.bfloat16, n, C)
    ssq_in = [(x.view(M, n, C // _ops.SSQ_COLS, _ops.SSQ_COLS).float().pow(2).sum(dim=(1, 3))
               .contiguous() if use_ssq else None) for x in xs]
    ssq_out = [torch.empty(M, C // _ops.SSQ_COLS, dtype=torch.float32, device=dev) if use_ssq
               else None for _ in range(sets)]

    # Outputs are allocated once per input set through the checked op wrappers,
    # and the timed launches call the C ABI on them directly (what a C caller
    # does): the wrappers' Python checks and allocations cost about as much
    # host time per call as the kernel takes, and a host that falls behind the
    # GPU leaves gaps between the timed launches.
    outs = [_ops.pre_full(xs[s], phi, packed, a, b0, a, b0, a, br, n, C, 2.0, 1e-6, 1e-6,
                          ITERS, 1e-6) for s in range(sets)]
    finals = [_ops.post(xs[s], outs[s]["h_res"], outs[s]["h_post"], fs[s], n, C)
              for s in range(sets)]
    lib = H.load()
    stream = H.stream(dev)
    BF = H.dtype_tag(xs[0])
    M_ = xs[0].shape[0] * xs[0].shape[1]
    pre_args = [(xs[s].data_ptr(), BF, phi.data_ptr(), BF, H.ptr(packed), a.data_ptr(),
                 b0.data_ptr(), a.data_ptr(), b0.data_ptr(), a.data_ptr(), br.data_ptr(), BF,
                 outs[s]["sub_in"].data_ptr(), None, outs[s]["h_post"].data_ptr(), None,
                 outs[s]["h_res"].data_ptr(), None, None, M_, n, C, 2.0, 1e-6, 1e-6, ITERS, 1e-6,
                 H.ptr(ssq_in[s]), stream) for s in range(sets)]
    post_args = [(xs[s].data_ptr(), BF, outs[s]["h_res"].data_ptr(), outs[s]["h_post"].data_ptr(),
                  BF, fs[s].data_ptr(), BF, finals[s].data_ptr(), M_, n, C, H.ptr(ssq_out[s]),
                  stream) for s in range(sets)]
    pre_fn, post_fn = lib.mhc_pre_fwd, lib.mhc_post_fwd

    def pre(s):
        H.check(pre_fn(*pre_args[s]), "mhc_pre_fwd")
        return outs[s]

    def post(s, o):
        H.check(post_fn(*post_args[s]), "mhc_post_fwd")
        return finals[s]

    def ev():
        return torch.cuda.Event(enable_timing=True)

    def step(rec):
        # one event pair around the `sets` back-to-back launches of each
        # kernel: per-launch time = elapsed / sets (bracketing every launch
        # would add the event packets' own dispatch latency to each one)
        e0, e1, e2 = ev(), ev(), ev()
        e0.record()
        outs = [pre(s) for s in range(sets)]
        e1.record()
        for s in range(sets):
            post(s, outs[s])
        e2.record()
        rec["pre"].append((e0, e1))
        rec["post"].append((e1, e2))

    warm = {"pre": [], "post": []}
    for _ in range(max(warmup, 2)):
        step(warm)
    _sync()
    # Settle: the GPU's clocks need ~15 ms of sustained load after an idle
    # spell (see _queue_ahead).  Where a launch takes well over the host's
    # ~10 us to enqueue one, the load is this step itself, enqueued for ~25 ms
    # ahead of the timed steps, so they run at the operating point their own
    # work sets (at config 2 that measured ~0.2 us a step faster than settling
    # on bf16 GEMMs, whose MFMA load leaves other clocks).  Shorter launches
    # (config 4's 64 tokens) would leave the host behind the GPU: there the
    # GEMMs of _queue_ahead give the host its head start.
    per_step = sum(a_.elapsed_time(b_) for a_, b_ in warm["pre"][1:] + warm["post"][1:])
    per_step /= len(warm["pre"]) - 1
    if per_step / (2 * sets) > 0.02:
        for _ in range(int(25.0 / per_step) + 1):
            step({"pre": [], "post": []})
    else:
        _queue_ahead()
    rec = {"pre": [], "post": []}
    for _ in range(steps):
        step(rec)
    _sync()
    t_pre = [a_.elapsed_time(b_) / sets for a_, b_ in rec["pre"]]
    t_post = [a_.elapsed_time(b_) / sets for a_, b_ in rec["post"]]
    steady = dict(t_pre=sum(t_pre) / len(t_pre), t_post=sum(t_post) / len(t_post),
                  t_pre_min=min(t_pre), t_post_min=min(t_post), chain=bool(use_ssq))
    if not cold:
        return steady, None

    # cold, clean cache: read-only 1 GiB flush before each kernel
    flush = torch.ones(256 * 1024 * 1024, dtype=torch.float32, device=dev)
    sink = torch.empty((), dtype=torch.float32, device=dev)
    cold = {"pre": [], "post": []}
    for it in range(steps + warmup):
        torch.sum(flush, dim=0, out=sink)
        e0, e1 = ev(), ev()
        e0.record()
        o = pre(0)
        e1.record()
        torch.sum(flush, dim=0, out=sink)
        e2, e3 = ev(), ev()
        e2.record()
        post(0, o)
        e3.record()
        if it >= warmup:
            cold["pre"].append((e0, e1))
            cold["post"].append((e2, e3))
    _sync()
    c_pre = [a_.elapsed_time(b_) for a_, b_ in cold["pre"]]
    c_post = [a_.elapsed_time(b_) for a_, b_ in cold["post"]]
    del flush
    return steady, dict(t_pre=sum(c_pre) / len(c_pre), t_post=sum(c_post) / len(c_post))


def backward_bytes(n: int, C: int, M: int, s: int = 2):
    """Compulsory HBM bytes per backward launch (bf16 tensors, fp32 saved
    inv_rms / mixes_raw / g_raw; FD = 2n + n*n):
      post_bwd     read g_out, x (n*C each), F (C), h_post, h_res; write g_x (n*C), g_F (C),
                   g_h_post, g_h_res
      sinkhorn_bwd read h_res_raw, g_h_res (n*n each); write g_h_res_raw
      pre_bwd      read x (n*C), g_sub (C), g_h_post, g_h_res_raw, inv_rms, mixes_raw (FD fp32),
                   phi once; write g_x (n*C), g_raw (FD fp32)
      weights      read x (n*C), inv_rms, mixes_raw, g_raw; write g_phi once"""
    fd = 2 * n + n * n
    h = n + n * n
    post = M * ((3 * n * C + 2 * C) * s + 2 * h * s)
    sk = M * 3 * n * n * s
    pre = M * ((2 * n * C + C + h) * s + 4 + 8 * fd) + n * C * fd * s
    wts = M * (n * C * s + 4 + 8 * fd) + n * C * fd * s
    return {"post_bwd": post, "sinkhorn_bwd": sk, "pre_bwd": pre, "pre_bwd_weights": wts}


def bench_backward(reps: int = 20, sets: int = 4, n: int = N_STREAMS, M: int = TOKENS):
    """Steady-state times of the four backward launches of one mHC connection
    (bf16, C = 768; config 2 by default: 16384 tokens, n = 4), rotating `sets`
    input sets as bench_mhc does, with the saved tensors of a real forward."""
    import torch
    from model import _hip as H, _ops

    dev = torch.device("cuda:0")
    C = C_DIM
    bf = torch.bfloat16
    g = torch.Generator().manual_seed(2)
    phi = (torch.randn(n * C, 2 * n + n * n, generator=g) * 0.02).to(bf).to(dev)
    a = torch.tensor(0.01, dtype=bf, device=dev)
    b0 = torch.zeros(n, dtype=bf, device=dev)
    br = torch.eye(n, dtype=bf, device=dev)
    packed = _ops.PhiPack(H.MODE_FULL).get(phi, n, C)
    S = []
    for _ in range(sets):
        x = torch.randn(M, n * C, generator=g).to(bf).to(dev)
        o = _ops.pre_full(x.view(1, M, n * C), phi, packed, a, b0, a, b0, a, br, n, C, 2.0, 1e-6,
                          1e-6, ITERS, 1e-6, want_raw=True, want_saved=True)
        f = torch.randn(M, C, generator=g).to(bf).to(dev)
        gout = torch.randn(M, n * C, generator=g).to(bf).to(dev)
        gsub = torch.randn(M, C, generator=g).to(bf).to(dev)
        S.append(dict(x=x, o=o, f=f, gout=gout, gsub=gsub))
    for s in S:  # the intermediate gradients each later kernel consumes
        _, s["ghr"], s["ghp"], _ = _ops.post_bwd(s["x"], s["o"]["h_res"], s["o"]["h_post"], s["f"],
                                                 n, C, s["gout"])
        s["graw_res"] = _ops.sinkhorn_bwd(s["o"]["h_res_raw"], s["ghr"], ITERS, 1e-6, out_dtype=bf)
        _, s["graw"] = _ops.pre_bwd(s["x"], phi, (a, a, a), (b0, b0, br), s["o"]["inv_rms"],
                                    s["o"]["mixes_raw"], n, C, H.MODE_FULL, 2.0, 1e-6, s["gsub"],
                                    None, s["ghp"], s["graw_res"])
    ops = {
        "post_bwd": lambda s: _ops.post_bwd(s["x"], s["o"]["h_res"], s["o"]["h_post"], s["f"], n,
                                            C, s["gout"]),
        "sinkhorn_bwd": lambda s: _ops.sinkhorn_bwd(s["o"]["h_res_raw"], s["ghr"], ITERS, 1e-6,
                                                    out_dtype=bf),
        "pre_bwd": lambda s: _ops.pre_bwd(s["x"], phi, (a, a, a), (b0, b0, br), s["o"]["inv_rms"],
                                          s["o"]["mixes_raw"], n, C, H.MODE_FULL, 2.0, 1e-6,
                                          s["gsub"], None, s["ghp"], s["graw_res"]),
        "pre_bwd_weights": lambda s: _ops.pre_bwd_weights(s["x"], s["o"]["inv_rms"],
                                                          s["o"]["mixes_raw"], s["graw"], phi,
                                                          (a, a, a), n, C, H.MODE_FULL),
    }
    nbytes = backward_bytes(n, C, M)
    out = {}
    for name, fn in ops.items():
        for s in S:
            fn(s)
        _sync()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        _queue_ahead()
        e0.record()
        for _ in range(reps):
            for s in S:
                fn(s)
        e1.record()
        _sync()
        ms = e0.elapsed_time(e1) / (reps * sets)
        gbs = nbytes["pre" if name == "pre_valu" else name] / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 5), "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": nbytes["pre" if name == "pre_valu" else name]}
    out["total_ms"] = round(sum(v["ms"] for v in out.values()), 5)
    out["note"] = ("timings include each launch's own small torch allocations (outputs, "
                   "workspace); the weights entry is two launches (partials + reduction)")
    return out


def bench_head_backward(reps: int = 20, sets: int = 4, n: int = N_STREAMS, M: int = TOKENS):
    """The MHCHead (the model's exit, FD = n) forward and its two backward
    launches at C = 768, in bf16 and in the fp32 trainer layout (model/
    mhc_common.py:311-400 forward; its autograd backward).  Bytes: forward
    reads x (n*C), writes out (C) and the saved inv_rms / mixes; pre_bwd reads
    x, g_out (C), inv_rms, mixes, phi, writes g_x (n*C) and g_raw; weights
    reads x, inv_rms, mixes, g_raw, writes g_phi."""
    import torch
    from model import _hip as H, _ops

    dev = torch.device("cuda:0")
    C = C_DIM
    out = {}
    for tag, dt in (("bf16", torch.bfloat16), ("fp32", torch.float32)):
        es = 2 if dt == torch.bfloat16 else 4
        g = torch.Generator().manual_seed(7)
        phi = (torch.randn(n * C, n, generator=g) * 0.02).to(dt).to(dev)
        a = torch.tensor(0.01, dtype=dt, device=dev)
        b = torch.zeros(n, dtype=dt, device=dev)
        packed = _ops.PhiPack(H.MODE_HEAD).get(phi, n, C)
        alphas, biases = (a, None, None), (b, None, None)
        S = []
        for _ in range(sets):
            x = torch.randn(M, n * C, generator=g).to(dt).to(dev)
            o, inv, mix = _ops.head(x.view(1, M, n * C), phi, packed, a, b, n, C, 1e-6, 1e-6,
                                    want_saved=True)
            go = torch.randn(M, C, generator=g).to(dt).to(dev)
            _, graw = _ops.pre_bwd(x, phi, alphas, biases, inv, mix, n, C, H.MODE_HEAD, 0.0, 1e-6,
                                   g_sub=go)
            S.append(dict(x=x, inv=inv, mix=mix, go=go, graw=graw))
        ops = {
            "head_fwd": lambda s: _ops.head(s["x"].view(1, M, n * C), phi, packed, a, b, n, C, 1e-6,
                                            1e-6, want_saved=True),
            "pre_bwd": lambda s: _ops.pre_bwd(s["x"], phi, alphas, biases, s["inv"], s["mix"], n, C,
                                              H.MODE_HEAD, 0.0, 1e-6, g_sub=s["go"]),
            "pre_bwd_weights": lambda s: _ops.pre_bwd_weights(s["x"], s["inv"], s["mix"], s["graw"],
                                                              phi, alphas, n, C, H.MODE_HEAD),
        }
        fd = n
        nbytes = {"head_fwd": M * ((n * C + C) * es + 4 + 4 * fd) + n * C * fd * es,
                  "pre_bwd": M * ((2 * n * C + C) * es + 4 + 8 * fd) + n * C * fd * es,
                  "pre_bwd_weights": M * (n * C * es + 4 + 8 * fd) + n * C * fd * es}
        res = {}
        for name, fn in ops.items():
            for s in S:
                fn(s)
            _sync()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            _queue_ahead()
            e0.record()
            for _ in range(reps):
                for s in S:
                    fn(s)
            e1.record()
            _sync()
            ms = e0.elapsed_time(e1) / (reps * sets)
            gbs = nbytes[name] / (ms * 1e-3) / 1e9
            res[name] = {"ms": round(ms, 5), "GBps": round(gbs, 1),
                         "frac": round(gbs / HBM_PEAK_GBS, 4), "algorithmic_bytes": nbytes[name]}
        res["config"] = f"MHCHead n={n} (FD={fd}), C={C}, {M} tokens, {tag} x / phi / gradients"
        out[tag] = res
    return out


def layout_bytes(n: int, C: int, M: int, sx: int = 4, sf: int = 2, sp: int = 4):
    """Compulsory HBM bytes per launch in the reference trainers' layout
    (trainer/train_pretrain.py:129-130: fp32 model under bf16 autocast): fp32
    stream, gates, gradients and parameters (sx, sp bytes), bf16 sublayer
    output F and its gradient (sf).  Same operand lists as algorithmic_bytes
    and backward_bytes."""
    fd = 2 * n + n * n
    h = n + n * n
    return {
        "pre": M * (n * C + C + h) * sx + n * C * fd * sp,
        "post": M * (2 * n * C * sx + C * sf + h * sx),
        "post_bwd": M * (3 * n * C * sx + 2 * C * sf + 2 * h * sx),
        "sinkhorn_bwd": M * 3 * n * n * sx,
        "pre_bwd": M * ((2 * n * C + C + h) * sx + 4 + 8 * fd) + n * C * fd * sp,
        "pre_bwd_weights": M * (n * C * sx + 4 + 8 * fd) + n * C * fd * sp,
    }


def bench_layout32(reps: int = 10, sets: int = 4, n: int = N_STREAMS, M: int = TOKENS):
    """The forward and backward launches of one connection at the config-2
    shape in the reference trainers' layout: fp32 stream x, fp32 phi and gate
    parameters, bf16 F (what F returns under autocast, model/mhc_fused.py:441),
    fp32 gradients of the stream.  Timed like bench_backward: `sets` rotating
    input sets, steady state."""
    import torch
    from model import _hip as H, _ops

    dev = torch.device("cuda:0")
    C = C_DIM
    f32, bf = torch.float32, torch.bfloat16
    g = torch.Generator().manual_seed(5)
    phi = (torch.randn(n * C, 2 * n + n * n, generator=g) * 0.02).to(dev)
    a = torch.tensor(0.01, dtype=f32, device=dev)
    b0 = torch.zeros(n, dtype=f32, device=dev)
    br = torch.eye(n, dtype=f32, device=dev)
    packed = _ops.PhiPack(H.MODE_FULL).get(phi, n, C)
    S = []
    for _ in range(sets):
        x = torch.randn(M, n * C, generator=g).to(dev)
        o = _ops.pre_full(x.view(1, M, n * C), phi, packed, a, b0, a, b0, a, br, n, C, 2.0, 1e-6,
                          1e-6, ITERS, 1e-6, want_raw=True, want_saved=True)
        f = torch.randn(M, C, generator=g).to(bf).to(dev)
        gout = torch.randn(M, n * C, generator=g).to(dev)
        gsub = torch.randn(M, C, generator=g).to(dev)
        S.append(dict(x=x, o=o, f=f, gout=gout, gsub=gsub))
    for s in S:
        _, s["ghr"], s["ghp"], _ = _ops.post_bwd(s["x"], s["o"]["h_res"], s["o"]["h_post"], s["f"],
                                                 n, C, s["gout"])
        s["graw_res"] = _ops.sinkhorn_bwd(s["o"]["h_res_raw"], s["ghr"], ITERS, 1e-6, out_dtype=f32)
        _, s["graw"] = _ops.pre_bwd(s["x"], phi, (a, a, a), (b0, b0, br), s["o"]["inv_rms"],
                                    s["o"]["mixes_raw"], n, C, H.MODE_FULL, 2.0, 1e-6, s["gsub"],
                                    None, s["ghp"], s["graw_res"])
    ops = {
        "pre": lambda s: _ops.pre_full(s["x"].view(1, M, n * C), phi, packed, a, b0, a, b0, a, br,
                                       n, C, 2.0, 1e-6, 1e-6, ITERS, 1e-6, want_raw=True,
                                       want_saved=True),
        # the same launch without the phi image: the VALU kernel (one workgroup
        # per token) the MFMA kernels replace for fp32 streams
        "pre_valu": lambda s: _ops.pre_full(s["x"].view(1, M, n * C), phi, None, a, b0, a, b0, a,
                                            br, n, C, 2.0, 1e-6, 1e-6, ITERS, 1e-6, want_raw=True,
                                            want_saved=True),
        "post": lambda s: _ops.post(s["x"], s["o"]["h_res"], s["o"]["h_post"], s["f"], n, C),
        "post_bwd": lambda s: _ops.post_bwd(s["x"], s["o"]["h_res"], s["o"]["h_post"], s["f"], n,
                                            C, s["gout"]),
        "sinkhorn_bwd": lambda s: _ops.sinkhorn_bwd(s["o"]["h_res_raw"], s["ghr"], ITERS, 1e-6,
                                                    out_dtype=f32),
        "pre_bwd": lambda s: _ops.pre_bwd(s["x"], phi, (a, a, a), (b0, b0, br), s["o"]["inv_rms"],
                                          s["o"]["mixes_raw"], n, C, H.MODE_FULL, 2.0, 1e-6,
                                          s["gsub"], None, s["ghp"], s["graw_res"]),
        "pre_bwd_weights": lambda s: _ops.pre_bwd_weights(s["x"], s["o"]["inv_rms"],
                                                          s["o"]["mixes_raw"], s["graw"], phi,
                                                          (a, a, a), n, C, H.MODE_FULL),
    }
    nbytes = layout_bytes(n, C, M)
    out = {}
    for name, fn in ops.items():
        for s in S:
            fn(s)
        _sync()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        _queue_ahead()
        e0.record()
        for _ in range(reps):
            for s in S:
                fn(s)
        e1.record()
        _sync()
        ms = e0.elapsed_time(e1) / (reps * sets)
        gbs = nbytes["pre" if name == "pre_valu" else name] / (ms * 1e-3) / 1e9
        out[name] = {"ms": round(ms, 5), "GBps": round(gbs, 1), "frac": round(gbs / HBM_PEAK_GBS, 4),
                     "algorithmic_bytes": nbytes["pre" if name == "pre_valu" else name]}
    fwd = out["pre"]["ms"] + out["post"]["ms"]
    bwd = sum(out[k]["ms"] for k in ("post_bwd", "sinkhorn_bwd", "pre_bwd", "pre_bwd_weights"))
    out["fwd_ms"] = round(fwd, 5)
    out["bwd_ms"] = round(bwd, 5)
    out["fwd_tokens_per_s"] = round(M / (fwd * 1e-3), 1)
    out["config"] = (f"{M} tokens, n={n}, C={C}: x / phi / gates / stream gradients fp32, "
                     "F and its gradient bf16 (autocast)")
    return out


def layout32_c5():
    """bench_layout32 at config 5's connection shape (n = 8, 8192 tokens)."""
    out = bench_layout32(n=8, M=8192)
    out["config"] = ("C5 shape: 8192 tokens, n=8, C=768: x / phi / gates / stream gradients "
                     "fp32, F and its gradient bf16 (autocast)")
    return out


TRAFFIC_FILE = ROOT / "profiles" / "traffic_mhc_fwd_c2.txt"


def read_traffic():
    """Measured bytes per launch from the committed counter summary:
    lines `<key>: <bytes>` for pre_fetch, pre_write, post_fetch, post_write
    (already scaled by the copy-kernel calibration)."""
    if not TRAFFIC_FILE.exists():
        return None
    vals = {}
    for ln in TRAFFIC_FILE.read_text().splitlines():
        k, sep, v = ln.partition(":")
        if sep and k.strip() in ("pre_fetch", "pre_write", "post_fetch", "post_write"):
            try:
                vals[k.strip()] = float(v.split()[0])
            except (ValueError, IndexError):
                pass
    return vals if len(vals) == 4 else None


def traffic_passes(vector_pre: bool = False, extra: bool = False):
    """What the FETCH_SIZE / WRITE_SIZE counter passes run: a plain copy of
    1 GiB -> 1 GiB and a plain sum over 1 GiB (known bytes, to calibrate the
    counters), then one pre and one post launch at config 2 on fresh data.
    With `extra`, also one launch of each other MFMA kernel (see below)."""
    import torch
    from model import _hip as H, _ops

    dev = torch.device("cuda:0")
    src = torch.ones(256 * 1024 * 1024, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    sink = torch.empty((), dtype=torch.float32, device=dev)
    dst.copy_(src)
    torch.sum(src, dim=0, out=sink)
    _sync()
    del src, dst
    n, C, M = N_STREAMS, C_DIM, TOKENS
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, M, n * C, generator=g).to(torch.bfloat16).to(dev)
    f = torch.randn(M, C, generator=g).to(torch.bfloat16).to(dev)
    phi = (torch.randn(n * C, 2 * n + n * n, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    a = torch.tensor(0.01, dtype=torch.bfloat16, device=dev)
    b0 = torch.zeros(n, dtype=torch.bfloat16, device=dev)
    br = torch.eye(n, dtype=torch.bfloat16, device=dev)
    packed = _ops.PhiPack(H.MODE_FULL).get(phi, n, C)
    _sync()
    o = _ops.pre_full(x, phi, packed, a, b0, a, b0, a, br, n, C, 2.0, 1e-6, 1e-6, ITERS, 1e-6)
    _ops.post(x, o["h_res"], o["h_post"], f, n, C)
    _sync()
    if vector_pre:
        # the same pre phase on the generic VALU kernel (projection as fp32
        # FMAs, no MFMA), for the MFMA-vs-VALU comparison
        _ops.pre_full(x, phi, None, a, b0, a, b0, a, br, n, C, 2.0, 1e-6, 1e-6, ITERS, 1e-6)
        _sync()
    if extra:
        # one launch of each other MFMA kernel, for the MFMA counter pass:
        # the config-2 backward (per-token pre phase, weight gradients) and
        # the config-5 pre phase (n = 8, 8192 tokens)
        o2 = _ops.pre_full(x, phi, packed, a, b0, a, b0, a, br, n, C, 2.0, 1e-6, 1e-6, ITERS, 1e-6,
                           want_raw=True, want_saved=True)
        gsub = torch.randn(M, C, generator=g).to(torch.bfloat16).to(dev)
        ghp = torch.randn(M, n, generator=g).to(torch.bfloat16).to(dev)
        ghr = torch.randn(M, n * n, generator=g).to(torch.bfloat16).to(dev)
        x2 = x.view(M, n * C)
        _, graw = _ops.pre_bwd(x2, phi, (a, a, a), (b0, b0, br), o2["inv_rms"], o2["mixes_raw"], n,
                               C, H.MODE_FULL, 2.0, 1e-6, gsub, None, ghp, ghr)
        _ops.pre_bwd_weights(x2, o2["inv_rms"], o2["mixes_raw"], graw, phi, (a, a, a), n, C,
                             H.MODE_FULL)
        _sync()
        del x, x2, f, o, o2, gsub
        n8, M8 = 8, 8192
        x8 = torch.randn(1, M8, n8 * C, generator=g).to(torch.bfloat16).to(dev)
        phi8 = (torch.randn(n8 * C, 2 * n8 + n8 * n8, generator=g) * 0.02).to(torch.bfloat16).to(dev)
        b08 = torch.zeros(n8, dtype=torch.bfloat16, device=dev)
        br8 = torch.eye(n8, dtype=torch.bfloat16, device=dev)
        pk8 = _ops.PhiPack(H.MODE_FULL).get(phi8, n8, C)
        # the model's launch (the rows' sums of squares handed over, as the
        # previous post launch writes them), then the same without them
        ssq8 = (x8.view(M8, n8, C // _ops.SSQ_COLS, _ops.SSQ_COLS).float().pow(2).sum(dim=(1, 3))
                .contiguous())
        _sync()
        _ops.pre_full(x8, phi8, pk8, a, b08, a, b08, a, br8, n8, C, 2.0, 1e-6, 1e-6, ITERS, 1e-6,
                      ssq=ssq8)
        _sync()
        _ops.pre_full(x8, phi8, pk8, a, b08, a, b08, a, br8, n8, C, 2.0, 1e-6, 1e-6, ITERS, 1e-6)
        _sync()


def hbm_calibration(reps: int = 10):
    """Plain torch kernels over 1 GiB: a copy (read + write) and a sum (read)."""
    import torch
    dev = torch.device("cuda:0")
    src = torch.ones(256 * 1024 * 1024, dtype=torch.float32, device=dev)
    dst = torch.empty_like(src)
    sink = torch.empty((), dtype=torch.float32, device=dev)
    out = {}
    for name, fn, nbytes in (("copy", lambda: dst.copy_(src), 2 * src.numel() * 4),
                             ("read", lambda: torch.sum(src, dim=0, out=sink), src.numel() * 4)):
        fn()
        _sync()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(reps):
            fn()
        e1.record()
        _sync()
        out[name + "_GBps"] = round(nbytes * reps / (e0.elapsed_time(e1) * 1e-3) / 1e9, 1)
    del src, dst
    return out


def _cpu_median(fn, warmup: int = 3, reps: int = 10):
    """Median seconds per call of fn over `reps` calls after `warmup` calls."""
    for _ in range(warmup):
        fn()
    times = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    times.sort()
    return times[len(times) // 2]


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads() -> int:
    """The host CPUs this process may use: its affinity set, capped at the 16
    CPUs a one-GPU box allots to its job (OMP_NUM_THREADS there)."""
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = os.cpu_count() or 1
    return max(1, min(avail, 16))


def cpu_baseline():
    """The oracle (torch CPU restatement of the reference _forward_ref) on the
    host cores, under torch.inference_mode(), 3 warm-up calls then the median of
    10:
      c2_bf16 : the config-2 workload itself, 16384 tokens, bf16, F a fixed tensor
                (the headline);
      c2_fp32 : the same in fp32;
      c1_fp32 : config 1, 256 tokens, fp32, F = Linear(768, 768) with N(0, 0.02)
                weights inside the timed call;
    each with its algorithmic GB/s (the GPU's byte formula)."""
    import torch
    from oracle import mhc_ref as R
    from tests._util import make_params

    threads = _cpu_threads()
    torch.set_num_threads(threads)
    n, C = N_STREAMS, C_DIM
    g = torch.Generator().manual_seed(0)
    res = {}
    with torch.inference_mode():
        for key, dt, m in (("c2_bf16", torch.bfloat16, TOKENS), ("c2_fp32", torch.float32, TOKENS),
                           ("c1_fp32", torch.float32, 256)):
            x = torch.randn(1, m, n * C, generator=g).to(dt)
            p = make_params("full", n, C, dt, g, stress=False)
            if key == "c1_fp32":
                lin = torch.nn.Linear(C, C, bias=False)
                torch.nn.init.normal_(lin.weight, 0.0, 0.02, generator=g)
                f = lin
            else:
                fz = torch.randn(1, m, C, generator=g).to(dt)
                f = (lambda z, fz=fz: fz)
            med = _cpu_median(lambda: R.mhc_full_forward(x, p, f, n, C, sinkhorn_iters=ITERS))
            nbytes = sum(algorithmic_bytes(n, C, m, s=x.element_size()))
            res[key] = {"tokens_per_s": round(m / med, 1), "GBps": round(nbytes / med / 1e9, 2),
                        "ms_per_call": round(med * 1e3, 2), "tokens": m}
            del x, f
    head = res["c2_bf16"]
    return {"value": head["tokens_per_s"], "unit": "tokens/s", "cores": threads, "kind": "port",
            "sample": f"oracle mhc_full_forward (reference _forward_ref restated) on the full "
                      f"config-2 shape, {TOKENS} tokens x n={n} x C={C}, bf16, F fixed; "
                      f"median of 10 calls after 3 warm-up",
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(),
            "threads_note": "torch threads = this process's CPU affinity set, capped at the 16 "
                            "CPUs a one-GPU box allots to its job",
            "runs": res}


def e2e_prefill(steps: int = 5, warmup: int = 2):
    """MiniMind-3-mHC, 8 layers, hidden 768, 8 q / 4 kv heads,
    head_dim 96, SwiGLU 2048, vocab 6400, n=4, bf16, N(0, 0.02) init;
    prefill B=8, T=1024 (logits for every position, as the reference forward)."""
    import torch
    from model.model_minimind import MiniMindForCausalLM, init_normal_

    dev = torch.device("cuda:0")
    cfg = _dense_config()
    torch.manual_seed(0)
    model = init_normal_(MiniMindForCausalLM(cfg)).to(torch.bfloat16).to(dev).eval()
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 6400, (8, 1024), generator=g).to(dev)
    with torch.inference_mode():
        for _ in range(warmup):
            model(ids)
        _sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            model(ids)
        _sync()
    dt = (time.perf_counter() - t0) / steps
    return {"value": round(ids.numel() / dt, 1), "unit": "tokens/s", "ms_per_forward": round(dt * 1e3, 3),
            "config": "C3: 8 layers, hidden 768, 8q/4kv heads, head_dim 96, SwiGLU 2048, vocab 6400, "
                      "n=4, bf16, B=8 T=1024, 16 mHC connections + StreamExpand + MHCHead"}


def isolated_configs(steps: int, warmup: int):
    """The isolated pre + post kernel pair at the other BASELINE shapes:
    config 5's n = 8 connection (B=4, T=2048: 8192 tokens, phi [6144, 80],
    8x8 Sinkhorn) and config 4's decode shape (64 tokens, n = 4), where the
    pair is launch-bound; and at the widest shapes the reference's module
    accepts (model/mhc_fused.py:599-600, :784): dim 2048 at n = 4 and n = 16
    at dim 768, 16384 tokens each (K-streamed pre kernel; one-wave-per-token
    post kernel at n = 16).  Timed as bench_mhc times config 2.  Where the shape
    carries the rows' sums of squares along the chain (bench_mhc), the entry
    is timed that way, and config 5 also without it (`_unchained`)."""
    out = {}
    for key, n, C, M, sets, chain in (("c5_n8_M8192", 8, C_DIM, 8192, 4, True),
                                      ("c5_n8_M8192_unchained", 8, C_DIM, 8192, 4, False),
                                      ("c4_n4_M64", 4, C_DIM, 64, 8, True),
                                      ("c4_n8_M64", 8, C_DIM, 64, 8, True),
                                      ("wide_n4_C2048_M16384", 4, 2048, TOKENS, 4, True),
                                      ("wide_n16_C768_M16384", 16, C_DIM, TOKENS, 4, True)):
        r, _ = bench_mhc(steps, warmup, sets=sets, n=n, C=C, M=M, cold=False, chain=chain)
        pre_b, post_b = algorithmic_bytes(n, C, M)
        t = r["t_pre"] + r["t_post"]
        out[key] = {"n": n, "C": C, "tokens": M, "ssq_chain": r["chain"],
                    "pre_ms": round(r["t_pre"], 5), "post_ms": round(r["t_post"], 5),
                    "pre_GBps": round(pre_b / (r["t_pre"] * 1e-3) / 1e9, 1),
                    "post_GBps": round(post_b / (r["t_post"] * 1e-3) / 1e9, 1),
                    "step_frac": round((pre_b + post_b) / (t * 1e-3) / 1e9 / HBM_PEAK_GBS, 4),
                    "tokens_per_s": round(M / (t * 1e-3), 1)}
    return out


REFERENCE_BENCH_SHAPES = ((4, 512, 4, 256), (4, 1024, 4, 512), (2, 2048, 8, 512))


def reference_bench_shapes(warmup: int = 10, runs: int = 50):
    """The reference's own speed workloads (model/mhc_fused.py:1028-1077 with
    the shapes of :1103-1108): one MHCConnection_Fused (bf16, default
    constructor, so 10 Sinkhorn iterations) around a sublayer MLP
    C -> 4C -> C (SiLU, no bias), loss out.float().pow(2).mean(), forward +
    backward, gradients cleared after each step; `runs` steps bracketed by one
    event pair after `warmup`, as the reference times them.  `mhc_only` is the
    same step with the identity as the sublayer (the connection's own forward
    and backward launches, plus the loss).  tokens_per_s = B * L / step."""
    import torch
    import torch.nn as nn
    from model.mhc_fused import MHCConnection_Fused

    dev = torch.device("cuda:0")
    out = {}
    for B, L, n, C in REFERENCE_BENCH_SHAPES:
        torch.manual_seed(0)
        mlp = nn.Sequential(nn.Linear(C, 4 * C, bias=False), nn.SiLU(),
                            nn.Linear(4 * C, C, bias=False)).to(dev).to(torch.bfloat16)
        mhc = MHCConnection_Fused(n, C).to(dev).to(torch.bfloat16)
        x_t = torch.randn(B, L, n * C, device=dev).to(torch.bfloat16)
        params = list(mhc.parameters()) + list(mlp.parameters())
        res = {"B": B, "L": L, "n": n, "C": C}
        for key, fn in (("with_mlp", mlp), ("mhc_only", lambda z: z)):
            def one():
                x = x_t.clone().requires_grad_(True)
                loss = mhc(x, fn).float().pow(2).mean()
                loss.backward()
                for p_ in params:
                    p_.grad = None
            for _ in range(warmup):
                one()
            _sync()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            e0.record()
            for _ in range(runs):
                one()
            e1.record()
            _sync()
            ms = e0.elapsed_time(e1) / runs
            res[key] = {"ms_per_step": round(ms, 4), "tokens_per_s": round(B * L / (ms * 1e-3), 1)}
        out[f"B{B}_L{L}_n{n}_C{C}"] = res
    return out


def _dense_config(**kw):
    from model.model_minimind import MiniMindConfig
    base = dict(hidden_size=768, num_hidden_layers=8, num_attention_heads=8, num_key_value_heads=4,
                head_dim=96, intermediate_size=2048, rope_theta=1e6, vocab_size=6400, use_mhc=1,
                mhc_residual_expansion=4, max_position_embeddings=4096)
    base.update(kw)
    return MiniMindConfig(**base)


def e2e_decode(steps: int = 30, warmup: int = 5, batch: int = 64, kv_len: int = 2048):
    """the config-3 model decoding one token per sequence
    per step for 64 sequences over a KV cache of 2048 positions per layer,
    filled with seeded N(0, 1) bf16.  Greedy: each step's ids are the argmax
    of the previous step's logits, kept on the device (no host sync inside
    the timed loop).  The cache is held at 2048 entries (each step's new K/V
    is not appended), so every step does the same work.

    Two timings: eager (one host launch per op) and the same step captured
    once in a HIP graph and replayed (torch.cuda.CUDAGraph), which removes
    the host launch cost that dominates at 64 tokens.  `graph_vs_eager`
    compares the graph's ids and logits with the eager run's over the same
    steps."""
    import torch
    from model.model_minimind import MiniMindForCausalLM, init_normal_

    dev = torch.device("cuda:0")
    cfg = _dense_config()
    torch.manual_seed(0)
    model = init_normal_(MiniMindForCausalLM(cfg)).to(torch.bfloat16).to(dev).eval()
    g = torch.Generator().manual_seed(3)
    kv = []
    for _ in range(cfg.num_hidden_layers):
        shape = (batch, kv_len, cfg.num_key_value_heads, cfg.head_dim)
        kv.append((torch.randn(shape, generator=g).to(torch.bfloat16).to(dev),
                   torch.randn(shape, generator=g).to(torch.bfloat16).to(dev)))
    ids0 = torch.randint(0, cfg.vocab_size, (batch, 1), generator=g).to(dev)

    def step(ids):
        logits = model(ids, past_key_values=kv, use_cache=False).logits
        return logits, logits[:, -1].argmax(-1, keepdim=True)

    res = {}
    with torch.inference_mode():
        ids = ids0.clone()
        for _ in range(warmup):
            _, ids = step(ids)
        _sync()
        ids = ids0.clone()
        eager_ids = []
        t0 = time.perf_counter()
        for _ in range(steps):
            logits, ids = step(ids)
            eager_ids.append(ids)
        _sync()
        dt = (time.perf_counter() - t0) / steps
        eager_last = logits.float()
        res["eager"] = {"ms_per_step": round(dt * 1e3, 4),
                        "tokens_per_s": round(batch / dt, 1)}

        static_ids = ids0.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(3):
                step(static_ids)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_logits, nxt = step(static_ids)
            static_ids.copy_(nxt)
        static_ids.copy_(ids0)
        for _ in range(warmup):
            graph.replay()
        _sync()
        static_ids.copy_(ids0)
        graph_ids = []
        t0 = time.perf_counter()
        for _ in range(steps):
            graph.replay()
            graph_ids.append(static_ids.clone())
        _sync()
        dt = (time.perf_counter() - t0) / steps
        res["hip_graph"] = {"ms_per_step": round(dt * 1e3, 4),
                            "tokens_per_s": round(batch / dt, 1)}
        same = all(torch.equal(a_, b_) for a_, b_ in zip(eager_ids, graph_ids))
        res["graph_vs_eager"] = {"ids_equal": bool(same),
                                 "logits_max_abs_diff": float((static_logits.float()
                                                               - eager_last).abs().max())}
    res["value"] = res["hip_graph"]["tokens_per_s"]
    res["unit"] = "tokens/s"
    res["config"] = (f"C4: config-3 model, batch {batch}, 1 token per sequence per step, KV cache "
                     f"{kv_len} per layer (N(0,1) bf16, held fixed), greedy ids on device")
    return res


def e2e_prefill_moe(steps: int = 3, warmup: int = 1):
    """8 layers, hidden 768, n = 8 streams (phi [6144, 80],
    8x8 Sinkhorn, 20 iterations), FFN = 8 routed SwiGLU experts of
    intermediate 1024, top-2 softmax routing, no shared expert; N(0, 0.02)
    init, bf16; prefill B=4, T=2048.  The expert dispatch is the reference's
    own loop over experts (a host sync per expert), timed as is."""
    import torch
    from model.model_minimind import MiniMindForCausalLM, init_normal_

    dev = torch.device("cuda:0")
    cfg = _dense_config(mhc_residual_expansion=8, use_moe=True, num_experts=8,
                        num_experts_per_tok=2, moe_intermediate_size=1024)
    torch.manual_seed(0)
    model = init_normal_(MiniMindForCausalLM(cfg)).to(torch.bfloat16).to(dev).eval()
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, cfg.vocab_size, (4, 2048), generator=g).to(dev)
    with torch.inference_mode():
        for _ in range(warmup):
            model(ids)
        _sync()
        t0 = time.perf_counter()
        for _ in range(steps):
            model(ids)
        _sync()
    dt = (time.perf_counter() - t0) / steps
    return {"value": round(ids.numel() / dt, 1), "unit": "tokens/s",
            "ms_per_forward": round(dt * 1e3, 3),
            "config": "C5: 8 layers, hidden 768, 8q/4kv heads, head_dim 96, n=8, 8 experts top-2, "
                      "expert intermediate 1024, vocab 6400, bf16, B=4 T=2048"}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-e2e", action="store_true")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--traffic", action="store_true",
                    help="run the counter-calibration and config-2 launches once, print nothing")
    ap.add_argument("--vector-pre", action="store_true",
                    help="with --traffic: also run the pre phase on the generic VALU kernel")
    ap.add_argument("--e2e-only", nargs="?", const="all", default=None,
                    choices=["all", "prefill", "decode", "moe"],
                    help="run only the end-to-end model figures (configs 3, 4, 5, or one of "
                         "them) and print them as one JSON line")
    ap.add_argument("--section", choices=["fp32-layout", "other-configs", "reference-shapes",
                                          "backward"],
                    default=None,
                    help="run only the fp32-layout launches or the isolated config-4 / config-5 "
                         "kernel pairs and print them as one JSON line (for profiler runs)")
    ap.add_argument("--mfma-kernels", action="store_true",
                    help="with --traffic: also run the config-2 backward MFMA kernels and the "
                         "config-5 (n = 8) pre phase, with and without the handed-over sums "
                         "of squares")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (the mHC forward is per-token and "
              f"shards by tokens with no exchange); --gpus {args.gpus} is not run.", file=sys.stderr)
        sys.exit(2)

    import torch
    if not torch.cuda.is_available():
        print("bench.py: no ROCm GPU visible", file=sys.stderr)
        sys.exit(1)

    if args.traffic:
        traffic_passes(args.vector_pre, args.mfma_kernels)
        return
    if args.section == "fp32-layout":
        print(json.dumps({"fp32_layout": bench_layout32(), "fp32_layout_c5": layout32_c5()}),
              flush=True)
        return
    if args.section == "backward":
        bw5 = bench_backward(n=8, M=8192)
        bw5["config"] = "C5 shape: 8192 tokens, n=8, C=768, bf16"
        print(json.dumps({"backward": bench_backward(), "backward_c5": bw5,
                          "head_backward": bench_head_backward()}), flush=True)
        return
    if args.section == "reference-shapes":
        print(json.dumps({"reference_bench_shapes": reference_bench_shapes()}), flush=True)
        return
    if args.section == "other-configs":
        print(json.dumps({"other_configs": isolated_configs(max(10, args.steps // 2),
                                                            max(3, args.warmup // 2))}), flush=True)
        return
    if args.e2e_only:
        runs = {"prefill": ("e2e_prefill", e2e_prefill), "decode": ("e2e_decode", e2e_decode),
                "moe": ("e2e_prefill_moe", e2e_prefill_moe)}
        keys = list(runs) if args.e2e_only == "all" else [args.e2e_only]
        print(json.dumps({runs[k][0]: runs[k][1]() for k in keys}), flush=True)
        return

    r, rc = bench_mhc(args.steps, args.warmup)
    pre_b, post_b = algorithmic_bytes(N_STREAMS, C_DIM, TOKENS)
    step_ms = r["t_pre"] + r["t_post"]
    value = TOKENS / (step_ms * 1e-3)
    post_gbs = post_b / (r["t_post"] * 1e-3) / 1e9
    pre_gbs = pre_b / (r["t_pre"] * 1e-3) / 1e9
    total_gbs = (pre_b + post_b) / (step_ms * 1e-3) / 1e9
    c_ms = rc["t_pre"] + rc["t_post"]
    tr = read_traffic()
    line = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(step_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "C2: isolated mHC fwd (pre+Sinkhorn kernel, post kernel), "
                               "16384 tok (B=16,T=1024), n=4, C=768, bf16, F fixed N(0,1)",
                   "tokens": TOKENS, "n": N_STREAMS, "C": C_DIM, "sinkhorn_iters": ITERS,
                   "parallelism": "single GPU",
                   "timing": "steady state over 8 rotating input sets, HIP events per kernel"},
        "roofline": {"bound": "hbm",
                     "kernel": "one mHC forward step: pre_persist_kernel (RMS + projection + gates "
                               "+ Sinkhorn + pre-aggregate) then post_vec_kernel (res-mix + "
                               "post-expand)",
                     "achieved": round(total_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(total_gbs / HBM_PEAK_GBS, 4),
                     "traffic": (round(tr["pre_fetch"] + tr["pre_write"] + tr["post_fetch"]
                                       + tr["post_write"]) if tr else None),
                     "algorithmic_bytes_per_launch": pre_b + post_b},
        "post_roofline": {"bound": "hbm", "kernel": "post_vec_kernel (res-mix + post-expand)",
                          "achieved": round(post_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                          "frac": round(post_gbs / HBM_PEAK_GBS, 4),
                          "traffic": round(tr["post_fetch"] + tr["post_write"]) if tr else None,
                          "algorithmic_bytes_per_launch": post_b},
        "pre_roofline": {"bound": "hbm", "kernel": "pre_persist_kernel (RMS + projection + gates "
                                                   "+ Sinkhorn + pre-aggregate)",
                         "achieved": round(pre_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(pre_gbs / HBM_PEAK_GBS, 4),
                         "traffic": round(tr["pre_fetch"] + tr["pre_write"]) if tr else None,
                         "algorithmic_bytes_per_launch": pre_b},
        "pre_mfma": {"flops_per_launch": 2 * TOKENS * N_STREAMS * C_DIM * 32,
                     "achieved_tflops": round(2 * TOKENS * N_STREAMS * C_DIM * 32 / (r["t_pre"] * 1e-3) / 1e12, 1),
                     "peak_tflops": 2500.0,
                     "frac": round(2 * TOKENS * N_STREAMS * C_DIM * 32 / (r["t_pre"] * 1e-3) / 2.5e15, 4),
                     "source": "flops from SQ_INSTS_VALU_MFMA_MOPS_BF16 x 512 "
                               "(profiles/mfma_util_and_traffic.txt), time from this run"},
        "kernels": {"pre_ms": round(r["t_pre"], 5), "post_ms": round(r["t_post"], 5),
                    "pre_min_ms": round(r["t_pre_min"], 5), "post_min_ms": round(r["t_post_min"], 5),
                    "pre_GBps": round(pre_gbs, 1), "post_GBps": round(post_gbs, 1),
                    "pre_bytes": pre_b, "post_bytes": post_b},
        "cold_clean_cache": {"pre_ms": round(rc["t_pre"], 5), "post_ms": round(rc["t_post"], 5),
                             "tokens_per_s": round(TOKENS / (c_ms * 1e-3), 1)},
        "hbm_calibration": hbm_calibration(),
    }
    bw = bench_backward()
    bw["fwd_bwd_tokens_per_s"] = round(TOKENS / ((step_ms + bw["total_ms"]) * 1e-3), 1)
    line["backward"] = bw
    bw5 = bench_backward(n=8, M=8192)
    bw5["config"] = "C5 shape: 8192 tokens, n=8, C=768, bf16"
    line["backward_c5"] = bw5
    line["head_backward"] = bench_head_backward()
    line["fp32_layout"] = bench_layout32()
    line["fp32_layout_c5"] = layout32_c5()
    line["other_configs"] = isolated_configs(max(10, args.steps // 2), max(3, args.warmup // 2))
    line["reference_bench_shapes"] = reference_bench_shapes()
    if not args.no_e2e:
        line["e2e_prefill"] = e2e_prefill()
        line["e2e_decode"] = e2e_decode()
        line["e2e_prefill_moe"] = e2e_prefill_moe()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
