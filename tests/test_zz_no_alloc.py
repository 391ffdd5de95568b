"""mhc_pre_bwd_weights_noalloc (static device scratch, no allocation) against
mhc_pre_bwd_weights (caller workspace), both through the C ABI.

Two calls in a row per case, the second with fewer tokens, so the second call
runs on scratch that still holds the first call's partials.  Where the
scratch holds as many token ranges as the workspace entry point uses, the two
agree bit for bit; where it caps the ranges (wide fp32 rows, many tokens) the
sums group differently and agree to the fp32 bar.
"""
from __future__ import annotations

import pytest
import torch

from _util import maxrel
from model import _hip as H

pytestmark = pytest.mark.gpu

SCRATCH_BYTES = 32 << 20


def _inputs(M, n, C, mode, x_dtype, dev, seed):
    g = torch.Generator().manual_seed(seed)
    FD = {H.MODE_FULL: 2 * n + n * n, H.MODE_NOHRES: 2 * n, H.MODE_HEAD: n}[mode]
    x = torch.randn(M, n * C, generator=g).to(x_dtype).to(dev)
    inv = (torch.rand(M, generator=g) + 0.5).to(dev)
    mixes = torch.randn(M, FD, generator=g).to(dev)
    g_raw = torch.randn(M, FD, generator=g).to(dev)
    alphas = [torch.tensor(v).to(dev) for v in (0.6, 0.4, 0.8)]
    return x, inv, mixes, g_raw, alphas, FD


def _outputs(n, C, FD, phi_dtype, dev):
    return (torch.full((n * C, FD), float("nan"), dtype=phi_dtype, device=dev),
            [torch.full((), float("nan"), device=dev) for _ in range(3)],
            [torch.full((k,), float("nan"), device=dev) for k in (n, n, n * n)])


def _call(lib, noalloc, x, inv, mixes, g_raw, alphas, n, C, mode, phi_dtype, dev):
    M = x.shape[0]
    FD = g_raw.shape[1]
    g_phi, g_a, g_b = _outputs(n, C, FD, phi_dtype, dev)
    if mode == H.MODE_HEAD:
        g_a[1] = g_a[2] = g_b[1] = g_b[2] = None
    elif mode == H.MODE_NOHRES:
        g_a[2] = g_b[2] = None
    common = [x.data_ptr(), H.dtype_tag(x), inv.data_ptr(), mixes.data_ptr(), g_raw.data_ptr(),
              alphas[0].data_ptr(), alphas[1].data_ptr(), alphas[2].data_ptr(), H.DTYPE_F32,
              g_phi.data_ptr(), H.dtype_tag(g_phi),
              H.ptr(g_a[0]), H.ptr(g_b[0]), H.ptr(g_a[1]), H.ptr(g_b[1]), H.ptr(g_a[2]),
              H.ptr(g_b[2])]
    stream = H.stream(dev)
    if noalloc:
        rc = lib.mhc_pre_bwd_weights_noalloc(*common, M, n, C, mode, stream)
        H.check(rc, "mhc_pre_bwd_weights_noalloc")
    else:
        nbytes = lib.mhc_pre_bwd_weights_workspace_bytes(M, n, C, mode)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        rc = lib.mhc_pre_bwd_weights(*common, ws.data_ptr(), nbytes, M, n, C, mode, stream)
        H.check(rc, "mhc_pre_bwd_weights")
    torch.cuda.synchronize()
    return g_phi, g_a, g_b


# (x dtype, phi dtype, n, C, mode, first M, second M, bit-exact)
CASES = [
    (torch.bfloat16, torch.bfloat16, 4, 768, H.MODE_FULL, 16384, 1000, True),   # MFMA kernel
    (torch.bfloat16, torch.float32, 8, 768, H.MODE_FULL, 8192, 300, True),      # MFMA, FD 80
    (torch.bfloat16, torch.bfloat16, 4, 256, H.MODE_HEAD, 5000, 17, True),
    (torch.float32, torch.float32, 4, 256, H.MODE_NOHRES, 3000, 65, True),      # generic kernel
    # generic kernel, 24 ranges wanted at 6000 tokens, (6144 * 80 + 160) * 4 B per range: the
    # scratch holds 17, so the token sums group differently
    (torch.float32, torch.float32, 8, 768, H.MODE_FULL, 6000, 2000, False),
]


@pytest.mark.parametrize("x_dt,phi_dt,n,C,mode,M1,M2,exact", CASES)
def test_noalloc_matches_workspace_entry(dev, x_dt, phi_dt, n, C, mode, M1, M2, exact):
    lib = H.load()
    for seed, M in ((1, M1), (2, M2)):
        print(f"noalloc case x={x_dt} phi={phi_dt} n={n} C={C} mode={mode} M={M}", flush=True)
        x, inv, mixes, g_raw, alphas, FD = _inputs(M, n, C, mode, x_dt, dev, seed)
        ref = _call(lib, False, x, inv, mixes, g_raw, alphas, n, C, mode, phi_dt, dev)
        got = _call(lib, True, x, inv, mixes, g_raw, alphas, n, C, mode, phi_dt, dev)
        pairs = [(ref[0], got[0])] + [(r, q) for r, q in zip(ref[1] + ref[2], got[1] + got[2])
                                      if r is not None]
        for r, q in pairs:
            assert not torch.isnan(q).any()
            if exact:
                assert torch.equal(r, q)
            else:
                assert maxrel(r, q) <= 1e-5


def test_noalloc_rejects_oversized_rows(dev):
    lib = H.load()
    n, C = 16, 2048                      # (32768 * 288 + 576) * 4 B > 32 MiB
    assert (n * C * (2 * n + n * n) + 2 * (2 * n + n * n)) * 4 > SCRATCH_BYTES
    # Null data pointers: should the size check ever regress, the host-side
    # null check still refuses the call (and the message assertion fails)
    # instead of a launch on buffers far smaller than the shape.
    rc = lib.mhc_pre_bwd_weights_noalloc(None, H.DTYPE_F32, None, None, None, None, None, None,
                                         H.DTYPE_F32, None, H.DTYPE_F32, None, None, None,
                                         None, None, None, 4, n, C, H.MODE_FULL, H.stream(dev))
    assert rc != 0
    assert "scratch" in lib.mhc_last_error().decode()


def test_noalloc_captured_in_hip_graph(dev):
    """The noalloc entry point captured in a HIP graph (the callers it is for)
    and replayed three times, with eager calls between the replays that
    overwrite the scratch; every replay equals the workspace entry point's
    eager result bit for bit."""
    lib = H.load()                       # runs mhc_init: scratch addresses set up before capture
    n, C, mode, M = 4, 768, H.MODE_FULL, 4096
    x, inv, mixes, g_raw, alphas, FD = _inputs(M, n, C, mode, torch.bfloat16, dev, 11)
    ref = _call(lib, False, x, inv, mixes, g_raw, alphas, n, C, mode, torch.bfloat16, dev)
    g_phi, g_a, g_b = _outputs(n, C, FD, torch.bfloat16, dev)
    args = [x.data_ptr(), H.dtype_tag(x), inv.data_ptr(), mixes.data_ptr(), g_raw.data_ptr(),
            alphas[0].data_ptr(), alphas[1].data_ptr(), alphas[2].data_ptr(), H.DTYPE_F32,
            g_phi.data_ptr(), H.dtype_tag(g_phi),
            g_a[0].data_ptr(), g_b[0].data_ptr(), g_a[1].data_ptr(), g_b[1].data_ptr(),
            g_a[2].data_ptr(), g_b[2].data_ptr(), M, n, C, mode]
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):        # one uncaptured call first, as torch's capture docs ask
        H.check(lib.mhc_pre_bwd_weights_noalloc(*args, H.stream(dev)), "noalloc warm-up")
    torch.cuda.current_stream(dev).wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    rcs = []
    with torch.cuda.graph(graph):
        rcs.append(lib.mhc_pre_bwd_weights_noalloc(*args, H.stream(dev)))
    assert rcs == [0], lib.mhc_last_error().decode()
    other = _inputs(1000, n, C, mode, torch.bfloat16, dev, 12)
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        # eager work between replays: another call fills the scratch with
        # other partials, and the outputs are reset
        _call(lib, True, *other[:5], n, C, mode, torch.bfloat16, dev)
        for t in [g_phi] + g_a + g_b:
            t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(ref[0], g_phi)
        for r, q in zip(ref[1] + ref[2], g_a + g_b):
            assert torch.equal(r, q)
