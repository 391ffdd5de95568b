"""The modules' autograd Functions see the caller's grad mode: under
torch.no_grad() / inference_mode they save nothing, ask the kernels for no
backward-only outputs and keep cached weight images, even when the parameters
require grad (ctx.needs_input_grad alone is True there).  CPU only: the
Functions' bookkeeping, not the kernels."""
from __future__ import annotations

import torch

from model import _ops


class _Probe(_ops.GradAwareFunction):
    seen = []

    @staticmethod
    def forward(ctx, x, w):
        _Probe.seen.append((_ops.grad_wanted(ctx), _ops.grad_wanted(ctx, 0), _ops.grad_wanted(ctx, 1)))
        return x * w

    @staticmethod
    def backward(ctx, g):
        return g, g


def test_grad_wanted_follows_the_callers_grad_mode():
    x = torch.ones(3)
    w = torch.ones(3, requires_grad=True)
    _Probe.seen.clear()
    _Probe.apply(x, w)
    with torch.no_grad():
        _Probe.apply(x, w)
    with torch.inference_mode():
        _Probe.apply(x, w)
    _Probe.apply(x, w.detach())
    assert _Probe.seen == [(True, False, True), (False, False, False), (False, False, False),
                           (False, False, False)]


def test_grad_mode_restored_after_nested_and_failing_calls():
    class _Boom(_ops.GradAwareFunction):
        @staticmethod
        def forward(ctx, x):
            raise RuntimeError("boom")

        @staticmethod
        def backward(ctx, g):
            return g

    w = torch.ones(2, requires_grad=True)
    with torch.no_grad():
        try:
            _Boom.apply(w)
        except RuntimeError:
            pass
    _Probe.seen.clear()
    _Probe.apply(torch.ones(2), w)
    assert _Probe.seen == [(True, False, True)]
