"""StreamChain (CPU): the sums of squares recorded for one tensor are handed
only to a call whose input is that very tensor object, of the right shape."""
from __future__ import annotations

import torch

from model import _ops


def test_chain_hands_sums_only_to_the_recorded_tensor():
    n, C, M = 8, 256, 5
    x = torch.zeros(1, M, n * C, dtype=torch.bfloat16)
    ssq = torch.ones(M, C // 128)
    chain = _ops.StreamChain()
    assert chain.take(x, n, C) is None
    assert chain.put(x, ssq) is x
    assert chain.take(x, n, C) is ssq
    assert chain.take(x.view(M, n * C), n, C) is None       # another tensor object
    assert chain.take(x.clone(), n, C) is None
    assert chain.take(x, 4, 2 * C) is None                  # other shape: other partial count
    chain.put(x, None)
    assert chain.take(x, n, C) is None


def test_chain_buffers_only_where_the_sums_are_used():
    # CPU tensors never get a buffer (the kernels run on the GPU)
    chain = _ops.StreamChain()
    assert chain.buffer(torch.zeros(4, 8 * 768, dtype=torch.bfloat16), 8, 768) is None
    assert _ops.ssq_wanted(torch.bfloat16, 8, 768)
    assert _ops.ssq_wanted(torch.bfloat16, 16, 256)
    assert _ops.ssq_wanted(torch.bfloat16, 4, 2048)
    assert not _ops.ssq_wanted(torch.bfloat16, 4, 768)    # formed in registers
    assert not _ops.ssq_wanted(torch.float32, 8, 768)     # bf16 streams only
    assert not _ops.ssq_wanted(torch.bfloat16, 8, 200)    # C % 128 != 0
