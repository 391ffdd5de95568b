"""The MiniMind-mHC decoder on the GPU (every mHC piece on the HIP kernels)
against the same weights on the CPU with every mHC piece replaced by the
oracle (model/model_minimind.py:300-403 is the call structure both follow);
the KV-cache decode path against a full prefill; and the decode step captured
in a HIP graph against eager execution, replay after replay."""
from __future__ import annotations

import types

import pytest
import torch

from oracle import mhc_ref as R

pytestmark = pytest.mark.gpu

from model.mhc_common import MHCHead, StreamExpand  # noqa: E402
from model.mhc_fused import MHCConnection_Fused  # noqa: E402
from model.mhc_fused_no_hres import MHCConnection_FusedNoHres  # noqa: E402
from model.model_minimind import MiniMindConfig, MiniMindForCausalLM, init_normal_  # noqa: E402


def _config(use_mhc: int, n: int, moe: bool = False) -> MiniMindConfig:
    return MiniMindConfig(hidden_size=64, num_hidden_layers=2, num_attention_heads=4,
                          num_key_value_heads=2, head_dim=16, intermediate_size=128,
                          vocab_size=128, use_mhc=use_mhc, mhc_residual_expansion=n,
                          max_position_embeddings=256, use_moe=moe, num_experts=4,
                          num_experts_per_tok=2, moe_intermediate_size=64)


def _model(cfg: MiniMindConfig, seed: int = 0) -> MiniMindForCausalLM:
    torch.manual_seed(seed)
    m = init_normal_(MiniMindForCausalLM(cfg))
    # gates away from their init values, so the projection drives every gate
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():
        for name, p in m.named_parameters():
            leaf = name.rsplit(".", 1)[-1]
            if leaf.startswith("alpha"):
                p.fill_(0.5)
            elif leaf.startswith("bias"):
                p.add_(torch.randn(p.shape, generator=g) * 0.3)
            elif leaf == "phi_weight":
                p.normal_(0.0, 0.1, generator=g)
    return m.eval()


def _with_norm(f, norm):
    """F(z) = f(norm(z)): the reference's sublayer closure (model/model_minimind.py:326-336)."""
    return f if norm is None else (lambda z: f(norm(z)))


def _oracle_copy(model: MiniMindForCausalLM) -> MiniMindForCausalLM:
    """Same weights, fp32 on the CPU, every mHC module's forward the oracle's
    (the norms handed to the mHC modules applied as separate torch ops, in the
    reference's order)."""
    ref = MiniMindForCausalLM(model.config)
    ref.load_state_dict({k: v.detach().float().cpu() for k, v in model.state_dict().items()})
    for mod in ref.modules():
        if isinstance(mod, MHCConnection_Fused):
            def fwd(self, x, f, in_norm=None, chain=None):
                return R.mhc_full_forward(x, R.module_params(self), _with_norm(f, in_norm), self.n,
                                          self.dim, eps=self.eps, pre_eps=self.pre_eps,
                                          post_mult=self.post_mult_value,
                                          sinkhorn_iters=self.sinkhorn_iters,
                                          sinkhorn_eps=self.sinkhorn_eps)["out"]
            mod.forward = types.MethodType(fwd, mod)
        elif isinstance(mod, MHCConnection_FusedNoHres):
            def fwd(self, x, f, in_norm=None, chain=None):
                return R.mhc_nohres_forward(x, R.module_params(self), _with_norm(f, in_norm),
                                            self.n, self.dim, eps=self.eps, pre_eps=self.pre_eps,
                                            post_mult=self.post_mult_value)["out"]
            mod.forward = types.MethodType(fwd, mod)
        elif isinstance(mod, MHCHead):
            def fwd(self, x, out_norm=None, chain=None):
                out = R.head(x, R.module_params(self), self.n, self.dim, pre_eps=self.pre_eps,
                             rms_eps=self.eps)
                return out if out_norm is None else out_norm(out)
            mod.forward = types.MethodType(fwd, mod)
        elif isinstance(mod, StreamExpand):
            mod.forward = types.MethodType(lambda self, x: R.stream_expand(x, self.n), mod)
    return ref.eval()


def _rel(a: torch.Tensor, b: torch.Tensor) -> float:
    a, b = a.float().cpu(), b.float().cpu()
    return float((a - b).abs().max() / b.abs().max().clamp_min(1e-30))


@pytest.mark.parametrize("use_mhc,n,moe", [(1, 4, False), (2, 4, False), (1, 8, True),
                                           (1, 2, False), (2, 1, False)])
def test_model_logits_vs_oracle_connections(dev, use_mhc, n, moe):
    cfg = _config(use_mhc, n, moe)
    model = _model(cfg)
    ref = _oracle_copy(model)
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, cfg.vocab_size, (2, 24), generator=g)
    with torch.no_grad():
        want = ref(ids).logits
        got = model.to(dev)(ids.to(dev)).logits
    # fp32 end to end; GEMM / attention summation order differs between the
    # GPU libraries and the CPU, so the bar is 1e-4 of the largest logit
    assert _rel(got, want) < 1e-4, (use_mhc, n, moe, _rel(got, want))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_with_cache_matches_prefill(dev, dtype):
    """Logits of the last position: one prefill of T+1 tokens against a
    prefill of T tokens followed by a one-token decode step over its cache
    (the mHC connections then run at M = batch)."""
    cfg = _config(1, 4)
    model = _model(cfg).to(dtype).to(dev)
    g = torch.Generator().manual_seed(6)
    ids = torch.randint(0, cfg.vocab_size, (3, 17), generator=g).to(dev)
    with torch.no_grad():
        full = model(ids).logits[:, -1]
        pre = model(ids[:, :-1], use_cache=True)
        step = model(ids[:, -1:], past_key_values=pre.past_key_values, use_cache=True).logits[:, -1]
        assert pre.past_key_values[0][0].shape[1] == 16
    bar = 1e-4 if dtype == torch.float32 else 3e-2
    assert _rel(step, full) < bar, _rel(step, full)


def test_decode_step_hip_graph_replays_match_eager(dev):
    """The decode step (mHC kernels, attention over a fixed cache, greedy
    argmax fed back into the ids buffer) captured once and replayed: every
    replay's logits and ids equal the eager step's, with eager work and
    synchronisations between the replays."""
    cfg = _config(1, 4)
    model = _model(cfg).to(torch.bfloat16).to(dev)
    g = torch.Generator().manual_seed(7)
    B, T = 8, 40
    kv = [(torch.randn(B, T, cfg.num_key_value_heads, cfg.head_dim, generator=g)
           .to(torch.bfloat16).to(dev),
           torch.randn(B, T, cfg.num_key_value_heads, cfg.head_dim, generator=g)
           .to(torch.bfloat16).to(dev)) for _ in range(cfg.num_hidden_layers)]
    ids0 = torch.randint(0, cfg.vocab_size, (B, 1), generator=g).to(dev)

    def step(ids):
        logits = model(ids, past_key_values=kv, use_cache=False).logits
        return logits, logits[:, -1].argmax(-1, keepdim=True)

    with torch.inference_mode():
        ids = ids0.clone()
        eager = []
        for _ in range(4):
            logits, ids = step(ids)
            eager.append((logits.clone(), ids.clone()))
        static_ids = ids0.clone()
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                step(static_ids)
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            static_logits, nxt = step(static_ids)
            static_ids.copy_(nxt)
        static_ids.copy_(ids0)
        for r in range(4):
            graph.replay()
            torch.cuda.synchronize()
            want_logits, want_ids = eager[r]
            assert torch.equal(static_ids, want_ids), r
            assert _rel(static_logits, want_logits) < 1e-6, (r, _rel(static_logits, want_logits))
            step(ids0)  # eager work between replays
            torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("use_mhc,n", [(1, 4), (2, 4), (1, 8), (1, 1)])
def test_fused_norm_path_matches_autograd_path(dev, dtype, use_mhc, n):
    """Without autograd the norms next to the mHC pieces run inside their
    launches; with autograd they are separate ops.  Same logits."""
    cfg = _config(use_mhc, n)
    model = _model(cfg).to(dtype).to(dev)
    g = torch.Generator().manual_seed(8)
    ids = torch.randint(0, cfg.vocab_size, (2, 40), generator=g).to(dev)
    with torch.no_grad():
        fused = model(ids).logits
    split = model(ids).logits.detach()  # parameters require grad: the autograd path
    bar = 1e-4 if dtype == torch.float32 else 3e-2
    assert _rel(fused, split) < bar, _rel(fused, split)
