"""Drop-in API checks (CPU): constructor signatures, parameter names and shapes,
state-dict layout of the model, and the absence of any CPU forward path."""
from __future__ import annotations

import inspect

import pytest
import torch

from model.mhc_common import MHCHead, StreamExpand
from model.mhc_fused import MHCConnection_Fused, sinkhorn_normalize
from model.mhc_fused_no_hres import MHCConnection_FusedNoHres


def _sig(f):
    return [(p.name, p.default) for p in inspect.signature(f).parameters.values()]


def test_constructor_signatures_match_reference():
    # model/mhc_fused.py:780-782
    assert _sig(MHCConnection_Fused.__init__) == [
        ("self", inspect._empty), ("n", inspect._empty), ("dim", inspect._empty),
        ("alpha_init", 0.01), ("sinkhorn_iters", 10), ("post_mult_value", 2.0),
        ("eps", 1e-6), ("pre_eps", 1e-6), ("sinkhorn_eps", 1e-6)]
    # model/mhc_fused_no_hres.py:589-591
    assert _sig(MHCConnection_FusedNoHres.__init__) == [
        ("self", inspect._empty), ("n", inspect._empty), ("dim", inspect._empty),
        ("alpha_init", 0.01), ("post_mult_value", 2.0), ("eps", 1e-6), ("pre_eps", 1e-6)]
    # model/mhc_common.py:414-415, :110
    assert _sig(MHCHead.__init__) == [
        ("self", inspect._empty), ("n", inspect._empty), ("dim", inspect._empty),
        ("alpha_init", 0.01), ("eps", 1e-6), ("pre_eps", 1e-6)]
    assert _sig(StreamExpand.__init__) == [("self", inspect._empty), ("n", inspect._empty),
                                           ("dim", inspect._empty)]
    # model/mhc_fused.py:141
    assert _sig(sinkhorn_normalize) == [("M", inspect._empty), ("iters", 10), ("eps", 1e-6)]
    # reference forward(x_flat, sublayer_fn) (model/mhc_fused.py:817); the
    # additions are optional trailing in_norm / chain (default None: the
    # reference call)
    for cls in (MHCConnection_Fused, MHCConnection_FusedNoHres):
        assert _sig(cls.forward)[1:] == [("x_flat", inspect._empty),
                                         ("sublayer_fn", inspect._empty), ("in_norm", None),
                                         ("chain", None)]
    assert _sig(MHCHead.forward)[1:] == [("x_flat", inspect._empty), ("out_norm", None),
                                         ("chain", None)]


def test_parameters_match_reference():
    m = MHCConnection_Fused(4, 768)
    shapes = {k: tuple(v.shape) for k, v in m.named_parameters()}
    assert shapes == {"phi_weight": (3072, 24), "alpha_pre": (), "bias_pre": (4,),
                      "alpha_post": (), "bias_post": (4,), "alpha_res": (), "bias_res": (4, 4)}
    assert torch.equal(m.bias_res, torch.eye(4)) and m.alpha_pre.item() == pytest.approx(0.01)
    # kaiming_uniform_(a=sqrt(5)) on (nC, FD): bound 1/sqrt(FD)
    assert m.phi_weight.abs().max().item() <= 1 / 24 ** 0.5
    m2 = MHCConnection_FusedNoHres(8, 768)
    assert {k: tuple(v.shape) for k, v in m2.named_parameters()} == {
        "phi_weight": (6144, 16), "alpha_pre": (), "bias_pre": (8,), "alpha_post": (), "bias_post": (8,)}
    h = MHCHead(4, 768)
    assert {k: tuple(v.shape) for k, v in h.named_parameters()} == {
        "phi_weight": (3072, 4), "bias": (4,), "alpha": (1,)}
    with pytest.raises(AssertionError):
        MHCConnection_Fused(3, 64)
    with pytest.raises(AssertionError):
        MHCConnection_Fused(4, 64, post_mult_value=1.0)


def test_model_state_dict_keys():
    from model.model_minimind import MiniMindConfig, MiniMindForCausalLM
    cfg = MiniMindConfig(hidden_size=64, num_hidden_layers=2, num_attention_heads=4,
                         num_key_value_heads=2, head_dim=16, intermediate_size=128,
                         vocab_size=100, use_mhc=1, mhc_residual_expansion=4,
                         max_position_embeddings=64)
    sd = MiniMindForCausalLM(cfg).state_dict()
    for k, shape in {"model.layers.1.attn_mhc.phi_weight": (256, 24),
                     "model.layers.0.mlp_mhc.bias_res": (4, 4),
                     "model.norm.0.phi_weight": (256, 4), "model.norm.0.alpha": (1,),
                     "model.norm.0.bias": (4,), "model.embed_up_norm.0.weight": (64,),
                     "model.norm.1.weight": (64,)}.items():
        assert tuple(sd[k].shape) == shape, k


def test_no_cpu_forward_path():
    m = MHCConnection_Fused(4, 64)
    x = torch.randn(1, 3, 256)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        m(x, lambda z: z)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        MHCConnection_FusedNoHres(4, 64)(x, lambda z: z)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        MHCHead(4, 64)(x)
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        sinkhorn_normalize(torch.randn(2, 4, 4))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        StreamExpand(4, 64)(torch.randn(1, 3, 64))
