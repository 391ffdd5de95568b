"""Checkpoint compatibility (CPU): the model's state dict has exactly the
reference model's keys, in the reference's registration order, with its
shapes; a checkpoint written the way the reference trainer writes one
(every tensor .half().cpu(), torch.save to a .pth, trainer/trainer_utils.py:63-73)
loads back with strict=True, and the reference's own non-strict load
(trainer/trainer_utils.py:124-127) reports nothing missing or unexpected."""
from __future__ import annotations

import pytest
import torch

from model.model_minimind import MiniMindConfig, MiniMindForCausalLM


def _config(use_mhc: int, n: int, moe: bool) -> MiniMindConfig:
    return MiniMindConfig(hidden_size=64, num_hidden_layers=2, num_attention_heads=4,
                          num_key_value_heads=2, head_dim=16, intermediate_size=128,
                          vocab_size=100, use_mhc=use_mhc, mhc_residual_expansion=n,
                          max_position_embeddings=64, use_moe=moe, num_experts=3,
                          num_experts_per_tok=2, moe_intermediate_size=48)


def _reference_keys(cfg: MiniMindConfig):
    """(key, shape) in the order the reference modules register parameters.

    Model: model/model_minimind.py:358-374 (embed_tokens, embed_up_norm, layers,
    norm) and :412 (lm_head, tied to embed_tokens).  Block :307-319 (self_attn,
    mlp, attn_in_norm, ffn_in_norm, attn_mhc, mlp_mhc).  Attention :175-180.
    FeedForward :262-264 (gate, down, up).  MoE :274-275.  MHCConnection_Fused
    model/mhc_fused.py:798-809; _FusedNoHres model/mhc_fused_no_hres.py:605-612;
    MHCHead model/mhc_common.py:426-429 (phi_weight, bias, alpha)."""
    D, hd, nq, nkv = cfg.hidden_size, cfg.head_dim, cfg.num_attention_heads, cfg.num_key_value_heads
    n = cfg.mhc_residual_expansion
    keys = [("model.embed_tokens.weight", (cfg.vocab_size, D))]
    if cfg.use_mhc:
        keys.append(("model.embed_up_norm.0.weight", (D,)))

    def ffn(prefix, inter):
        return [(f"{prefix}.gate_proj.weight", (inter, D)), (f"{prefix}.down_proj.weight", (D, inter)),
                (f"{prefix}.up_proj.weight", (inter, D))]

    def conn(prefix):
        fd = 2 * n + (n * n if cfg.use_mhc == 1 else 0)
        out = [(f"{prefix}.phi_weight", (n * D, fd)), (f"{prefix}.alpha_pre", ()),
               (f"{prefix}.bias_pre", (n,)), (f"{prefix}.alpha_post", ()), (f"{prefix}.bias_post", (n,))]
        if cfg.use_mhc == 1:
            out += [(f"{prefix}.alpha_res", ()), (f"{prefix}.bias_res", (n, n))]
        return out

    for i in range(cfg.num_hidden_layers):
        p = f"model.layers.{i}"
        keys += [(f"{p}.self_attn.q_proj.weight", (nq * hd, D)),
                 (f"{p}.self_attn.k_proj.weight", (nkv * hd, D)),
                 (f"{p}.self_attn.v_proj.weight", (nkv * hd, D)),
                 (f"{p}.self_attn.o_proj.weight", (D, nq * hd)),
                 (f"{p}.self_attn.q_norm.weight", (hd,)), (f"{p}.self_attn.k_norm.weight", (hd,))]
        if cfg.use_moe:
            keys.append((f"{p}.mlp.gate.weight", (cfg.num_experts, D)))
            for e in range(cfg.num_experts):
                keys += ffn(f"{p}.mlp.experts.{e}", cfg.moe_intermediate_size)
        else:
            keys += ffn(f"{p}.mlp", cfg.intermediate_size)
        keys += [(f"{p}.attn_in_norm.weight", (D,)), (f"{p}.ffn_in_norm.weight", (D,))]
        if cfg.use_mhc:
            keys += conn(f"{p}.attn_mhc") + conn(f"{p}.mlp_mhc")
    if cfg.use_mhc:
        keys += [("model.norm.0.phi_weight", (n * D, n)), ("model.norm.0.bias", (n,)),
                 ("model.norm.0.alpha", (1,)), ("model.norm.1.weight", (D,))]
    else:
        keys.append(("model.norm.weight", (D,)))
    keys.append(("lm_head.weight", (cfg.vocab_size, D)))
    return keys


CASES = [(1, 4, False), (2, 4, False), (1, 8, True), (2, 2, True), (0, 1, False)]


@pytest.mark.parametrize("use_mhc,n,moe", CASES)
def test_state_dict_keys_order_and_shapes(use_mhc, n, moe):
    cfg = _config(use_mhc, n, moe)
    sd = MiniMindForCausalLM(cfg).state_dict()
    assert [(k, tuple(v.shape)) for k, v in sd.items()] == _reference_keys(cfg)


@pytest.mark.parametrize("use_mhc,n,moe", CASES)
def test_fp16_pth_checkpoint_round_trip(tmp_path, use_mhc, n, moe):
    cfg = _config(use_mhc, n, moe)
    torch.manual_seed(0)
    src = MiniMindForCausalLM(cfg)
    with torch.no_grad():  # move every mHC gate off its init value
        for name, p in src.named_parameters():
            if name.rsplit(".", 1)[-1].startswith(("alpha", "bias")):
                p.add_(torch.randn(p.shape) * 0.1)
    # what lm_checkpoint writes: fp16 CPU tensors, torch.save to <name>.pth
    path = tmp_path / f"full_sft_{cfg.hidden_size}{'_moe' if moe else ''}.pth"
    torch.save({k: v.half().cpu() for k, v in src.state_dict().items()}, path)

    weights = torch.load(path, map_location="cpu", weights_only=True)
    assert all(v.dtype == torch.float16 for v in weights.values())
    dst = MiniMindForCausalLM(cfg)
    res = dst.load_state_dict(weights, strict=False)  # the reference's own load call
    assert not res.missing_keys and not res.unexpected_keys
    MiniMindForCausalLM(cfg).load_state_dict(weights, strict=True)
    for k, v in dst.state_dict().items():
        assert torch.equal(v, src.state_dict()[k].half().float()), k
    # the tied head follows the embedding, as in the reference (:414)
    assert dst.lm_head.weight.data_ptr() == dst.model.embed_tokens.weight.data_ptr()
