"""MiniMind decoder with mHC residual streams: the caller of the mHC kernels.

Restates the reference model (model/model_minimind.py:76-461) as the
end-to-end harness for prefill / decode measurements: same config fields,
module tree and parameter names (so reference state dicts load), with the
sublayers F (attention, SwiGLU FFN, MoE) on PyTorch-ROCm ops and every mHC
piece (StreamExpand, MHCConnection_Fused / _FusedNoHres, MHCHead) on the HIP
kernels of this package.  Attention uses torch SDPA (the reference's second
backend, model/model_minimind.py:208-232); flash-attn is not used.

Differences from the reference, all outside the mHC path:
  * MiniMindConfig is a plain class (no transformers.PretrainedConfig) and
    MiniMindForCausalLM a plain nn.Module (no PreTrainedModel/GenerationMixin);
  * the RoPE tables are computed once at construction (the reference
    recomputes them after meta-device init and pays a host sync per forward,
    model/model_minimind.py:387-389);
  * the norms next to the mHC pieces are handed to them instead of being
    applied inside F: each sublayer's input RMSNorm goes to its connection
    (in_norm), the entry RMSNorm to StreamExpand.forward_normed and the final
    RMSNorm to MHCHead (out_norm).  Without autograd each runs inside the
    neighbouring HIP launch; with autograd they run as separate ops in the
    reference's order (model/model_minimind.py:326-336, :365-370);
  * one StreamChain per forward is passed to every mHC call, so each launch
    that writes the residual stream hands its rows' sums of squares to the
    next pre launch (used at n >= 8 or hidden > 1024).
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch
import torch.nn.functional as F
from torch import nn

from ._ops import StreamChain
from .mhc_common import MHCHead, StreamExpand
from .mhc_fused import MHCConnection_Fused
from .mhc_fused_no_hres import MHCConnection_FusedNoHres


class MiniMindConfig:
    """Fields and defaults of model/model_minimind.py:76-125."""

    model_type = "minimind"

    def __init__(self, hidden_size=1024, num_hidden_layers=24, use_moe=False, use_mhc=0,
                 mhc_residual_expansion=4, **kwargs):
        self.hidden_size = hidden_size
        self.num_hidden_layers = num_hidden_layers
        self.use_moe = use_moe
        self.dropout = kwargs.get("dropout", 0.0)
        self.vocab_size = kwargs.get("vocab_size", 6400)
        self.bos_token_id = kwargs.get("bos_token_id", 1)
        self.eos_token_id = kwargs.get("eos_token_id", 2)
        self.flash_attn = kwargs.get("flash_attn", True)
        self.num_attention_heads = kwargs.get("num_attention_heads", 8)
        self.num_key_value_heads = kwargs.get("num_key_value_heads", 4)
        self.head_dim = kwargs.get("head_dim", self.hidden_size // self.num_attention_heads)
        self.hidden_act = kwargs.get("hidden_act", "silu")
        self.intermediate_size = kwargs.get("intermediate_size",
                                            math.ceil(hidden_size * math.pi / 64) * 64)
        self.max_position_embeddings = kwargs.get("max_position_embeddings", 32768)
        self.rms_norm_eps = kwargs.get("rms_norm_eps", 1e-6)
        self.rope_theta = kwargs.get("rope_theta", 1e6)
        self.tie_word_embeddings = kwargs.get("tie_word_embeddings", True)
        self.inference_rope_scaling = kwargs.get("inference_rope_scaling", False)
        self.rope_scaling = {
            "beta_fast": 32, "beta_slow": 1, "factor": 16,
            "original_max_position_embeddings": 2048, "attention_factor": 1.0, "type": "yarn",
        } if self.inference_rope_scaling else None
        self.num_experts = kwargs.get("num_experts", 4)
        self.num_experts_per_tok = kwargs.get("num_experts_per_tok", 1)
        self.moe_intermediate_size = kwargs.get("moe_intermediate_size", self.intermediate_size)
        self.norm_topk_prob = kwargs.get("norm_topk_prob", True)
        self.router_aux_loss_coef = kwargs.get("router_aux_loss_coef", 5e-4)
        self.use_mhc = use_mhc
        self.mhc_residual_expansion = mhc_residual_expansion
        assert use_mhc in (0, 1, 2), f"use_mhc must be in {{0,1,2}}, got {use_mhc}"
        if use_mhc:
            assert isinstance(mhc_residual_expansion, int) and mhc_residual_expansion >= 1


def precompute_freqs_cis(dim: int, end: int = 32 * 1024, rope_base: float = 1e6,
                         rope_scaling: dict = None):
    """RoPE cos/sin tables with optional YaRN ramp (model/model_minimind.py:132-148)."""
    freqs = 1.0 / (rope_base ** (torch.arange(0, dim, 2)[: dim // 2].float() / dim))
    attn_factor = 1.0
    if rope_scaling is not None:
        orig_max = rope_scaling.get("original_max_position_embeddings", 2048)
        factor = rope_scaling.get("factor", 16)
        beta_fast = rope_scaling.get("beta_fast", 32.0)
        beta_slow = rope_scaling.get("beta_slow", 1.0)
        attn_factor = rope_scaling.get("attention_factor", 1.0)
        if end / orig_max > 1.0:
            def inv_dim(b):
                return (dim * math.log(orig_max / (b * 2 * math.pi))) / (2 * math.log(rope_base))
            low = max(math.floor(inv_dim(beta_fast)), 0)
            high = min(math.ceil(inv_dim(beta_slow)), dim // 2 - 1)
            ramp = torch.clamp((torch.arange(dim // 2).float() - low) / max(high - low, 0.001), 0, 1)
            freqs = freqs * (1 - ramp + ramp / factor)
    t = torch.arange(end)
    freqs = torch.outer(t, freqs).float()
    cos = torch.cat([torch.cos(freqs), torch.cos(freqs)], dim=-1) * attn_factor
    sin = torch.cat([torch.sin(freqs), torch.sin(freqs)], dim=-1) * attn_factor
    return cos, sin


def apply_rotary_pos_emb(q, k, cos, sin, unsqueeze_dim=1):
    def rotate_half(x):
        return torch.cat((-x[..., x.shape[-1] // 2:], x[..., : x.shape[-1] // 2]), dim=-1)
    q_embed = ((q * cos.unsqueeze(unsqueeze_dim)) + (rotate_half(q) * sin.unsqueeze(unsqueeze_dim))).to(q.dtype)
    k_embed = ((k * cos.unsqueeze(unsqueeze_dim)) + (rotate_half(k) * sin.unsqueeze(unsqueeze_dim))).to(k.dtype)
    return q_embed, k_embed


def repeat_kv(x: torch.Tensor, n_rep: int) -> torch.Tensor:
    bs, slen, kvh, hd = x.shape
    if n_rep == 1:
        return x
    return x[:, :, :, None, :].expand(bs, slen, kvh, n_rep, hd).reshape(bs, slen, kvh * n_rep, hd)


class Attention(nn.Module):
    """GQA attention with q/k RMSNorm, RoPE and a (k, v) cache
    (model/model_minimind.py:161-256), evaluated with torch SDPA."""

    def __init__(self, config: MiniMindConfig):
        super().__init__()
        self.num_key_value_heads = config.num_key_value_heads or config.num_attention_heads
        self.n_local_heads = config.num_attention_heads
        self.n_local_kv_heads = self.num_key_value_heads
        self.n_rep = self.n_local_heads // self.n_local_kv_heads
        self.head_dim = config.head_dim
        self.is_causal = True
        D = config.hidden_size
        self.q_proj = nn.Linear(D, config.num_attention_heads * self.head_dim, bias=False)
        self.k_proj = nn.Linear(D, self.num_key_value_heads * self.head_dim, bias=False)
        self.v_proj = nn.Linear(D, self.num_key_value_heads * self.head_dim, bias=False)
        self.o_proj = nn.Linear(config.num_attention_heads * self.head_dim, D, bias=False)
        self.q_norm = nn.RMSNorm(self.head_dim, eps=config.rms_norm_eps)
        self.k_norm = nn.RMSNorm(self.head_dim, eps=config.rms_norm_eps)
        self.dropout = config.dropout

    def forward(self, x, position_embeddings, past_key_value=None, use_cache=False,
                attention_mask=None):
        bsz, seq_len, _ = x.shape
        xq = self.q_proj(x).view(bsz, seq_len, self.n_local_heads, self.head_dim)
        xk = self.k_proj(x).view(bsz, seq_len, self.n_local_kv_heads, self.head_dim)
        xv = self.v_proj(x).view(bsz, seq_len, self.n_local_kv_heads, self.head_dim)
        xq, xk = self.q_norm(xq), self.k_norm(xk)
        cos, sin = position_embeddings
        xq, xk = apply_rotary_pos_emb(xq, xk, cos, sin)
        if past_key_value is not None:
            xk = torch.cat([past_key_value[0], xk], dim=1)
            xv = torch.cat([past_key_value[1], xv], dim=1)
        past_kv = (xk, xv) if use_cache else None
        q_len, kv_len = xq.shape[1], xk.shape[1]
        drop_p = self.dropout if self.training else 0.0
        q = xq.transpose(1, 2)
        k = repeat_kv(xk, self.n_rep).transpose(1, 2)
        v = repeat_kv(xv, self.n_rep).transpose(1, 2)
        if attention_mask is None:
            if not self.is_causal or q_len == 1:
                out = F.scaled_dot_product_attention(q, k, v, dropout_p=drop_p, is_causal=False)
            elif q_len == kv_len:
                out = F.scaled_dot_product_attention(q, k, v, dropout_p=drop_p, is_causal=True)
            else:  # chunked prefill: right-aligned causal mask
                m = torch.full((q_len, kv_len), float("-inf"), device=q.device, dtype=q.dtype)
                m = m.triu(kv_len - q_len + 1)
                out = F.scaled_dot_product_attention(q, k, v, attn_mask=m, dropout_p=drop_p)
        else:
            neg = torch.finfo(q.dtype).min
            am = (1.0 - attention_mask.to(q.dtype)).unsqueeze(1).unsqueeze(2) * neg
            if self.is_causal and q_len > 1:
                cm = torch.full((q_len, kv_len), float("-inf"), device=q.device, dtype=q.dtype)
                am = am + cm.triu(kv_len - q_len + 1)
            out = F.scaled_dot_product_attention(q, k, v, attn_mask=am, dropout_p=drop_p)
        out = out.transpose(1, 2).reshape(bsz, q_len, -1)
        return self.o_proj(out), past_kv


class FeedForward(nn.Module):
    """SwiGLU FFN (model/model_minimind.py:258-268)."""

    def __init__(self, config: MiniMindConfig, intermediate_size: int = None):
        super().__init__()
        inter = intermediate_size or config.intermediate_size
        self.gate_proj = nn.Linear(config.hidden_size, inter, bias=False)
        self.down_proj = nn.Linear(inter, config.hidden_size, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, inter, bias=False)

    def forward(self, x):
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class MOEFeedForward(nn.Module):
    """Top-k softmax-routed experts (model/model_minimind.py:270-298), inference path."""

    def __init__(self, config: MiniMindConfig):
        super().__init__()
        self.config = config
        self.gate = nn.Linear(config.hidden_size, config.num_experts, bias=False)
        self.experts = nn.ModuleList([FeedForward(config, config.moe_intermediate_size)
                                      for _ in range(config.num_experts)])
        self.aux_loss = None

    def forward(self, x):
        b, l, d = x.shape
        xf = x.view(-1, d)
        scores = F.softmax(self.gate(xf), dim=-1)
        w, idx = torch.topk(scores, k=self.config.num_experts_per_tok, dim=-1, sorted=False)
        if self.config.norm_topk_prob:
            w = w / (w.sum(dim=-1, keepdim=True) + 1e-20)
        y = torch.zeros_like(xf)
        for i, expert in enumerate(self.experts):
            mask = idx == i
            tok = mask.any(dim=-1).nonzero().flatten()
            if tok.numel():
                y.index_add_(0, tok, (expert(xf[tok]) * w[mask].view(-1, 1)).to(y.dtype))
        if self.training and self.config.router_aux_loss_coef > 0:
            load = F.one_hot(idx, self.config.num_experts).float().mean(0)
            self.aux_loss = (load * scores.mean(0)).sum() * self.config.num_experts * \
                self.config.router_aux_loss_coef
        else:
            self.aux_loss = scores.new_zeros(1).squeeze()
        return y.view(b, l, d)


class MiniMindBlock(nn.Module):
    """Pre-norm block; with use_mhc each sublayer is wrapped by an mHC
    connection that receives F as a closure (model/model_minimind.py:300-350)."""

    def __init__(self, layer_id: int, config: MiniMindConfig):
        super().__init__()
        self.self_attn = Attention(config)
        self.mlp = FeedForward(config) if not config.use_moe else MOEFeedForward(config)
        self.use_mhc = config.use_mhc
        eps, D = config.rms_norm_eps, config.hidden_size
        self.attn_in_norm = nn.RMSNorm(D, eps=eps)
        self.ffn_in_norm = nn.RMSNorm(D, eps=eps)
        if config.use_mhc:
            n = config.mhc_residual_expansion
            cls = MHCConnection_Fused if config.use_mhc == 1 else MHCConnection_FusedNoHres
            self.attn_mhc = cls(n, D, eps=eps)
            self.mlp_mhc = cls(n, D, eps=eps)

    def forward(self, hidden_states, position_embeddings, past_key_value=None, use_cache=False,
                attention_mask=None, chain=None):
        if self.use_mhc:
            holder = [None]

            # F(z) = sublayer(in_norm(z)); the connection applies in_norm (inside
            # its pre launch when no autograd is needed).
            def attn_fn(zn):
                out, kv = self.self_attn(zn, position_embeddings, past_key_value, use_cache,
                                         attention_mask)
                holder[0] = kv
                return out

            hidden_states = self.attn_mhc(hidden_states, attn_fn, in_norm=self.attn_in_norm,
                                          chain=chain)
            hidden_states = self.mlp_mhc(hidden_states, self.mlp, in_norm=self.ffn_in_norm,
                                         chain=chain)
            return hidden_states, holder[0]
        attn_out, kv = self.self_attn(self.attn_in_norm(hidden_states), position_embeddings,
                                      past_key_value, use_cache, attention_mask)
        hidden_states = hidden_states + attn_out
        hidden_states = hidden_states + self.mlp(self.ffn_in_norm(hidden_states))
        return hidden_states, kv


class MiniMindModel(nn.Module):
    """Embedding -> (RMSNorm, StreamExpand) -> blocks -> (MHCHead, RMSNorm)
    (model/model_minimind.py:353-403)."""

    def __init__(self, config: MiniMindConfig):
        super().__init__()
        self.config = config
        self.vocab_size, self.num_hidden_layers = config.vocab_size, config.num_hidden_layers
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.dropout = nn.Dropout(config.dropout)
        eps, D = config.rms_norm_eps, config.hidden_size
        if config.use_mhc:
            n = config.mhc_residual_expansion
            self.embed_up_norm = nn.Sequential(nn.RMSNorm(D, eps=eps), StreamExpand(n, D))
            self.layers = nn.ModuleList([MiniMindBlock(i, config) for i in range(self.num_hidden_layers)])
            self.norm = nn.Sequential(MHCHead(n, D, eps=eps), nn.RMSNorm(D, eps=eps))
        else:
            self.embed_up_norm = nn.Identity()
            self.layers = nn.ModuleList([MiniMindBlock(i, config) for i in range(self.num_hidden_layers)])
            self.norm = nn.RMSNorm(D, eps=eps)
        cos, sin = precompute_freqs_cis(config.head_dim, config.max_position_embeddings,
                                        config.rope_theta, config.rope_scaling)
        self.register_buffer("freqs_cos", cos, persistent=False)
        self.register_buffer("freqs_sin", sin, persistent=False)

    def forward(self, input_ids, attention_mask=None, past_key_values=None, use_cache=False,
                **kwargs):
        bsz, seq_len = input_ids.shape
        past_key_values = past_key_values or [None] * len(self.layers)
        start = past_key_values[0][0].shape[1] if past_key_values[0] is not None else 0
        h = self.dropout(self.embed_tokens(input_ids))
        # Each mHC launch that writes the stream hands its rows' sums of squares
        # to the next one that reads it (the stream passes from call to call
        # unchanged): a chain per forward.
        chain = StreamChain() if self.config.use_mhc else None
        if self.config.use_mhc:  # RMSNorm + StreamExpand, one launch without autograd
            h = self.embed_up_norm[1].forward_normed(h, self.embed_up_norm[0], chain=chain)
        else:
            h = self.embed_up_norm(h)
        pos = (self.freqs_cos[start:start + seq_len], self.freqs_sin[start:start + seq_len])
        presents = []
        for layer, pkv in zip(self.layers, past_key_values):
            h, present = layer(h, pos, past_key_value=pkv, use_cache=use_cache,
                               attention_mask=attention_mask, chain=chain)
            presents.append(present)
        if self.config.use_mhc:  # MHCHead + final RMSNorm, one launch without autograd
            h = self.norm[0](h, out_norm=self.norm[1], chain=chain)
        else:
            h = self.norm(h)
        aux = sum([l.mlp.aux_loss for l in self.layers if isinstance(l.mlp, MOEFeedForward)],
                  h.new_zeros(1).squeeze())
        return h, presents, aux


class MiniMindForCausalLM(nn.Module):
    """Causal LM head tied to the embedding (model/model_minimind.py:405-426)."""

    def __init__(self, config: MiniMindConfig = None):
        super().__init__()
        self.config = config or MiniMindConfig()
        self.model = MiniMindModel(self.config)
        self.lm_head = nn.Linear(self.config.hidden_size, self.config.vocab_size, bias=False)
        if self.config.tie_word_embeddings:
            self.model.embed_tokens.weight = self.lm_head.weight

    def forward(self, input_ids, attention_mask=None, past_key_values=None, use_cache=False,
                logits_to_keep=0, labels=None, **kwargs):
        h, pkv, aux = self.model(input_ids, attention_mask, past_key_values, use_cache, **kwargs)
        sl = slice(-logits_to_keep, None) if isinstance(logits_to_keep, int) else logits_to_keep
        logits = self.lm_head(h[:, sl, :])
        loss = None
        if labels is not None:
            x, y = logits[..., :-1, :].contiguous(), labels[..., 1:].contiguous()
            loss = F.cross_entropy(x.view(-1, x.size(-1)), y.view(-1), ignore_index=-100)
        return SimpleNamespace(loss=loss, aux_loss=aux, logits=logits, past_key_values=pkv,
                               hidden_states=h)


def init_normal_(model: nn.Module, std: float = 0.02) -> nn.Module:
    """Every parameter ~ N(0, std) except RMSNorm gains (1), mHC alphas / biases
    (reference constructor values) -- the benchmark models' random init."""
    with torch.no_grad():
        for name, p in model.named_parameters():
            leaf = name.rsplit(".", 1)[-1]
            if leaf in ("alpha_pre", "alpha_post", "alpha_res", "alpha", "bias_pre",
                        "bias_post", "bias_res", "bias"):
                continue
            if p.dim() == 1 and leaf == "weight":  # RMSNorm gains
                continue
            p.normal_(0.0, std)
    return model
