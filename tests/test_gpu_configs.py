"""BASELINE configs 3, 4 and 5 at their model configuration, on the GPU
against the CPU copy whose mHC pieces are the oracle.

  C3: dense MiniMind-3-mHC, 8 layers, hidden 768, 8 q / 4 kv heads, head_dim
      96, SwiGLU 2048, vocab 6400, n = 4, use_mhc = 1; prefill.
  C4: the C3 model decoding one token for 64 sequences over a KV cache of 2048
      positions per layer filled with N(0, 1) values (bf16-representable).
  C5: n = 8, 8 routed experts top-2 of intermediate 1024; prefill.

The models run in fp32 on both sides (the comparison is of the kernels, not of
bf16 rounding; the bf16 layer rows at C = 768 are tests/golden's c2 / c5
fixtures).  Prefills use B = 2, T = 128 instead of the benchmark's batch so
the CPU side finishes in seconds.  Bar: 1e-4 of the largest logit (GEMM and
attention summation orders differ between the GPU libraries and the CPU).
"""
from __future__ import annotations

import pytest
import torch

from tests.test_gpu_model import _model, _oracle_copy, _rel

pytestmark = pytest.mark.gpu

from model.model_minimind import MiniMindConfig, MiniMindForCausalLM, init_normal_  # noqa: E402


def _c3(**kw) -> MiniMindConfig:
    base = dict(hidden_size=768, num_hidden_layers=8, num_attention_heads=8, num_key_value_heads=4,
                head_dim=96, intermediate_size=2048, rope_theta=1e6, vocab_size=6400, use_mhc=1,
                mhc_residual_expansion=4, max_position_embeddings=4096)
    base.update(kw)
    return MiniMindConfig(**base)


def _c5() -> MiniMindConfig:
    return _c3(mhc_residual_expansion=8, use_moe=True, num_experts=8, num_experts_per_tok=2,
               moe_intermediate_size=1024)


def _build(cfg, init: str):
    """init: "baseline" = N(0, 0.02) for every weight, the
    mHC gate parameters at the reference's initial values; "stress" = gates
    moved off their init (alphas 0.5, biases + N(0, 0.3), phi N(0, 0.1)) so the
    projection drives every gate."""
    if init == "stress":
        return _model(cfg)
    torch.manual_seed(0)
    return init_normal_(MiniMindForCausalLM(cfg)).eval()


@pytest.mark.parametrize("config", ["c3", "c5"])
@pytest.mark.parametrize("init", ["baseline", "stress"])
def test_prefill_model_config_vs_oracle(dev, config, init):
    cfg = _c3() if config == "c3" else _c5()
    model = _build(cfg, init)
    ref = _oracle_copy(model)
    g = torch.Generator().manual_seed(11)
    ids = torch.randint(0, cfg.vocab_size, (2, 128), generator=g)
    print(f"prefill {config} {init}", flush=True)
    with torch.no_grad():
        want = ref(ids).logits
        got = model.to(dev)(ids.to(dev)).logits
    assert _rel(got, want) < 1e-4, (config, init, _rel(got, want))


def test_decode_model_config_c4_vs_oracle(dev):
    """C4's step: batch 64, one new token per sequence, a 2048-entry cache per
    layer, the mHC connections at M = 64."""
    cfg = _c3()
    model = _build(cfg, "stress")
    ref = _oracle_copy(model)
    B, T = 64, 2048
    g = torch.Generator().manual_seed(12)
    kv = []
    for _ in range(cfg.num_hidden_layers):
        shape = (B, T, cfg.num_key_value_heads, cfg.head_dim)
        kv.append(tuple(torch.randn(shape, generator=g).to(torch.bfloat16).float()
                        for _ in range(2)))
    ids = torch.randint(0, cfg.vocab_size, (B, 1), generator=g)
    print("decode c4 B=64 cache=2048", flush=True)
    with torch.no_grad():
        want = ref(ids, past_key_values=kv).logits
        kv_d = [(k.to(dev), v.to(dev)) for k, v in kv]
        got = model.to(dev)(ids.to(dev), past_key_values=kv_d).logits
    assert got.shape == (B, 1, cfg.vocab_size)
    assert _rel(got, want) < 1e-4, _rel(got, want)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_decode_model_config_c4_matches_prefill(dev, dtype):
    """Batch 64: a prefill of T tokens, then a one-token decode over its cache,
    against one prefill of T + 1 tokens (last position's logits)."""
    cfg = _c3()
    model = _build(cfg, "stress").to(dtype).to(dev)
    g = torch.Generator().manual_seed(13)
    ids = torch.randint(0, cfg.vocab_size, (64, 97), generator=g).to(dev)
    with torch.no_grad():
        full = model(ids).logits[:, -1]
        pre = model(ids[:, :-1], use_cache=True)
        step = model(ids[:, -1:], past_key_values=pre.past_key_values, use_cache=True).logits[:, -1]
    bar = 1e-4 if dtype == torch.float32 else 3e-2
    assert _rel(step, full) < bar, _rel(step, full)


@pytest.mark.parametrize("use_mhc,n,moe", [(1, 4, False), (2, 4, False), (1, 8, True)])
def test_reference_fp16_checkpoint_runs_on_hip_model(dev, tmp_path, use_mhc, n, moe):
    """A .pth written the way the reference trainer writes one (every tensor
    .half().cpu(), torch.save; trainer/trainer_utils.py:63-73), loaded with the
    reference's own call (load_state_dict(strict=False), :124-127) into the
    HIP model on the GPU: logits equal the oracle copy's on the same fp16
    weights (fp32 compute on both sides)."""
    cfg = _c3(num_hidden_layers=2, use_mhc=use_mhc, mhc_residual_expansion=n, use_moe=moe,
              num_experts=8, num_experts_per_tok=2, moe_intermediate_size=1024)
    src = _model(cfg)
    path = tmp_path / f"full_sft_{cfg.hidden_size}{'_moe' if moe else ''}.pth"
    torch.save({k: v.half().cpu() for k, v in src.state_dict().items()}, path)

    weights = torch.load(path, map_location="cpu", weights_only=True)
    model = MiniMindForCausalLM(cfg)
    res = model.load_state_dict(weights, strict=False)
    assert not res.missing_keys and not res.unexpected_keys
    model = model.eval()
    ref = _oracle_copy(model)
    g = torch.Generator().manual_seed(14)
    ids = torch.randint(0, cfg.vocab_size, (2, 64), generator=g)
    with torch.no_grad():
        want = ref(ids).logits
        got = model.to(dev)(ids.to(dev)).logits
    assert _rel(got, want) < 1e-4, _rel(got, want)


def _hook_mhc(model):
    """Wrap every mHC piece of a model so that each call records its inputs
    and outputs: the connections (x, the sublayer's input, the sublayer's
    output, out), the entry RMSNorm + StreamExpand and the exit MHCHead +
    final RMSNorm.  Returns the record list (filled in call order)."""
    from model.mhc_common import MHCHead, StreamExpand
    from model.mhc_fused import MHCConnection_Fused

    records = []
    for name, mod in model.named_modules():
        if isinstance(mod, MHCConnection_Fused):
            def conn(x, f, in_norm=None, chain=None, _orig=mod.forward, _mod=mod, _name=name):
                rec = {"kind": "conn", "name": _name, "mod": _mod, "norm": in_norm,
                       "x": x.detach().clone()}

                def fw(z):
                    rec["z"] = z.detach().clone()
                    o = f(z)
                    rec["f"] = o.detach().clone()
                    return o
                out = _orig(x, fw, in_norm, chain=chain)
                rec["out"] = out.detach().clone()
                records.append(rec)
                return out
            mod.forward = conn
        elif isinstance(mod, StreamExpand):
            def expand(x, norm, chain=None, _orig=mod.forward_normed, _mod=mod):
                out = _orig(x, norm, chain=chain)
                records.append({"kind": "entry", "mod": _mod, "norm": norm,
                                "x": x.detach().clone(), "out": out.detach().clone()})
                return out
            mod.forward_normed = expand
        elif isinstance(mod, MHCHead):
            def head(x, out_norm=None, chain=None, _orig=mod.forward, _mod=mod):
                out = _orig(x, out_norm, chain=chain)
                records.append({"kind": "exit", "mod": _mod, "norm": out_norm,
                                "x": x.detach().clone(), "out": out.detach().clone()})
                return out
            mod.forward = head
    return records


def _cpu_norm(norm):
    """The GPU model's nn.RMSNorm as a bf16 CPU module with the same gain."""
    c = torch.nn.RMSNorm(norm.normalized_shape, eps=norm.eps).to(torch.bfloat16)
    with torch.no_grad():
        c.weight.copy_(norm.weight.detach().cpu())
    return c


def _check_record(rec):
    """One recorded mHC call against the oracle on its captured inputs (bf16,
    the reference's rounding points, max-norm 1e-2).  A connection's sublayer
    returns the captured sublayer output, so the comparison is of the mHC
    arithmetic alone; its sublayer input (normed) is compared too."""
    from oracle import mhc_ref as R

    mod, x = rec["mod"], rec["x"].cpu()
    norm = _cpu_norm(rec["norm"]) if rec["norm"] is not None else (lambda t: t)
    if rec["kind"] == "conn":
        seen = {}

        def f(s):
            seen["z"] = norm(s)
            return rec["f"].cpu()
        d = R.mhc_full_forward(x, R.module_params(mod), f, mod.n, mod.dim, eps=mod.eps,
                               pre_eps=mod.pre_eps, post_mult=mod.post_mult_value,
                               sinkhorn_iters=mod.sinkhorn_iters, sinkhorn_eps=mod.sinkhorn_eps)
        return {"out": _rel(rec["out"], d["out"]), "sublayer_in": _rel(rec["z"], seen["z"])}
    if rec["kind"] == "entry":
        want = R.stream_expand(norm(x), mod.n)
    else:
        want = norm(R.head(x, R.module_params(mod), mod.n, mod.dim, pre_eps=mod.pre_eps,
                           rms_eps=mod.eps))
    return {"out": _rel(rec["out"], want)}


@pytest.mark.parametrize("config", ["c3", "c5"])
@pytest.mark.parametrize("kernels", ["small_batch", "large_batch"])
def test_bf16_model_every_connection_vs_oracle(dev, config, kernels):
    """The bf16 C3 (n = 4) and C5 (n = 8, MoE) models with stress gates, B = 2,
    T = 128: every connection, the entry RMSNorm + StreamExpand and the exit
    MHCHead + final RMSNorm, each against the oracle on the inputs it saw in
    the model (1e-2, the bf16 layer bar).  256 tokens take the small-batch
    group kernel; kernels="large_batch" drops the token threshold to 0 so the
    same model runs the persistent (n = 4) / K-streamed (n = 8) kernels.  The
    model runs without autograd, so the norms are the fused epilogues."""
    from model import _ops

    cfg = _c3() if config == "c3" else _c5()
    model = _build(cfg, "stress").to(torch.bfloat16).to(dev)
    records = _hook_mhc(model)
    g = torch.Generator().manual_seed(17)
    ids = torch.randint(0, cfg.vocab_size, (2, 128), generator=g).to(dev)
    prev = _ops.pre_token_threshold(0 if kernels == "large_batch" else 1024)
    try:
        print(f"bf16 per-connection {config} {kernels}", flush=True)
        with torch.no_grad():
            logits = model(ids).logits
        torch.cuda.synchronize()
    finally:
        _ops.pre_token_threshold(prev)
    assert torch.isfinite(logits.float()).all()
    kinds = [r["kind"] for r in records]
    assert kinds.count("entry") == 1 and kinds.count("exit") == 1
    assert kinds.count("conn") == 2 * cfg.num_hidden_layers
    worst = {}
    for rec in records:
        errs = _check_record(rec)
        for k, v in errs.items():
            key = (rec["kind"], rec.get("name", ""), k)
            worst[key] = v
    bad = {k: v for k, v in worst.items() if not v <= 1e-2}
    assert not bad, bad
    print(f"max per-connection error {max(worst.values()):.2e}", flush=True)
