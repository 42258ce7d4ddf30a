"""Shared test helpers: HF GraniteMoe models as oracles, weight conversion,
error metrics."""
import torch

from litemoe_amd.config import ModelConfig


def rel_l2(a, b):
    a, b = a.float(), b.float()
    return float((a - b).norm() / b.norm().clamp_min(1e-12))


def config_from_hf(hf_cfg, **overrides):
    d = dict(model_type="granitemoe", hidden_act="silu", attention_bias=False, rope_scaling=None,
             vocab_size=hf_cfg.vocab_size, hidden_size=hf_cfg.hidden_size,
             intermediate_size=hf_cfg.intermediate_size, num_hidden_layers=hf_cfg.num_hidden_layers,
             num_attention_heads=hf_cfg.num_attention_heads, num_key_value_heads=hf_cfg.num_key_value_heads,
             num_local_experts=hf_cfg.num_local_experts, num_experts_per_tok=hf_cfg.num_experts_per_tok,
             max_position_embeddings=hf_cfg.max_position_embeddings, rms_norm_eps=hf_cfg.rms_norm_eps,
             rope_theta=10000.0, embedding_multiplier=hf_cfg.embedding_multiplier,
             attention_multiplier=hf_cfg.attention_multiplier, residual_multiplier=hf_cfg.residual_multiplier,
             logits_scaling=hf_cfg.logits_scaling, eos_token_id=hf_cfg.eos_token_id,
             tie_word_embeddings=hf_cfg.tie_word_embeddings)
    d.update(overrides)
    return ModelConfig(**d)


def hf_weights(hf, dtype=torch.float32, device="cpu"):
    """HF GraniteMoe state dict -> the reference's per-layer weight dicts
    (litemoe/weights.py:84-108; names mapped as the reference's
    tests/conftest.py:20-25)."""
    sd = hf.state_dict()
    cfg = hf.config
    cast = lambda t: t.detach().to(device=device, dtype=dtype).contiguous()
    layers = []
    for l in range(cfg.num_hidden_layers):
        p = f"model.layers.{l}."
        layer = {name: cast(sd[p + name + ".weight"]) for name in (
            "input_layernorm", "post_attention_layernorm", "self_attn.q_proj", "self_attn.k_proj",
            "self_attn.v_proj", "self_attn.o_proj")}
        layer["block_sparse_moe.router.layer"] = cast(sd[p + "block_sparse_moe.router.weight"])
        layer["input_linear"] = cast(sd[p + "block_sparse_moe.experts.gate_up_proj"])
        layer["output_linear"] = cast(sd[p + "block_sparse_moe.experts.down_proj"])
        layer["physical"] = torch.arange(cfg.num_local_experts, device=device)
        layer["logical"] = layer["physical"][:0]
        layers.append(layer)
    return dict(embedding=cast(sd["model.embed_tokens.weight"]), layers=layers, norm=cast(sd["model.norm.weight"]),
                head=cast(sd["lm_head.weight"]))


def make_hf(seed=7, randomize_norms=True, **geometry):
    from transformers import GraniteMoeConfig, GraniteMoeForCausalLM
    torch.manual_seed(seed)
    base = dict(vocab_size=47, hidden_size=32, intermediate_size=24, num_hidden_layers=2,
                num_attention_heads=4, num_key_value_heads=2, num_local_experts=4, num_experts_per_tok=2,
                max_position_embeddings=64, eos_token_id=0, embedding_multiplier=3.0,
                attention_multiplier=0.125, residual_multiplier=0.3, logits_scaling=2.0, rope_theta=10000.0)
    base.update(geometry)
    cfg = GraniteMoeConfig(**base)
    cfg._attn_implementation = "eager"
    hf = GraniteMoeForCausalLM(cfg).eval()
    if randomize_norms:
        with torch.no_grad():
            for name, p in hf.named_parameters():
                if name.endswith("layernorm.weight") or name == "model.norm.weight":
                    p.copy_(1 + 0.2 * torch.randn_like(p))
    return hf


def tiny_hf_model():
    hf = make_hf()
    return hf, config_from_hf(hf.config), hf_weights(hf)


def bf16_ordered(t):
    """bf16 bit patterns on a monotone integer line (-0 and +0 coincide)."""
    i = t.contiguous().view(torch.int16).to(torch.int32)
    return torch.where(i >= 0, i, -(i & 0x7FFF))


def bf16_within_ulp_or_abs(a, b, ulps, floor):
    """Every element of two bf16 tensors within ``ulps`` units in the last
    place, or within ``floor`` absolutely (sums near zero cancel)."""
    close = (bf16_ordered(a) - bf16_ordered(b)).abs() <= ulps
    return bool((close | ((a.float() - b.float()).abs() <= floor)).all())
