"""Granite MoE model configuration (HF ``GraniteMoeConfig`` field names).

The field names and the validation follow the reference loader,
litemoe/weights.py:11-37 (``ModelConfig``) and :68-77 (``validate_config``).
Presets are the Granite 3.1 geometries the benchmark configurations name.
"""
from __future__ import annotations

from types import SimpleNamespace


class ModelConfig(SimpleNamespace):
    """Attribute bag with the HF GraniteMoe field names (weights.py:11-13)."""

    def to_dict(self):
        return vars(self).copy()

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


# Multipliers are Granite-3.1-like values; the benchmark's random-init
# weights make them a choice, recorded with the configuration.
_COMMON = dict(
    model_type="granitemoe", hidden_act="silu", attention_bias=False, rope_scaling=None,
    rope_theta=10000.0, rms_norm_eps=1e-6, max_position_embeddings=4096,
    embedding_multiplier=12.0, attention_multiplier=0.015625, residual_multiplier=0.22,
    logits_scaling=6.0, tie_word_embeddings=True, eos_token_id=0, vocab_size=49155,
    num_experts_per_tok=8, intermediate_size=512,
)

PRESETS = {
    # Granite-3.1-1B-a400m shape.
    "granite-1b": dict(_COMMON, hidden_size=1024, num_hidden_layers=24, num_attention_heads=16,
                       num_key_value_heads=8, num_local_experts=32),
    # Granite-3.1-3B-a800m shape.
    "granite-3b": dict(_COMMON, hidden_size=1536, num_hidden_layers=32, num_attention_heads=24,
                       num_key_value_heads=8, num_local_experts=40),
}


def preset(name: str, **overrides) -> ModelConfig:
    cfg = ModelConfig(**{**PRESETS[name], **overrides})
    validate_config(cfg)
    return cfg


def validate_config(cfg) -> None:
    """Reject geometries the Granite adapter does not implement (weights.py:68-77)."""
    if getattr(cfg, "model_type", "granitemoe") != "granitemoe" or cfg.hidden_act != "silu":
        raise ValueError("This adapter implements Granite MoE / SwiGLU only")
    if getattr(cfg, "attention_bias", False) or getattr(cfg, "rope_scaling", None) is not None:
        raise ValueError("Attention bias and scaled RoPE require a separate validated adapter")
    if cfg.hidden_size % cfg.num_attention_heads or cfg.num_attention_heads % cfg.num_key_value_heads:
        raise ValueError("Invalid GQA geometry")
    for field in ("embedding_multiplier", "attention_multiplier", "residual_multiplier", "logits_scaling"):
        if not getattr(cfg, field, 0) > 0:
            raise ValueError(f"Invalid checkpoint field {field}")
