"""Deterministic synthetic inputs and random-init Granite weights.

Two generators:

* ``numpy`` (default for tests and fixtures): ``numpy.random.RandomState(seed)``
  float64 normals (the frozen legacy stream), scaled, cast to float32, then
  rounded to bfloat16 to nearest-even by bit arithmetic. The bytes do not
  depend on the torch version, so committed fixtures regenerate exactly.
  Each tensor has its own seed ``base * 1_000_003 + index``.
* ``torch``: ``torch.Generator`` on the target device, for benchmark-sized
  models (gigabytes of weights) where the CPU stream would dominate start-up.

Weights follow the HF GraniteMoe init (linears and embeddings N(0, 0.02), norm
weights 1) in the reference's in-memory layout, litemoe/weights.py:84-108.
"""
from __future__ import annotations

import hashlib

import numpy as np
import torch

STD = 0.02
SEED_STRIDE = 1_000_003


def tensor_seed(base: int, index: int) -> int:
    return (base * SEED_STRIDE + index) % (2 ** 32)


def bf16_bits(values: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bit patterns, round to nearest even, NaN -> 0x7fc0."""
    u = np.ascontiguousarray(values, dtype=np.float32).view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rounded[nan] = 0x7FC0
    return rounded


def bits_to_tensor(bits: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(bits.astype(np.int16, copy=False).copy()).view(torch.bfloat16)


def normal_bf16(shape, std: float, seed: int) -> torch.Tensor:
    """N(0, std^2) bfloat16 CPU tensor from the legacy numpy stream."""
    values = np.random.RandomState(seed).standard_normal(size=tuple(shape))
    return bits_to_tensor(bf16_bits((values * std).astype(np.float32)))


def sha256(t: torch.Tensor) -> str:
    return hashlib.sha256(t.detach().cpu().contiguous().view(torch.uint8).numpy().tobytes()).hexdigest()


class _Source:
    def __init__(self, seed: int, method: str, device, dtype):
        self.seed, self.method, self.device, self.dtype = seed, method, torch.device(device), dtype
        self.index = 0
        if method == "torch":
            self.gen = torch.Generator(device=self.device)
            self.gen.manual_seed(seed)
        elif method != "numpy":
            raise ValueError(f"unknown generator {method!r}")

    def normal(self, shape, std=STD):
        i, self.index = self.index, self.index + 1
        if self.method == "numpy":
            return normal_bf16(shape, std, tensor_seed(self.seed, i)).to(self.device, self.dtype)
        out = torch.empty(shape, device=self.device, dtype=torch.float32)
        out.normal_(0.0, std, generator=self.gen)
        return out.to(self.dtype)


def granite_weights(cfg, seed: int = 0, device="cpu", dtype=torch.bfloat16, method: str = "numpy"):
    """Random-init Granite MoE weights in the reference's layout.

    Keys per layer: ``input_layernorm``, ``post_attention_layernorm``,
    ``self_attn.{q,k,v,o}_proj``, ``block_sparse_moe.router.layer``,
    ``input_linear`` [E, 2I, H] (gate rows first), ``output_linear`` [E, H, I],
    ``physical`` (identity placement) and ``logical`` (empty = identity),
    exactly the names of litemoe/weights.py:88-105.
    """
    src = _Source(seed, method, device, dtype)
    H, I, E = cfg.hidden_size, cfg.intermediate_size, cfg.num_local_experts
    D = H // cfg.num_attention_heads
    q_out, kv_out = cfg.num_attention_heads * D, cfg.num_key_value_heads * D
    embedding = src.normal((cfg.vocab_size, H))
    ones = lambda: torch.ones(H, device=device, dtype=dtype)
    layers = []
    for _ in range(cfg.num_hidden_layers):
        layer = {
            "input_layernorm": ones(),
            "post_attention_layernorm": ones(),
            "self_attn.q_proj": src.normal((q_out, H)),
            "self_attn.k_proj": src.normal((kv_out, H)),
            "self_attn.v_proj": src.normal((kv_out, H)),
            "self_attn.o_proj": src.normal((H, q_out)),
            "block_sparse_moe.router.layer": src.normal((E, H)),
            "input_linear": src.normal((E, 2 * I, H)),
            "output_linear": src.normal((E, H, I)),
            "physical": torch.arange(E, device=device, dtype=torch.int64),
        }
        layer["logical"] = layer["physical"][:0]
        layers.append(layer)
    head = embedding if getattr(cfg, "tie_word_embeddings", True) else src.normal((cfg.vocab_size, H))
    return dict(embedding=embedding, layers=layers, norm=ones(), head=head)


def prompts(count: int, length, vocab: int, seed: int):
    """Token-id prompts uniform in [0, vocab); ``length`` is an int or a list."""
    rng = np.random.RandomState(seed)
    lengths = [length] * count if isinstance(length, int) else list(length)
    return [rng.randint(0, vocab, size=n).tolist() for n in lengths]


def ragged_lengths(count: int, low: int, high: int, seed: int):
    """Lengths uniform in [low, high] (inclusive)."""
    return np.random.RandomState(seed).randint(low, high + 1, size=count).tolist()
