"""Granite MoE checkpoints (safetensors) into the model's weight dict.

The drop-in for the reference loader (litemoe/weights.py:16-37 load_config,
:40-54 TensorSource, :84-108 load_weights) on one GPU: the same config
checks, the same checkpoint names (the original Granite schema,
``block_sparse_moe.input_linear.weight`` [E, 2I, H] gate rows first,
``output_linear.weight`` [E, H, I], ``router.layer.weight`` [E, H]) and the
same dict (``embedding``, ``layers`` of per-layer dicts with ``physical`` /
``logical``, ``norm``, ``head``). Expert tensors stay in the checkpoint's
layout: the decode kernels read whole rows of it as stored.

Differences from the reference, all in how bytes move: every shard is
opened once (not once per tensor); an expert tensor is read whole and
copied to the device in one transfer when all experts are local (one GPU,
identity placement), instead of one host slice per expert.
"""
from __future__ import annotations

import json
import math
from pathlib import Path

import torch

from .config import ModelConfig, validate_config


def load_config(path) -> ModelConfig:
    """config.json of a Granite MoE checkpoint directory, with the RoPE
    semantics of the file kept whatever encoding the installed Transformers
    parses it into (litemoe/weights.py:16-37): ``rope_theta`` must be a
    finite positive number, no RoPE scaling, and a parsed
    ``rope_parameters`` must say the same as the file."""
    from transformers import AutoConfig

    raw = json.loads((Path(path) / "config.json").read_text(encoding="utf-8"))
    theta = raw.get("rope_theta")
    plain = {"rope_type": "default", "rope_theta": theta}
    theta_ok = isinstance(theta, (int, float)) and not isinstance(theta, bool) and math.isfinite(theta) \
        and theta > 0
    if raw.get("model_type") != "granitemoe" or raw.get("rope_scaling") is not None or not theta_ok \
            or raw.get("rope_parameters", plain) != plain:
        raise ValueError("Checkpoint must declare unscaled Granite RoPE with a finite positive theta")
    values = AutoConfig.from_pretrained(path, local_files_only=True).to_dict()
    parsed_params = values.pop("rope_parameters", None)
    if parsed_params is not None:
        if parsed_params != plain or values.get("rope_scaling") not in (None, plain) \
                or values.get("rope_theta", theta) != theta:
            raise ValueError("Parsed RoPE differs from the original checkpoint")
    elif values.get("rope_theta") != theta or values.get("rope_scaling") is not None:
        raise ValueError("Parsed RoPE differs from the original checkpoint")
    values["rope_theta"], values["rope_scaling"] = theta, None
    cfg = ModelConfig(**values)
    validate_config(cfg)
    return cfg


class CheckpointSource:
    """Tensors of a checkpoint directory: ``model.safetensors``, or the shards
    a ``model.safetensors.index.json`` maps (litemoe/weights.py:40-54).
    ``get(key)`` returns a CPU tensor; ``get(key, expert=e)`` the slice of
    expert e only."""

    def __init__(self, path):
        from safetensors import safe_open

        self.path = Path(path)
        index = self.path / "model.safetensors.index.json"
        if index.exists():
            self.index = json.loads(index.read_text(encoding="utf-8"))["weight_map"]
        else:
            with safe_open(str(self.path / "model.safetensors"), framework="pt", device="cpu") as f:
                self.index = {key: "model.safetensors" for key in f.keys()}
        self._open = safe_open
        self._files = {}

    def _file(self, key):
        if key not in self.index:
            raise KeyError(f"{key} is not in the checkpoint")
        name = self.index[key]
        handle = self._files.get(name)
        if handle is None:
            handle = self._open(str(self.path / name), framework="pt", device="cpu")
            self._files[name] = handle
        return handle

    def get(self, key, expert=None):
        f = self._file(key)
        return f.get_tensor(key) if expert is None else f.get_slice(key)[expert]

    def close(self):
        self._files.clear()


# The reference's name for the same object.
TensorSource = CheckpointSource

_DENSE = ("input_layernorm", "post_attention_layernorm", "self_attn.q_proj", "self_attn.k_proj",
          "self_attn.v_proj", "self_attn.o_proj", "block_sparse_moe.router.layer")


def load_weights(cfg, source, placement=None, rank=0, device="cuda", dtype=torch.bfloat16, backend=None):
    """The weight dict ``Granite`` takes (litemoe/weights.py:80-108).

    One GPU holds every expert: ``placement`` may be None or a placement of
    world size 1. ``placement.physical[layer][e]`` is the slot of checkpoint
    expert ``e`` (the router's ids are mapped through it before the expert
    GEMMs), so slot ``s`` is filled with expert ``argsort(physical)[s]`` and
    ``logical`` is that inverse permutation, as the reference builds it
    (litemoe/placement.py:31-38, weights.py:92-105). ``backend`` is accepted for signature compatibility
    and not used (the reference passes it through unused as well)."""
    validate_config(cfg)
    layers_n, experts = cfg.num_hidden_layers, cfg.num_local_experts
    if placement is not None:
        if getattr(placement, "world", 1) != 1 or rank != 0:
            raise ValueError("Expert parallelism is not part of this single-GPU path")
        placement.validate(layers_n, experts, 1)
    shapes = {"input_linear": (experts, 2 * cfg.intermediate_size, cfg.hidden_size),
              "output_linear": (experts, cfg.hidden_size, cfg.intermediate_size)}

    def load(key):
        return source.get(key).to(device=device, dtype=dtype).contiguous()

    embedding = load("model.embed_tokens.weight")
    layers = []
    for layer in range(layers_n):
        prefix = f"model.layers.{layer}."
        weights = {name: load(prefix + name + ".weight") for name in _DENSE}
        physical = list(range(experts)) if placement is None else list(placement.physical[layer])
        if sorted(physical) != list(range(experts)):
            raise ValueError("A single GPU must hold every expert exactly once")
        identity = physical == list(range(experts))
        for name, shape in shapes.items():
            key = prefix + "block_sparse_moe." + name + ".weight"
            if identity:
                value = source.get(key)
                if tuple(value.shape) != shape:
                    raise ValueError(f"Checkpoint expert geometry mismatch: {name}")
                weights[name] = value.to(device=device, dtype=dtype).contiguous()
            else:
                target = torch.empty(shape, dtype=dtype, device=device)
                holder = sorted(range(experts), key=physical.__getitem__)  # slot -> expert
                for local, logical in enumerate(holder):
                    value = source.get(key, expert=logical)
                    if tuple(value.shape) != shape[1:]:
                        raise ValueError(f"Checkpoint expert geometry mismatch: {name}")
                    target[local].copy_(value)
                weights[name] = target
        weights["physical"] = torch.tensor(physical, dtype=torch.int64, device=device)
        # Empty means identity (the lean path), as in the reference.
        weights["logical"] = weights["physical"][:0] if identity else weights["physical"].argsort()
        layers.append(weights)
    head = embedding if cfg.tie_word_embeddings else load("lm_head.weight")
    return dict(embedding=embedding, layers=layers, norm=load("model.norm.weight"), head=head)
