"""Checkpoint loading: config checks and the saved-checkpoint round trip.

Follows the reference's tests/test_config_loading.py: a tiny HF GraniteMoe
model exported to the original Granite checkpoint schema (the mapping of
tests/conftest.py:20-25) and read back by ``load_config`` /
``CheckpointSource`` / ``load_weights``; the dict must equal the one built
from the HF state dict directly, tensor for tensor. The config cases are the
reference's rejection cases (test_config_loading.py:51-76).
"""
import copy
import json
from types import SimpleNamespace

import pytest
import torch

from helpers import config_from_hf, hf_weights, make_hf
from litemoe_amd import weights as W


def checkpoint_state(hf):
    """HF GraniteMoe names -> the original Granite checkpoint names (a tied
    head is not stored)."""
    tied = hf.config.tie_word_embeddings
    return {key.replace(".router.weight", ".router.layer.weight")
               .replace(".experts.gate_up_proj", ".input_linear.weight")
               .replace(".experts.down_proj", ".output_linear.weight"): value.detach().clone().contiguous()
            for key, value in hf.state_dict().items() if not (tied and key == "lm_head.weight")}


def write_config(hf, path):
    raw = hf.config.to_dict()
    raw.update(rope_theta=10000.0, rope_scaling=None)
    raw.pop("rope_parameters", None)
    (path / "config.json").write_text(json.dumps(raw))
    return raw


def save_checkpoint(hf, path, shards=1):
    from safetensors.torch import save_file
    write_config(hf, path)
    state = checkpoint_state(hf)
    if shards == 1:
        save_file(state, str(path / "model.safetensors"))
        return
    keys = sorted(state)
    weight_map = {}
    for s in range(shards):
        name = f"model-{s + 1:05d}-of-{shards:05d}.safetensors"
        part = {k: state[k] for k in keys[s::shards]}
        save_file(part, str(path / name))
        weight_map.update({k: name for k in part})
    (path / "model.safetensors.index.json").write_text(json.dumps({"metadata": {}, "weight_map": weight_map}))


def assert_same_weights(got, expected):
    for key in ("embedding", "norm", "head"):
        assert torch.equal(got[key], expected[key]), key
    assert len(got["layers"]) == len(expected["layers"])
    for g, e in zip(got["layers"], expected["layers"]):
        assert set(g) == set(e)
        for name in e:
            assert g[name].dtype == e[name].dtype and torch.equal(g[name], e[name]), name


@pytest.mark.parametrize("shards", [1, 3])
@pytest.mark.parametrize("tied", [False, True])
def test_saved_checkpoint_loads_the_hf_weights(tmp_path, shards, tied):
    hf = make_hf(seed=11, tie_word_embeddings=tied)
    save_checkpoint(hf, tmp_path, shards)
    cfg = W.load_config(tmp_path)
    assert cfg.rope_theta == 10000.0 and cfg.rope_scaling is None
    assert cfg.num_local_experts == hf.config.num_local_experts and cfg.tie_word_embeddings == tied
    got = W.load_weights(cfg, W.CheckpointSource(tmp_path), None, 0, "cpu", torch.float32)
    assert_same_weights(got, hf_weights(hf, torch.float32))
    if tied:
        assert got["head"] is got["embedding"]
    bf = W.load_weights(cfg, W.TensorSource(tmp_path), device="cpu", dtype=torch.bfloat16)
    assert_same_weights(bf, hf_weights(hf, torch.bfloat16))


def test_reordering_placement_fills_slots_by_inverse(tmp_path):
    """``physical[layer][e]`` is the slot of expert e (litemoe/placement.py:31-38):
    the router's id e is mapped to physical[e] before the GEMMs, so that slot
    must hold expert e's weights. [2, 0, 3, 1] is not an involution, so
    filling slot s with expert physical[s] instead would fail here."""
    hf = make_hf(seed=12)
    save_checkpoint(hf, tmp_path)
    cfg = W.load_config(tmp_path)
    physical = [[2, 0, 3, 1], [0, 1, 2, 3]]
    placement = SimpleNamespace(world=1, physical=physical, validate=lambda layers, experts, world: None)
    got = W.load_weights(cfg, W.CheckpointSource(tmp_path), placement, 0, "cpu", torch.float32)
    ref = hf_weights(hf, torch.float32)
    for layer, order in enumerate(physical):
        g, e = got["layers"][layer], ref["layers"][layer]
        for name in ("input_linear", "output_linear"):
            for expert, slot in enumerate(order):
                assert torch.equal(g[name][slot], e[name][expert]), (name, expert)
            assert torch.equal(g[name], e[name][torch.tensor(order).argsort()]), name
        assert g["physical"].tolist() == order
        expect_logical = [] if order == sorted(order) else torch.tensor(order).argsort().tolist()
        assert g["logical"].tolist() == expect_logical
        # the ids -> slot map and the combine's slot -> expert map are inverse
        if expect_logical:
            assert [expect_logical[slot] for slot in order] == list(range(len(order)))
    with pytest.raises(ValueError):
        W.load_weights(cfg, W.CheckpointSource(tmp_path), SimpleNamespace(world=2), 0, "cpu")
    bad = SimpleNamespace(world=1, physical=[[0, 0, 1, 2]] * 2, validate=lambda *a: None)
    with pytest.raises(ValueError):
        W.load_weights(cfg, W.CheckpointSource(tmp_path), bad, 0, "cpu")


def test_expert_geometry_mismatch_is_rejected(tmp_path):
    hf = make_hf(seed=13)
    save_checkpoint(hf, tmp_path)
    cfg = W.load_config(tmp_path)
    cfg.intermediate_size += 8
    with pytest.raises(ValueError):
        W.load_weights(cfg, W.CheckpointSource(tmp_path), None, 0, "cpu", torch.float32)


@pytest.mark.parametrize("encoding", ["legacy", "default-parameters"])
def test_config_encoding_keeps_original_semantics(tmp_path, monkeypatch, encoding):
    from transformers import AutoConfig
    hf = make_hf(seed=14)
    raw = write_config(hf, tmp_path)
    parsed = copy.deepcopy(raw)
    if encoding == "default-parameters":
        theta = parsed.pop("rope_theta")
        parsed["rope_parameters"] = {"rope_type": "default", "rope_theta": theta}
        parsed["rope_scaling"] = parsed["rope_parameters"].copy()
    before = copy.deepcopy(parsed)

    class Parsed:
        def to_dict(self):
            return copy.deepcopy(parsed)

    monkeypatch.setattr(AutoConfig, "from_pretrained", lambda *a, **k: Parsed())
    cfg = W.load_config(tmp_path)
    assert cfg.rope_theta == 10000.0 and cfg.rope_scaling is None
    assert parsed == before


@pytest.mark.parametrize("case", ["scaled", "theta", "extra", "nan", "missing", "bool", "bias", "conflict",
                                  "legacy-conflict", "model-type"])
def test_loading_rejects_unsupported_or_changed_config(tmp_path, monkeypatch, case):
    from transformers import AutoConfig
    hf = make_hf(seed=15)
    raw = write_config(hf, tmp_path)
    parsed = copy.deepcopy(raw)
    parsed["rope_parameters"] = {"rope_type": "default", "rope_theta": raw["rope_theta"]}
    if case == "scaled": raw["rope_scaling"] = {"rope_type": "linear", "factor": 2}
    if case == "theta": parsed["rope_parameters"]["rope_theta"] *= 2
    if case == "extra": parsed["rope_parameters"]["factor"] = 2
    if case == "nan": raw["rope_theta"] = float("nan")
    if case == "missing": del raw["rope_theta"]
    if case == "bool": raw["rope_theta"] = True
    if case == "bias": parsed["attention_bias"] = True
    if case == "conflict": parsed["rope_scaling"] = {"rope_type": "linear", "factor": 2}
    if case == "legacy-conflict":
        del parsed["rope_parameters"]
        parsed["rope_theta"] *= 2
    if case == "model-type": raw["model_type"] = "granite"
    (tmp_path / "config.json").write_text(json.dumps(raw))

    class Parsed:
        def to_dict(self):
            return copy.deepcopy(parsed)

    monkeypatch.setattr(AutoConfig, "from_pretrained", lambda *a, **k: Parsed())
    with pytest.raises(ValueError):
        W.load_config(tmp_path)


@pytest.mark.gpu
@torch.inference_mode()
def test_checkpoint_on_gpu_generates_as_the_state_dict_model(tmp_path):
    """The model built from a saved checkpoint on the GPU generates the same
    greedy tokens as the one built from the HF state dict."""
    from litemoe_amd.ep import ExpertParallel
    from litemoe_amd.experts import HipFusedExperts
    from litemoe_amd.engine import Request
    from litemoe_amd.model import Granite
    from litemoe_amd.optimized import OptimizedEngine
    geometry = dict(vocab_size=97, hidden_size=256, intermediate_size=128, num_hidden_layers=2,
                    num_attention_heads=4, num_key_value_heads=2, num_local_experts=8, num_experts_per_tok=2,
                    max_position_embeddings=256)
    hf = make_hf(seed=16, **geometry)
    save_checkpoint(hf, tmp_path, shards=2)
    cfg = W.load_config(tmp_path)
    loaded = W.load_weights(cfg, W.CheckpointSource(tmp_path), None, 0, "cuda", torch.bfloat16)
    assert_same_weights(loaded, hf_weights(hf, torch.bfloat16, "cuda"))
    requests = [Request("a", [3, 8, 2], 6), Request("b", [4], 4)]
    outputs = []
    for weights, c in ((loaded, cfg), (hf_weights(hf, torch.bfloat16, "cuda"), config_from_hf(hf.config))):
        ep = ExpertParallel(1, 0, 4096, c.hidden_size, c.num_experts_per_tok, torch.bfloat16, "cuda",
                            HipFusedExperts())
        model = Granite(c, weights, ep, 64)
        outputs.append(OptimizedEngine(model, requests, ignore_eos=True, capacity=16).generate()[0])
    assert outputs[0] == outputs[1]
