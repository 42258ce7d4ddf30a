"""Host logic on the CPU: generators, configuration, request validation,
execution policy, packed layout, argument validation before any launch."""
import subprocess
import sys
from types import SimpleNamespace

import numpy as np
import pytest
import torch

from litemoe_amd import synth
from litemoe_amd.config import ModelConfig, preset, validate_config


def test_bf16_rounding_matches_torch_conversion():
    rng = np.random.RandomState(0)
    values = np.concatenate([rng.standard_normal(100000).astype(np.float32) * 10.0 ** rng.randint(-30, 30, 100000),
                             np.array([0.0, -0.0, np.inf, -np.inf, 1.0, 65504.0, 1e-40, -1e-40], np.float32)])
    # exact halfway cases: low 16 bits 0x8000, with even and odd upper halves
    halfway = (np.arange(0x3F800000, 0x3F800000 + 64 * 0x10000, 0x10000, dtype=np.uint32) | 0x8000).view(np.float32)
    values = np.concatenate([values, halfway])
    ours = synth.bf16_bits(values)
    theirs = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)
    assert synth.bf16_bits(np.array([np.nan], np.float32))[0] == 0x7FC0


def test_generator_is_deterministic_and_seeded_per_tensor():
    cfg = preset("granite-1b", num_hidden_layers=1, vocab_size=64, hidden_size=256, num_attention_heads=4,
                 num_key_value_heads=2, num_local_experts=4, intermediate_size=128)
    a = synth.granite_weights(cfg, seed=3)
    b = synth.granite_weights(cfg, seed=3)
    c = synth.granite_weights(cfg, seed=4)
    assert synth.sha256(a["layers"][0]["input_linear"]) == synth.sha256(b["layers"][0]["input_linear"])
    assert synth.sha256(a["layers"][0]["input_linear"]) != synth.sha256(c["layers"][0]["input_linear"])
    assert a["layers"][0]["input_linear"].shape == (4, 256, 256)
    assert a["layers"][0]["output_linear"].shape == (4, 256, 128)
    std = a["layers"][0]["input_linear"].float().std().item()
    assert abs(std - 0.02) < 0.001
    assert a["head"] is a["embedding"]


def test_presets_and_validation():
    cfg = preset("granite-3b")
    assert (cfg.hidden_size, cfg.num_hidden_layers, cfg.num_local_experts, cfg.head_dim) == (1536, 32, 40, 64)
    with pytest.raises(ValueError, match="GQA"):
        validate_config(ModelConfig(**{**cfg.to_dict(), "num_key_value_heads": 7}))
    with pytest.raises(ValueError, match="logits_scaling"):
        validate_config(ModelConfig(**{**cfg.to_dict(), "logits_scaling": 0}))


def _fake_model():
    cfg = preset("granite-1b", num_hidden_layers=1, vocab_size=50)
    w = {"embedding": torch.zeros(1, device="cpu", dtype=torch.bfloat16), "layers": []}
    ep = SimpleNamespace(backend=SimpleNamespace(graph_safe=True), capacity=0)
    return SimpleNamespace(cfg=cfg, w=w, ep=ep, capacity=4096, trace=None)


@pytest.mark.parametrize("kwargs,requests,match", [
    (dict(mode="bogus"), [("a", [1], 1)], "mode"),
    ({}, [("a", [1], -1)], "budgets"),
    ({}, [("a", [1], 1), ("a", [2], 1)], "unique"),
    ({}, [("a", [], 1)], "vocabulary"),
    ({}, [("a", [60], 1)], "vocabulary"),
    ({}, [("a", [1] * 4000, 200)], "context"),
    (dict(capacity=4), [("a", [1, 2, 3], 3)], "capacity"),
    (dict(world=2), [("a", [1], 1)], "world"),
    ({}, [("a", [1], 2)], "GPU"),
])
def test_engine_rejects_invalid_requests(kwargs, requests, match):
    from litemoe_amd.engine import Engine, Request
    with pytest.raises(ValueError, match=match):
        Engine(_fake_model(), [Request(*r) for r in requests], **kwargs)


def test_empty_requests_return_without_gpu():
    from litemoe_amd.engine import Engine, Request
    engine = Engine(_fake_model(), [Request("z", [], 0)])
    assert engine.generate()[0] == {"z": []}


def test_policy_key_and_restore_on_failure():
    """Reference test_fused_norm.py:15-48 / test_moe_finish.py:8-17: changing a
    captured policy requires a new engine; flags are restored on exit/failure."""
    from litemoe_amd.optimized import optimized_policy
    model = SimpleNamespace(decode_flash=None, decode_lean=False, prefill_lean=False,
                            ep=SimpleNamespace(decode_lean=False, backend=SimpleNamespace(native=True, fused_combine=True)),
                            w={"layers": [{"logical": torch.empty(0)}]})
    run = SimpleNamespace(model=model, world=1, requests=[SimpleNamespace(prompt=[1, 2], budget=3)], capacity=8,
                          lean_decode=True, flash_decode=True, flash_attention="flash", graph=None)
    with pytest.raises(RuntimeError, match="injected"):
        with optimized_policy(run):
            with optimized_policy(run):
                assert model.decode_lean and model.decode_flash == "flash" and model.prefill_lean
            raise RuntimeError("injected")
    assert not model.decode_lean and model.decode_flash is None and not model.prefill_lean
    with optimized_policy(run):
        run.graph = object()
    run.flash_decode = False
    with pytest.raises(ValueError, match="Recreate"):
        with optimized_policy(run):
            pytest.fail("captured policy changed silently")
    run.flash_decode = True
    model.w["layers"][0]["logical"] = torch.tensor([1, 0])
    with pytest.raises(ValueError, match="Recreate"):  # lean needs identity placement
        with optimized_policy(run):
            pass


def test_packed_layout():
    from litemoe_amd.packed import build_packed
    packed, ends = build_packed([3, 1, 2], "cpu", slot_start=4)
    assert packed.cu.tolist() == [0, 3, 4, 6] and packed.maximum == 3
    assert packed.positions.tolist() == [0, 1, 2, 0, 0, 1]
    assert packed.slots.tolist() == [4, 4, 4, 5, 6, 6]
    assert ends.tolist() == [3, 4, 6]
    with pytest.raises(ValueError, match="nonempty"):
        build_packed([2, 0], "cpu")


def test_host_validation_before_launch():
    from litemoe_amd import moe_finish, norm
    from litemoe_amd.ep import ExpertParallel
    from litemoe_amd.flash_decode import FlashDecode
    x = torch.zeros(2, 8, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="contiguous CUDA"):
        norm.rmsnorm(x, torch.ones(8, dtype=torch.bfloat16), 1e-6)
    ids = torch.zeros(2, 2, dtype=torch.int32)
    with pytest.raises(ValueError, match="one CUDA device"):
        moe_finish.finish(torch.zeros(4, 8), ids, torch.arange(4), torch.ones(2, 2), x, 0, 1)
    with pytest.raises(ValueError, match="length bound"):
        FlashDecode(2, 2, 2, 256, "cpu", maximum=257)
    with pytest.raises(ValueError, match="world"):
        ExpertParallel(2, 0, 8, 8, 2, torch.bfloat16, "cpu", None)


def test_bench_refuses_multi_gpu():
    out = subprocess.run([sys.executable, "bench.py", "--gpus", "2"], capture_output=True, text=True,
                         cwd=str(__import__("pathlib").Path(__file__).resolve().parents[1]))
    assert out.returncode == 2 and "one GPU" in out.stderr


def test_workspace_growth_keeps_handed_out_buffers():
    """A captured graph keeps the address of the scratch it was given, so a
    larger request must not release the earlier buffer (its storage stays
    referenced and unchanged)."""
    from litemoe_amd.experts import _Workspace
    ws = _Workspace()
    small = ws.get("cpu", 1000)
    address = small.data_ptr()
    assert ws.get("cpu", 800) is small  # fits: reused
    large = ws.get("cpu", 5000)
    assert large.numel() >= 5000 and large.data_ptr() != address
    assert any(buf.data_ptr() == address for buf in ws.retired)
    del small
    assert any(buf.data_ptr() == address for buf in ws.retired)
    assert ws.get("cpu", 5000) is large


def test_graph_recording_runs_with_the_collector_off():
    """A recording starts after a collection and runs with automatic
    collection off (a dead cycle freed mid-capture could make a forbidden
    runtime call); the collector's state is restored, also on an error."""
    import gc

    from litemoe_amd.execution import no_collection_while_recording

    class Cycle:
        def __init__(self):
            self.me = self

    freed = []
    Cycle.__del__ = lambda self: freed.append(1)
    Cycle()  # unreachable, kept alive only by its cycle
    assert gc.isenabled()
    with no_collection_while_recording():
        assert freed == [1]  # collected before the recording starts
        assert not gc.isenabled()
    assert gc.isenabled()
    with pytest.raises(RuntimeError):
        with no_collection_while_recording():
            raise RuntimeError("capture failed")
    assert gc.isenabled()
    gc.disable()
    try:
        with no_collection_while_recording():
            assert not gc.isenabled()
        assert not gc.isenabled()  # a caller that had it off keeps it off
    finally:
        gc.enable()


def test_capacity_zero_chooses_like_none():
    """The reference picks a capacity for any falsy value (`capacity or ...`,
    litemoe/engine.py:47): 0 and None give the same plan."""
    from litemoe_amd.engine import plan_requests
    from litemoe_amd.engine import Request
    cfg = preset("granite-1b", num_hidden_layers=1, vocab_size=50)
    reqs = [Request("a", [1, 2, 3], 4), Request("b", [5], 2)]
    for mode in ("eager", "graph"):
        assert plan_requests(reqs, cfg, mode, 0, 4096).capacity == plan_requests(reqs, cfg, mode, None, 4096).capacity
    assert plan_requests(reqs, cfg, "eager", 0, 4096).capacity == 6
    assert plan_requests(reqs, cfg, "graph", 0, 4096).capacity == 8


def test_output_ring_dropped_during_capture_is_parked(monkeypatch):
    """A ring freed while a stream capture runs keeps its pinned slots and
    events alive (their release is a runtime call a capture forbids) until
    release_parked() runs outside the capture."""
    from litemoe_amd import execution
    host, events = object(), [object(), object()]
    ring = execution.OutputRing.__new__(execution.OutputRing)
    ring.asynchronous, ring.host, ring.events = True, host, events
    monkeypatch.setattr(execution, "_capturing", lambda: True)
    del ring
    assert execution._PARKED and execution._PARKED[-1] == (host, events)
    execution.release_parked()  # still capturing: kept
    assert execution._PARKED
    monkeypatch.setattr(execution, "_capturing", lambda: False)
    execution.release_parked()
    assert execution._PARKED == []
    ring = execution.OutputRing.__new__(execution.OutputRing)
    ring.asynchronous, ring.host, ring.events = True, host, events
    del ring  # outside a capture: freed at once
    assert execution._PARKED == []
