"""The emit ring and the step graph on the GPU.

Contract of litemoe/execution.py:6-45 (kept): every step's emit snapshot is
delivered once, in step order, whatever the ring's mechanism. Checked for
the copy mode and for the mode where the greedy epilogue kernel writes the
pinned host slots itself (a system-scope store per value), with the host
running ahead of the device by up to depth - 1 steps.
"""
import pytest
import torch

from litemoe_amd import step
from litemoe_amd.execution import OutputRing, capture_decode

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _state(rows, budget):
    s = {name: torch.zeros(rows, dtype=dtype, device=DEV) for name, dtype in (
        ("next", torch.int64), ("length", torch.int64), ("generated", torch.int64), ("budget", torch.int64),
        ("active", torch.bool))}
    s["budget"].fill_(budget)
    s["active"].fill_(True)
    s["length"].copy_(torch.arange(rows, device=DEV) + 3)
    return s


@pytest.mark.parametrize("device_writes", [False, True])
@pytest.mark.parametrize("depth", [2, 4])
@torch.inference_mode()
def test_ring_delivers_each_step_once_in_order(device_writes, depth):
    rows, vocab, steps = 7, 301, 23
    emit = torch.zeros(rows, 3, dtype=torch.int64, device=DEV)
    delivered = []
    ring = OutputRing(emit, delivered.append, asynchronous=True, depth=depth)
    target = ring.device_target(rows) if device_writes else None
    ring.start()
    s = _state(rows, budget=steps - 4)  # rows stop before the end: later snapshots have valid = 0
    eos = torch.tensor([5], dtype=torch.int64, device=DEV)
    gen = torch.Generator(device=DEV).manual_seed(1)
    snapshots = []
    for n in range(steps):
        logits = torch.randn(rows, vocab, device=DEV, generator=gen).to(torch.bfloat16)
        valid = s["active"].clone()
        if target is not None:
            target[2].add_(1)  # what lm_decode_prologue does for the step
        step.greedy_epilogue(logits, 2.0, valid, s, emit, eos, ignore_eos=True, ring_target=target)
        snapshots.append(emit.clone())  # queued behind the step, before the next one
        ring.publish(n)
        assert len(delivered) >= n + 2 - depth  # the host is never more than depth - 1 steps ahead
    ring.drain()
    assert len(delivered) == steps
    assert delivered == [t.tolist() for t in snapshots]
    assert delivered[-1][0][2] == 0 and delivered[0][0][2] == 1


@torch.inference_mode()
def test_prologue_counts_steps_for_the_ring():
    rows, hidden, vocab = 4, 64, 50
    s = _state(rows, budget=9)
    table = torch.randn(vocab, hidden, device=DEV).to(torch.bfloat16)
    weight = torch.ones(hidden, device=DEV, dtype=torch.bfloat16)
    counter = torch.zeros(1, dtype=torch.int64, device=DEV)
    for _ in range(5):
        step.decode_prologue(s["active"], s["length"], s["next"], table, 1.0, weight, 1e-6, step_counter=counter)
    assert counter.item() == 5


@torch.inference_mode()
def test_step_graph_replays_device_ring_writes():
    """A captured step whose epilogue writes the ring: replays land in
    successive slots, numbered by the captured prologue-side counter."""
    rows, vocab = 3, 97
    emit = torch.zeros(rows, 3, dtype=torch.int64, device=DEV)
    delivered = []
    ring = OutputRing(emit, delivered.append, asynchronous=True, depth=3)
    target = ring.device_target(rows)
    s = _state(rows, budget=100)
    eos = torch.zeros(0, dtype=torch.int64, device=DEV)
    logits = torch.zeros(rows, vocab, device=DEV, dtype=torch.bfloat16)

    def one_step():
        target[2].add_(1)
        logits.zero_()
        logits.scatter_(1, (s["length"] % vocab)[:, None], 1.0)
        step.greedy_epilogue(logits, 1.0, s["active"].clone(), s, emit, eos, ignore_eos=True, ring_target=target)

    def reset():
        s["length"].copy_(torch.arange(rows, device=DEV) + 10)
        s["generated"].zero_()

    graph = capture_decode(one_step, reset)
    ring.start()
    for n in range(8):
        graph.replay()
        ring.publish(n)
    ring.drain()
    tokens = [[row[0] for row in snap] for snap in delivered]
    assert tokens == [[(10 + r + n) % vocab for r in range(rows)] for n in range(8)]
    assert [snap[0][1] for snap in delivered] == list(range(8))
