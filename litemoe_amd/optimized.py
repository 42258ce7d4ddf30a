"""Execution policy for the fused decode path (litemoe/optimized.py:23-90).

``optimized_policy(run)`` scopes the model's fast-path flags to one
prefill/decode/capture: lean decode (stopped rows keep position 0 and their
outputs are not masked; requires identity placement) and a ``FlashDecode``
bounded by the longest request. A graph captured under one policy key may
not be replayed under another ("Recreate Engine"), as optimized.py:34-37.
"""
from contextlib import contextmanager

from .engine import Engine
from .flash_decode import FlashDecode


@contextmanager
def optimized_policy(run):
    model = run.model
    if run.world != 1:
        raise ValueError("Optimized execution currently requires EP1")
    limit = max((len(r.prompt) + r.budget - 1 for r in run.requests), default=1)
    if limit > run.capacity:
        raise ValueError("Optimized attention exceeds KV capacity")
    lean = run.lean_decode and getattr(model.ep.backend, "native", False) and all(
        w["logical"].numel() == 0 for w in model.w["layers"])
    key = (run.capacity, limit, id(model.ep.backend), run.flash_decode,
           getattr(model.ep.backend, "fused_combine", False), lean)
    if run.graph is not None and getattr(run, "_optimized_graph_policy", None) != key:
        raise ValueError("Recreate Engine before changing captured execution policy")
    previous = (model.decode_flash, model.decode_lean, model.ep.decode_lean)
    model.decode_flash = run.flash_attention if run.flash_decode else None
    model.decode_lean = model.ep.decode_lean = lean
    try:
        yield
    finally:
        if run.graph is not None:
            run._optimized_graph_policy = key
        model.decode_flash, model.decode_lean, model.ep.decode_lean = previous


class OptimizedEngine(Engine):
    flash_decode = True
    lean_decode = True

    def __init__(self, *args, num_splits=None, **kwargs):
        super().__init__(*args, **kwargs)
        cfg = self.model.cfg
        self.flash_attention = None
        if self.requests:
            maximum = max(len(r.prompt) + r.budget - 1 for r in self.requests)
            # A ragged batch (the longest prompt more than 1.25x the shortest)
            # dispatches its attention rows longest first.
            lengths = [len(r.prompt) for r in self.requests]
            ragged = max(lengths) > 1.25 * min(lengths)
            self.flash_attention = FlashDecode(self.batch, cfg.num_key_value_heads,
                                               cfg.num_attention_heads // cfg.num_key_value_heads,
                                               self.capacity, self.device, maximum, num_splits,
                                               ordered=ragged)

    def prepare_graph(self):
        with optimized_policy(self):
            return super().prepare_graph()

    def prefill(self):
        with optimized_policy(self):
            return super().prefill()

    def decode_step(self):
        with optimized_policy(self):
            return super().decode_step()
