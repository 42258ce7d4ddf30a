"""The decode fast-path policy and the engine that runs under it.

The reference scopes its fast paths with a context manager
(litemoe/optimized.py:23-54) and runs prefill, capture and eager steps
inside it (optimized.py:57-90). Here the policy is a value:
:class:`DecodePolicy` is resolved from an engine (validating it as the
reference does, with the same messages), compared with the policy a graph
was captured under, and applied to the model for the duration of one call
by :func:`optimized_policy`.

The policy chooses:
* ``flash`` -- the engine's :class:`FlashDecode`, bounded by its longest
  request, as the model's decode attention;
* ``lean`` -- stopped rows keep position 0 and their outputs are not masked,
  which lets the layer tail run fused (``Granite.greedy_step``). It needs
  this library's experts (the ``native`` capability) and the identity
  expert placement, as the reference's lean mode needs vLLM's experts and
  the identity placement (optimized.py:32-33);
* ``prefill_lean`` -- lean and the engine's ``lean_prefill``: the batched
  prefill packs every prompt into one ragged batch
  (``packed.optimized_prefill_logits``, optimized.py:46).
"""
from contextlib import contextmanager
from dataclasses import dataclass

from .batch import BatchPrefillEngine
from .flash_decode import FlashDecode
from .packed import optimized_prefill_logits

_MODEL_FLAGS = ("decode_flash", "decode_lean", "prefill_lean")


@dataclass(frozen=True)
class DecodePolicy:
    capacity: int
    limit: int          # longest prompt + budget - 1 over the requests
    backend: int        # identity of the expert backend object
    flash: bool
    fused_combine: bool
    lean: bool

    @classmethod
    def resolve(cls, run):
        if run.world != 1:
            raise ValueError("Optimized execution currently requires EP1")
        limit = max((len(r.prompt) + r.budget - 1 for r in run.requests), default=1)
        if limit > run.capacity:
            raise ValueError("Optimized attention exceeds KV capacity")
        model = run.model
        backend = model.ep.backend
        identity = all(w["logical"].numel() == 0 for w in model.w["layers"])
        lean = bool(run.lean_decode and getattr(backend, "native", False) and identity)
        return cls(run.capacity, limit, id(backend), bool(run.flash_decode),
                   bool(getattr(backend, "fused_combine", False)), lean)

    def settings(self, run):
        """Model attribute values under this policy."""
        return {"decode_flash": run.flash_attention if self.flash else None, "decode_lean": self.lean,
                "prefill_lean": self.lean and bool(getattr(run, "lean_prefill", True))}


@contextmanager
def optimized_policy(run):
    """Apply the engine's policy to its model for the body; flags are
    restored afterwards, also on error. Once a graph has been captured under
    a policy, any other policy is refused: the recorded step would no longer
    match it."""
    policy = DecodePolicy.resolve(run)
    captured = getattr(run, "_optimized_graph_policy", None)
    if run.graph is not None and captured != policy:
        raise ValueError("Recreate Engine before changing captured execution policy")
    model = run.model
    saved = {name: getattr(model, name) for name in _MODEL_FLAGS}
    saved_ep = model.ep.decode_lean
    for name, value in policy.settings(run).items():
        setattr(model, name, value)
    model.ep.decode_lean = policy.lean
    try:
        yield policy
    finally:
        if run.graph is not None and captured is None:
            run._optimized_graph_policy = policy
        for name, value in saved.items():
            setattr(model, name, value)
        model.ep.decode_lean = saved_ep


class OptimizedEngine(BatchPrefillEngine):
    flash_decode = True
    lean_decode = True
    lean_prefill = True
    prefill_function = staticmethod(optimized_prefill_logits)

    def __init__(self, *args, num_splits=None, **kwargs):
        super().__init__(*args, **kwargs)
        self.flash_attention = None
        if not self.requests:
            return
        cfg = self.model.cfg
        prompts = [len(r.prompt) for r in self.requests]
        longest = max(n + r.budget - 1 for n, r in zip(prompts, self.requests))
        # A ragged batch (longest prompt above 1.25x the shortest) dispatches
        # its attention rows longest first.
        ragged = max(prompts) > 1.25 * min(prompts)
        self.flash_attention = FlashDecode(self.batch, cfg.num_key_value_heads,
                                           cfg.num_attention_heads // cfg.num_key_value_heads,
                                           self.capacity, self.device, longest, num_splits, ordered=ragged)

    def prepare_graph(self):
        with optimized_policy(self):
            return super().prepare_graph()

    def prefill(self):
        with optimized_policy(self):
            return super().prefill()

    def decode_step(self):
        with optimized_policy(self):
            return super().decode_step()
