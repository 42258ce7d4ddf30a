"""Right-padded batched prefill with request-local KV slots (EP1).

The reference's ``batch`` module (litemoe/batch.py:7-64): ``prepare_batch``
sizes the expert output buffer, ``prefill_logits`` runs one right-padded
batch through ``Granite.forward(..., slot=slice(...), last=...)``,
``bucket_prefill_logits`` groups prompts whose lengths stay within a factor
8, and ``BatchPrefillEngine`` prefills all requests with one such call.
On this path the model runs a padded batch on the packed kernels (its valid
tokens form one packed sequence per row), so padding costs no attention or
expert work.
"""
import torch

from .engine import Engine


def prepare_batch(model, tokens):
    if model.ep.world != 1:
        raise ValueError("Batched Prefill requires EP1")
    model.ep.capacity = max(model.ep.capacity, tokens)
    model.ep.prepare(tokens)


def prefill_logits(model, prompts, cache, slot_start=0):
    """Last-position logits ``[len(prompts), 1, V]`` of one right-padded
    batch written to cache rows ``slot_start ..``."""
    device = cache.k.device
    lengths = torch.tensor([len(x) for x in prompts], device=device)
    width = max(map(len, prompts))
    tokens = torch.tensor([x + [0] * (width - len(x)) for x in prompts], device=device)
    positions = torch.arange(width, device=device)[None].expand(len(prompts), -1)
    valid = positions < lengths[:, None]
    return model.forward(tokens, positions, valid, cache, slot=slice(slot_start, slot_start + len(prompts)),
                         last=lengths - 1)


def bucket_prefill_logits(model, prompts, cache, slot_start=0):
    """Contiguous groups of prompts whose lengths stay within a factor 8,
    each prefilled as one padded batch."""
    outputs, start = [], 0
    while start < len(prompts):
        end = start + 1
        low = high = len(prompts[start])
        while end < len(prompts):
            length = len(prompts[end])
            if max(high, length) > 8 * min(low, length):
                break
            low, high = min(low, length), max(high, length)
            end += 1
        group = prompts[start:end]
        prepare_batch(model, len(group) * max(map(len, group)))
        outputs.append(prefill_logits(model, group, cache, slot_start + start))
        start = end
    return outputs[0] if len(outputs) == 1 else torch.cat(outputs)


class BatchPrefillEngine(Engine):
    """An :class:`Engine` whose prefill is one batched call of
    ``prefill_function`` instead of one forward per request."""
    prefill_function = staticmethod(prefill_logits)

    def __init__(self, *args, **kwargs):
        super().__init__(*args, **kwargs)
        if self.world != 1:
            raise ValueError("Batched Prefill requires EP1")
        if self.requests:
            prepare_batch(self.model, self.batch * max(len(r.prompt) for r in self.local))

    def prefill(self):
        if getattr(self.model, "trace", None):
            raise ValueError("Batched Prefill does not support per-request traces")
        first = self.prefill_function(self.model, [r.prompt for r in self.local], self.cache)[:, 0].argmax(-1)
        self.start_rows(first)
