"""Write golden vectors of the reference's CPU expert path for BASELINE config 1.

Runs ONLY in the build container, where the reference checkout exists
(/root/reference, read-only). It imports the reference's own
``litemoe.ops.reference_experts`` (ops.py:25-56: per-row bf16 GEMMs, silu,
bf16 scale multiply, bf16 index_add combine) because the exact bf16 bits of
that path are pinned by nothing else. Inputs are regenerated from seeds by
litemoe_amd.synth (numpy legacy stream), so only outputs and input hashes are
stored.

Config 1: hidden 1024, 32 experts, top-8, intermediate 512, 16 decode tokens;
weights N(0, 0.02) (seed 0, one stream per tensor), hidden states N(0, 1)
(seed 1). Router as the reference CPU path computes it (model.py:110,115-118):
scores = F.linear(x, W_r) in bf16; top, ids = scores.float().topk(8);
scales = top.softmax(-1).to(bf16); EP1 then passes scales.float() (ep.py:48).
"""
import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from litemoe_amd import synth  # noqa: E402


def inputs():
    h, e, i, m = 1024, 32, 512, 16
    wr = synth.normal_bf16((e, h), 0.02, synth.tensor_seed(0, 0))
    w1 = synth.normal_bf16((e, 2 * i, h), 0.02, synth.tensor_seed(0, 1))
    w2 = synth.normal_bf16((e, h, i), 0.02, synth.tensor_seed(0, 2))
    x = synth.normal_bf16((m, h), 1.0, synth.tensor_seed(1, 0))
    return x, wr, w1, w2


def main():
    sys.path.insert(0, "/root/reference")
    from litemoe.ops import reference_experts
    torch.set_num_threads(1)
    x, wr, w1, w2 = inputs()
    scores = F.linear(x, wr)
    top, ids = scores.float().topk(8, dim=-1)
    scales = top.softmax(-1).to(torch.bfloat16)
    out = reference_experts(x, ids, scales.float(), w1, w2, singleton=True)
    batched = reference_experts(x, ids, scales.float(), w1, w2, singleton=False)
    np.savez(HERE / "reference_experts_cfg1.npz",
             scores=scores.view(torch.int16).numpy(), ids=ids.numpy(),
             scales=scales.view(torch.int16).numpy(), out=out.view(torch.int16).numpy(),
             out_batched=batched.view(torch.int16).numpy())
    manifest = {name: synth.sha256(t) for name, t in (("x", x), ("wr", wr), ("w1", w1), ("w2", w2))}
    manifest["torch"] = torch.__version__
    manifest["source"] = "litemoe/ops.py:25-56 reference_experts (singleton=True and False), model.py:110,115-118"
    (HERE / "reference_experts_cfg1.json").write_text(json.dumps(manifest, indent=1) + "\n")
    print("wrote", HERE / "reference_experts_cfg1.npz")


if __name__ == "__main__":
    main()
