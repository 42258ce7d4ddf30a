"""Golden vectors written by the reference's own CPU expert path (config 1);
see tests/golden/make_reference_experts.py. The inputs are regenerated from
seeds and checked by SHA-256 before use."""
import json
from pathlib import Path

import numpy as np
import pytest
import torch

from helpers import bf16_within_ulp_or_abs, rel_l2
from litemoe_amd import synth
from oracle import ops

GOLDEN = Path(__file__).resolve().parent / "golden"


@pytest.fixture(scope="module")
def cfg1():
    import importlib.util
    spec = importlib.util.spec_from_file_location("make_golden", GOLDEN / "make_reference_experts.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    x, wr, w1, w2 = mod.inputs()
    manifest = json.loads((GOLDEN / "reference_experts_cfg1.json").read_text())
    for name, t in (("x", x), ("wr", wr), ("w1", w1), ("w2", w2)):
        assert synth.sha256(t) == manifest[name], f"regenerated {name} differs from the fixture's input"
    data = np.load(GOLDEN / "reference_experts_cfg1.npz", allow_pickle=False)
    bf = lambda a: torch.from_numpy(a).view(torch.bfloat16)
    return dict(x=x, wr=wr, w1=w1, w2=w2, scores=bf(data["scores"]), ids=torch.from_numpy(data["ids"]),
                scales=bf(data["scales"]), out=bf(data["out"]), out_batched=bf(data["out_batched"]))


def canonical(scores, ids):
    """Order each row's ids by (logit desc, id asc)."""
    out = []
    for s, row in zip(scores.float(), ids.tolist()):
        out.append(sorted(row, key=lambda e: (-float(s[e]), e)))
    return torch.tensor(out)


def test_oracle_router_reproduces_reference_selection(cfg1):
    """Same selected sets; torch's CPU topk orders equal logits arbitrarily
    (row 10 of this fixture has a tie), the oracle by ascending id."""
    scores = torch.nn.functional.linear(cfg1["x"], cfg1["wr"])
    assert torch.equal(scores, cfg1["scores"])
    top, ids = ops.select_topk(cfg1["scores"], 8)
    assert torch.equal(ids, canonical(cfg1["scores"], cfg1["ids"]))
    tie_rows = (ids != cfg1["ids"]).any(-1).nonzero().flatten().tolist()
    assert tie_rows == [10]
    assert torch.equal(top.softmax(-1).to(torch.bfloat16), cfg1["scales"])


@torch.inference_mode()
def test_oracle_experts_bit_exact_with_reference(cfg1):
    args = (cfg1["x"], cfg1["ids"], cfg1["scales"].float(), cfg1["w1"], cfg1["w2"])
    assert torch.equal(ops.reference_experts(*args, singleton=True), cfg1["out"])
    assert torch.equal(ops.reference_experts(*args, singleton=False), cfg1["out_batched"])
    # the production rounding (fp32 ordered combine) stays within the bar
    fused = ops.fused_moe(cfg1["x"], cfg1["ids"].int(), cfg1["scales"].float(), cfg1["w1"], cfg1["w2"])
    assert rel_l2(fused, cfg1["out"]) < 1e-2


@pytest.mark.gpu
@torch.inference_mode()
def test_gpu_router_and_experts_against_reference_vectors(cfg1):
    from litemoe_amd import experts, router
    dev = "cuda"
    logits = torch.empty(16, 32, device=dev, dtype=torch.bfloat16)
    weights, ids = router.route(cfg1["x"].to(dev), cfg1["wr"].to(dev), 8, logits_out=logits)
    got_logits, ref_logits = logits.cpu(), cfg1["scores"]
    # The kernel's logits are a GEMV in another accumulation order than the
    # reference's CPU product: within one bf16 ulp (2e-3 absolute near zero).
    assert bf16_within_ulp_or_abs(got_logits, ref_logits, 1, 2e-3)
    # Selection: every row whose ids differ from the reference's (canonical
    # tie order) must have a logit that differs; rows with equal logits must
    # select bit-exactly. Checked unconditionally.
    expected_ids = canonical(ref_logits, cfg1["ids"])
    mismatched = (ids.cpu().long() != expected_ids).any(-1)
    logit_differs = (got_logits != ref_logits).any(-1)
    assert not (mismatched & ~logit_differs).any(), mismatched.nonzero().flatten().tolist()
    assert int(mismatched.sum()) <= 1, "more than one row re-ranked by a one-ulp logit difference"
    # and on the kernel's own logits the selection is exact
    _, own = ops.select_topk(got_logits, 8)
    assert torch.equal(ids.cpu().long(), own.long())
    out = experts.fused_experts(cfg1["x"].to(dev), cfg1["w1"].to(dev), cfg1["w2"].to(dev),
                                cfg1["scales"].float().to(dev), cfg1["ids"].int().to(dev)).cpu()
    assert rel_l2(out, cfg1["out"]) < 2e-2
