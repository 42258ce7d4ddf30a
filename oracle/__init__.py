"""CPU oracle of LiteMoE's MoE decode/prefill hot path — TEST INFRASTRUCTURE ONLY.

A restatement, in torch on the CPU, of the reference algorithm
(ZhuLinsen/LiteMoE, read-only at /root/reference; file:line cited on every
function). It is the checker the GPU parity tests compare the gfx950 kernels
against. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import it; the product package ``litemoe_amd``
never does, and has no CPU fallback.

How each part is pinned (the tests that do it are named in brackets):
  ops.select_topk / route      brute force over subsets, HF GraniteMoeTopKRouter
                               [tests/test_oracle_pins.py]
  ops.permutation              independent counting sort
  ops.reference_experts        the hand-computed known answer of the reference's
                               test_core.py:22-36 example, EP-split/linearity
                               invariants, and golden vectors written by the
                               reference's own ops.py in this container
                               (tests/golden/)
  ops.finish                   exact sums on bf16-exact inputs; rel-L2 vs combine
  ops.rmsnorm / rope_tables    HF GraniteMoe RMSNorm / rotary tables (bitwise)
  ops.kv_store                 index formula brute force (loop over every element)
  ops.decode_attention /       torch.nn.functional.scaled_dot_product_attention
    varlen_attention
  granite.Granite              HF GraniteMoeForCausalLM logits (fp32, 2e-6) and
                               HF greedy generation
"""
