"""CPU oracle of the diffusion attention path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of what dLLM-Serve's attention hot path computes
(dllmserve/layers/attention.py, sparse/state.py, engine/sequence.py,
engine/model_runner.py:152-321, layers/rotary_embedding.py).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and
only to compute expected results; the product path (dllm-serve_amd/) never does.

Modules
  bf16       bf16 <-> f32 bit conversions (round to nearest even)
  attention  varlen bidirectional attention, block-vs-cache attention and the
             per-sequence mode semantics of _mixed_sparse_dense_attention
  select     head / token KV selection with the explicit rounding and
             tie-break rule the GPU kernels implement
  kvcache    store_kvcache / load_kvcache by slot
  rope       NeoX rotary embedding (input preparation; expected results of the K7 kernel)
  sampler    low-confidence remasking: softmax-max of logit rows (with the
             Gumbel transform at temperature > 0) and the unmasking step
  step       per-step inputs of a batch: sparse state and its advance, rows
             fed and positions, cu_seqlens_k, slot lists
  configs    seeded synthetic inputs of the benchmark configurations

Parity pins (what checks each function; see tests/test_oracle_*.py):
  attention  torch scaled_dot_product_attention (library routine), fp64 vs
             fp32, closed-form special cases and invariants
  select     exact rational arithmetic + full sort on small inputs, torch.topk
             on tie-free inputs, torch bf16 einsum agreement, special cases
  kvcache    brute-force loops, round trips, untouched-slot sentinels
  rope       norm preservation, relative-position invariance, position 0,
             quarter-turn / half-turn tables (exact swaps and negations),
             agreement with the torch f32 expression
  sampler    torch's CPU softmax + max on the same bf16 rows, closed forms,
             planted exact and rounding ties; torch.topk on tie-free
             confidences, counting and tie-order invariants; the published
             SplitMix64 outputs, the reference's add_gumbel_noise ops on the
             same draws, Gumbel-max frequencies against softmax
  step       hand-derived state sequences for delay 0 / 1 / 2 / 5, block
             spans (including the reference's past-the-end over-count), n_keep
             and slot-list closed forms on hand-checked cases
The reference's own tests hold no numeric fixtures for this path, and its
package cannot be imported here (it needs flash_attn), so no function is
pinned against reference-produced vectors.
"""
