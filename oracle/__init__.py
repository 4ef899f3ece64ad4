"""CPU oracle of the diffusion attention path -- TEST INFRASTRUCTURE ONLY.

A numpy restatement of what dLLM-Serve's attention hot path computes
(dllmserve/layers/attention.py, sparse/state.py, engine/sequence.py,
engine/model_runner.py:152-321, layers/rotary_embedding.py).  Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and
only as the checker; the product path (dllm-serve_amd/) never does.

Modules
  bf16       bf16 <-> f32 bit conversions (round to nearest even)
  attention  varlen bidirectional attention, block-vs-cache attention and the
             per-sequence mode semantics of _mixed_sparse_dense_attention
  select     head / token KV selection with the explicit rounding and
             tie-break rule the GPU kernels implement
  kvcache    store_kvcache / load_kvcache by slot
  rope       NeoX rotary embedding (input preparation; checker of the K7 kernel)
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
The reference's own tests hold no numeric fixtures for this path, and its
package cannot be imported here (it needs flash_attn), so no function is
pinned against reference-produced vectors.
"""
