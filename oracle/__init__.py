"""CPU oracle of the DiT attention path: TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this package, and only as the checker (or the timed CPU baseline). The product
path (h3metal_amd) never calls it and fails loudly when its HIP library is
missing.

  oracle.prepass    float32 op-by-op restatement of qk_norm_rope
                    (reference kernels/ops.metal:365-468)
  oracle.rot_q8     float32 op-by-op restatement of rot_q8, the row rotation +
                    int8 that consumes the attention output
                    (reference kernels/ops.metal:272-334)
  oracle.gemm       the int8 projection product (reference kernels/gemm.metal,
                    weight format q8): exact integer product, float32 epilogue
  oracle.attention  float64 softmax attention (reference tests/test_attention.py:9-21)
                    and exact integer scores
  oracle.bf16       bf16 <-> float32 conversions (round to nearest even)

How each function is pinned (checks that do not retype its formula) is in
tests/test_oracle.py. The reference ships no golden vectors, and its kernels
are Metal code that cannot be built or run here, so nothing is compared with
the reference's own output; see each function's docstring for its status.
"""
