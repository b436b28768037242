"""CPU oracle for the Wan2.2 DiT-block hot path -- TEST INFRASTRUCTURE ONLY.

A restatement, in numpy / torch-on-CPU, of the reference's arithmetic for this path
(reecedantin/vllm-omni-neuron). Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
CPU-baseline leg may import it, and only to check results or as the reported CPU baseline; the
product package never imports it and has no CPU fallback.

Modules and what pins each:

- ``fp8``: e4m3fn / bf16 rounding and e8m0 scales, bit level. Pinned against torch's own
  float8_e4m3fn and bfloat16 casts on every bf16 bit pattern plus random fp32 and ties.
- ``mx``: MX block quantization (shared exponent = block max - 7) and ROW packing. Pinned by
  known-answer blocks whose codes follow from the rule by hand, and by dequantization bounds.
- ``adaln``: the canonical fused adaLN (fixed-order fp32 row statistics in the kernel's lane
  order). Pinned against ``math.fsum`` sums within the fp32 error bound, the distance to
  ``F.layer_norm`` / the eager restatement, and LayerNorm invariants.
- ``rope``: Wan 3D RoPE tables, interleaved rotation and the across-heads RMSNorm. Pinned by
  closed-form angles, norm preservation, the rotate-half equivalence, and closed-form norms of rows
  whose heads differ in scale (fails a per-head norm) or sit near eps (fails a misplaced eps).
- ``attention``: exact softmax attention and the constant-max form. Pinned by fp64 brute force,
  invariance to the subtracted constant, and the underflow clamp.
- ``gemm``: MXFP8 dequantized fp64 products and GELU-tanh. Pinned by scalar brute-force loops on
  tiny shapes (codes decoded by torch's own float8 cast; block, row and column scales and bias
  placement), published values of the GELU tanh approximation, and the transposed weight layout.
- ``block``: the Wan transformer block composed from the above (MXFP8 path and BF16 eager path).
"""
