"""CPU oracle for the attention forward and the module's other operators - TEST INFRASTRUCTURE ONLY.

This package restates the reference's semantics on the CPU so the HIP kernel can be
checked against them. It is never part of the product path: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may import
it, and only as the checker or as the timed CPU baseline. The product
(``flash_attention_2_lab_amd``) never imports it and has no CPU fallback.

Contents (each function cites the reference file:line it restates):

* ``attention_reference``        - FP32 softmax(Q K^T * s [+ causal]) V, cast to the
                                   input dtype (flash_attention/reference.py:9-61).
* ``attention_reference_fp32``   - the same, returning the FP32 result before the cast.
* ``validate_inputs``            - input checks (flash_attention/reference.py:65-100).
* ``attention_rows_fp32``        - the FP32 result for a subset of (batch, head, query
                                   row) triples, for shapes too large to materialise.
* ``attention_float64_rowwise``  - independent float64 per-row evaluation (numpy), for
                                   tiny shapes.
* ``flash_forward_tiled``        - model of the reference production kernel's
                                   arithmetic: 128-key tiles, FP32 online softmax, P
                                   rounded to FP16 for P.V, FP32 denominator
                                   (csrc/tensorcore_attention.cu:2229-2561, 448-671).
* ``attention_scores_fp32``      - FP32 Q K^T * s, [B, H, N, N] (naive_attention_scores,
                                   csrc/naive_attention.cu:174-201, 330-418).
* ``matmul_16x64x16_fp32``       - FP32 product of [b, 16, 64] and [b, 64, 16] FP16
                                   matrices (wmma_matmul_16x64x16,
                                   csrc/wmma_matmul.cu:51-193).
The FP32 SIMT forwards (naive, block, tiled, tilewise) are checked against
``attention_reference_fp32``, which is what the reference's tests use for them.

How each is pinned (tests/test_oracle.py):
  attention_reference       - torch's scaled_dot_product_attention on CPU (a library
                              routine, as reference tests/test_reference.py:10-52 does),
                              the float64 row-wise evaluation, closed-form known answers
                              (default/custom scale, causal row 0 = V[0], constant V,
                              Q = 0 gives prefix means) and planted-mistake mutants.
  attention_float64_rowwise - agrees with SDPA in float64 and with the closed forms.
  attention_rows_fp32       - equals attention_reference on every sampled row.
  flash_forward_tiled       - within the kernel tolerance of attention_reference, and
                              exactly equal to it in FP32 when the FP16 rounding of P is
                              switched off and one tile covers the sequence.
  attention_scores_fp32     - a float64 loop over (i, j, d) on small inputs, and the
                              known answer of constant per-(batch, head) inputs
                              (reference tests/test_naive_scores.py:71-107).
  matmul_16x64x16_fp32      - a float64 loop on random inputs, and the identity-block
                              known answer A [I; 0] = A[:, :, :16]
                              (reference tests/test_wmma_matmul.py:13-75).
"""

from oracle.reference import (
    attention_float64_rowwise,
    attention_scores_fp32,
    matmul_16x64x16_fp32,
    attention_reference,
    attention_reference_fp32,
    attention_rows_fp32,
    flash_forward_tiled,
    validate_inputs,
)

__all__ = [
    "attention_float64_rowwise",
    "attention_scores_fp32",
    "matmul_16x64x16_fp32",
    "attention_reference",
    "attention_reference_fp32",
    "attention_rows_fp32",
    "flash_forward_tiled",
    "validate_inputs",
]
