"""CPU oracle for the FP16 D=64 attention forward - TEST INFRASTRUCTURE ONLY.

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
"""

from oracle.reference import (
    attention_float64_rowwise,
    attention_reference,
    attention_reference_fp32,
    attention_rows_fp32,
    flash_forward_tiled,
    validate_inputs,
)

__all__ = [
    "attention_float64_rowwise",
    "attention_reference",
    "attention_reference_fp32",
    "attention_rows_fp32",
    "flash_forward_tiled",
    "validate_inputs",
]
