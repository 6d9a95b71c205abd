"""CPU oracle for the GGUF quantized-matmul path.

TEST INFRASTRUCTURE ONLY. Nothing in the product package (``dracort_amd``)
imports, links or executes anything under ``oracle/``. Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` use
it, and only as the checker or as the timed CPU restatement of the reference
path -- never as the thing being measured on the GPU.

Contents
--------
``gguf_ref``     numpy restatement of the reference GGUF block dequantizer
                 (``draco/format/gguf.py:53-87,256-259,272-316,425-468,470-495``),
                 op-for-op so the fp32 rounding sequence is identical.
``loop_ref``     plain-loop K-quant decoders restated from the reference's own
                 independent test decoders (``tests/format/test_gguf.py:281-337``).
``encoders``     the reference's Q8_0 / Q4_0 test encoders
                 (``tests/format/test_gguf.py:145-169``), the "repo's quantizer"
                 for the Q8_0 / Q4_0 configurations.
``matmul_ref``   fp64 closed forms for the dequant-then-matmul
                 (``draco/runtime/cpu/kernels/generic.py:32-33``) and the MoE FFN
                 (``draco/models/moe/router.py:81-120``,
                 ``draco/models/moe/expert.py:47-49,77-116``), the acceptance
                 metric, and the reference's own fp32 numpy matmul used as the
                 timed CPU baseline.

Pinning status (what checks each function, in ``tests/test_oracle.py``)
-----------------------------------------------------------------------
* ``gguf_ref.dequantize`` Q8_0 / Q4_0 / Q4_K / Q6_K: golden vectors written by
  running the reference ``_dequantize`` (``tests/golden/make_golden.py``), the
  reference's known-answer K-quant blocks, the restated loop decoders, and
  closed forms (d = 1, d = 0, power-of-two scales, exhaustive 6-bit scale/min
  unpacking, 6-bit Q6_K code ordering).
* ``encoders``: golden bytes from the reference test encoders, plus the
  reference's round-trip tolerances.
* ``matmul_ref.linear_ref`` / ``moe_ref``: fp64 closed forms, checked against
  brute force on tiny inputs and against exact small-integer cases.  The MoE
  routing semantics have no reference test; they are pinned by the closed form
  (top-2, softmax of the two logits, renormalise, expert-ascending combine).
"""
