"""CPU oracle for the altxs per-symbol step -- TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import, call, link or execute anything in this package, and only as
the checker (or as the timed CPU baseline).  The product path
(``altxs_amd``) never imports it and fails loudly when its HIP library is
missing.

Contents (each function cites the reference file:line it restates):

* ``cdf_coder.c`` / :mod:`oracle.coder` -- ``_scale_cum_np`` and the 32-bit
  WNC range coder (src/model/arithmetic_coder_lm.py), plain C, -ffp-contract=off.
* :mod:`oracle.codec_ref` -- mixed-bit codec arithmetic
  (src/hyperflow_distillation/mixed_bit_delta.py:96-229) and the group-64
  symmetric variant, numpy.
* :mod:`oracle.model_ref` -- the fp32 eager step of the reference GPT
  (src/xsa_ttt/model.py), PyTorch on CPU, B=1 per segment.
* :mod:`oracle.stages_ref` -- the stage-fused FFN kernels with their bf16
  rounding points (src/xsa_ttt/ac_gemv.py:89-310) and the split attention's
  result (src/xsa_ttt/split_attn.py), numpy.

Pinning (what fixes each function beyond retyping the formula) is listed in
each module's docstring; see also tests/golden/.
"""
