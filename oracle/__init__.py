"""CPU restatement of Vesper's quantized MoE expert arithmetic -- TEST INFRASTRUCTURE ONLY.

This package is the parity oracle for the MI355X kernels in ``vesper_amd``. It is
imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, and there only as the checker (or the timed CPU baseline),
never as the product path. ``vesper_amd`` never imports it and fails loudly when
its HIP library is missing.

Every function cites the reference file:line whose behaviour it restates
(paths relative to the shell-term/vesper checkout). The code is written from
the behaviour, not copied: encoders use bit arithmetic where the reference
searches a table, and the tests check each against an independent method.

Pinning status (what checks each function):
  formats.fp4_values / e8m0_values / e4m3_values  exhaustive code tables + reference goldens
  formats.encode_e4m3                             brute-force nearest search over all finite BF16
                                                  + midpoints +-1 ulp, torch float8 cast, goldens
  formats.bf16_bits                               reference goldens + torch bfloat16 cast
  formats.quantize_activation                     reference golden (zero -> 105) + closed form
  formats.mxfp4_gemv_spec                         exact Fraction dot on small shapes + goldens
  expert.expert_forward                           stage op order; exp stages via float64 exp
  router.topk_indices                             232 recorded CUDA selection cases (E=384, k=6),
                                                  tie goldens, brute-force sort on untied input
  router.route_weights                            recorded weight bits (k=6); k=8 tree is
                                                  "parity unpinned" beyond the k=6 restriction
  moe.participation / moe.combine                 38 recorded aggregation cases (SHA-256 of every
                                                  stage) + the reference's negative controls
  projections.fp8_block128_gemm_fp32             exact float64 block dots + closed-form scaling
"""
