"""CPU oracle for the MoE expert hot path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (and in plain C under ``oracle/c``), the reference's
arithmetic for the expert-FFN path: MXFP4 / FP8 formats, routers, the token->expert
permute, the fp32 dequant-then-matmul expert FFN, the shared expert, the combine,
MTP acceptance and the slot-cache replacement policy.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it, and only as the checker or the timed CPU baseline.
The product (``whallm_amd``) never imports it and has no CPU fallback.

Pinning status of each module is stated in its own header.
"""
