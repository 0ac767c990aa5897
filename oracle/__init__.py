"""CPU restatement of HS-Guard's streaming slot step -- TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it. The shipped path (``hs-guard_amd/hs_guard``) never
imports it and fails loudly when the HIP library is missing.

Every function restates the reference algorithm it cites (paths relative to the HS-Guard repository) in
numpy, computing in float64 unless a reference rounding point says otherwise (bf16 rounding is applied
exactly where the reference rounds). Pinning of each function is listed in its docstring; the tests in
``tests/test_oracle_*.py`` carry the checks.

Modules:
  bf16     -- round-to-nearest-even bf16 / fp16 helpers
  pack     -- pack_inputs (slot_engine_v7.py:7-25) and the ring_pos / length bookkeeping
  gdn      -- gated-delta-rule recurrent slot step (fused_kernels.py:140-211) and its chunked WY/UT form
  ring     -- window-512 ring attention with gate and ring write (fused_kernels.py:288-376,
              ring_attention_kernel.py:7-26)
  glue     -- conv+SiLU pool update, RMSNorms, norm+RoPE, SiLU-mul, risk head
  backbone -- the whole streaming step (slot_engine_v8.py:30-89) over per-slot pools
"""
