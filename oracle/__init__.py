"""TEST INFRASTRUCTURE ONLY: a CPU restatement of UMA-QMoE's MoE operator path.

This package is the checker. The product (``uma-qmoe_amd/``) never imports,
links or runs anything here; only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg may. Each function cites the reference file
and lines it restates (paths relative to the zihaomu/UMA-QMoE checkout).

Modules
-------
codec  ctypes wrapper over ``codec.c`` (Q4 / Q8 / BF16 codecs, plain C)
moe    torch-CPU restatement of the operator's correctness path, the
       Transformers router / shared-expert MLP / RMSNorm, and block composition

Pinning (what checks each function; see tests/test_oracle_*.py):
  codec       reference known-answer vectors (tests/unit/test_q4.py:19-67,
              tests/unit/test_bf16.py:44-63) + closed forms + brute force
  router      brute-force sort on tiny inputs, forced ties, Transformers'
              Qwen2MoeTopKRouter on tie-free inputs
  experts     Transformers' Qwen2MoeExperts / Qwen2MoeSparseMoeBlock run in fp32
              on the same dequantized weights, the reference's stacked-expert
              fixture (tests/unit/test_fixed_model_runners.py:185-204), and
              invariants (k=1 / zero weights / slot permutation / linearity)
  rmsnorm     Transformers' Qwen2MoeRMSNorm
"""
