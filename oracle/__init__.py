"""CPU oracle for the ragged paged-attention path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or, for the
baseline, as the thing timed on the host); the product package
``slipstream_amd`` never imports it and has no CPU path.

Modules:
  paged_attention  numpy restatement (float64) of the scatter, the gather and
                   paged attention (slipstream/kernels/attention_ref.py,
                   slipstream/models/layers/attention.py:20-88,
                   slipstream/kernels/triton_paged.py:65-95,133-206)
  quant            numpy restatement of the W4A16 format and GEMM
                   (slipstream/kernels/quant_ref.py:38-133)
  reference_path   torch-CPU restatement of the reference's own dtype sequence
                   (bf16 GEMMs, fp32 softmax), timed as the CPU baseline

How each function is pinned (golden fixtures, known answers, library routines,
invariants) is listed in tests/test_oracle_*.py; every oracle function has at
least one check that does not re-evaluate its own formula.
"""
