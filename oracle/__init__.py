"""CPU oracle for the packed-KV decode hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in this package is part of the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may import it, and only as
the checker (or, in the bench, as the timed CPU baseline), never as the thing measured or
shipped.  The product path (``kv-project_amd/kvq``) never imports it and fails loudly when the
HIP library is missing.

Each function restates, in numpy, the reference algorithm it names (``FILE:LINE`` into
TahirSher/KV-Project).  The restatements follow the reference's operation order wherever the
result is bit-exact (quantisation codes, fp16 metadata, packed bytes, retained indices) and use
float64 for attention outputs, which the reference only defines to float32 rounding.

Pinning (what fixes each function independently of this restatement) is listed per module
header and in the tests under ``tests/test_oracle_*.py``.
"""
