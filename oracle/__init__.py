"""CPU oracle for the weight-streaming data path — TEST INFRASTRUCTURE ONLY.

This package restates, in numpy and plain Python, what the reference computes
on the host for the path the native library replaces:

* ``oracle.squareq`` — bf16 round-to-nearest-even, the SquareQ INT8 row-scale
  dequant, fp32→bf16 packing, the parameter layout and the block staging
  helpers (src/stagehand/scheduler.py:148-346), each function citing the
  reference lines it follows;
* ``oracle.torch_ref`` — the reference's exact torch CPU op sequence for the
  dequant and cast, used as the timed CPU baseline.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker or the reported
baseline — never as the thing measured or shipped. Nothing in
``stagehand_amd`` imports it.

Pinning (what makes this oracle trustworthy; the tests are in
tests/test_oracle.py):

* ``bf16_rne_bits`` — compared with torch's CPU float→bfloat16 conversion (the
  library the reference calls at scheduler.py:181/300/1071) on every one of the
  2^32 fp32 bit patterns, and with an independent exact-rational rounding on
  edge values;
* ``dequant_rows`` — the reference's known-answer test
  (tests/test_scheduler.py:294-375: q = arange(64)-32, scale 1, zp 0), the
  identical torch CPU expression on seeded inputs, and brute force over all
  255 int8 values × a scale sweep against exact rational arithmetic;
* ``build_param_layout`` / ``stage_*`` — prefix-sum and round-trip invariants,
  plus the fallback branches (zero fill, evicted params, padded_in slicing)
  checked against closed forms.
"""
