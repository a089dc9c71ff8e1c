"""CPU oracle for the ASRN layer hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, what the reference (KIROKOWA/ASRN) computes on the path the HIP library
replaces: sign-hash bucketing and the stable bucket sort, the recent-mates candidate attention forward (its
backward comes from torch autograd over the restatement), the n-gram keys and their stable sort, the Hawkes, streak
and clock scans, and the O(1) generation state (per-bucket rings and per-key Hawkes memory). Every function cites
the reference file:line it follows.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only as the checker or the
timed CPU baseline. The product path (asrn_amd) never imports it and has no CPU fallback.

Pinning (what keeps this restatement honest) lives in tests/test_oracle_golden.py, tests/test_oracle_defs.py and
tests/test_oracle_generation.py:
  - golden fixtures written from the reference itself (tests/golden/make_golden.py) for the whole layer, its
    candidate stage and its repetition stage, forward and gradients;
  - definitions: brute-force candidate sets, the O(N^2) Hawkes sum, the sequential scan, the cumprod suffix
    length, numpy's stable argsort, n-gram keys against a Python-float loop (one rounding per operation), the
    per-query candidate restatement against the sorted-window one.
"""
