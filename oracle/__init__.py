"""CPU oracle for the GEMM and attention path -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import, call or link anything under oracle/, and only as the checker (or the
timed CPU baseline), never as the thing measured or shipped.  The product
path (frisk_amd) never falls back to it.

Contents
  gemm.py       fp64 textbook GEMM on decoded inputs, the reference's fp32
                sequential-k rank-1 GEMM, exact integer GEMM, OCP e4m3fn
                decoding.
  attention.py  fp64 stable-softmax attention (+ causal mask, LSE), the
                reference's strict/fp64 D64 tile oracle with its ordered FP32
                sum tree and f16 P boundary, its analytic fixtures, and the
                64x16 fixed-ABI attention oracle with its 15 input cases.
  oracle.c      the same fp64 GEMM / attention in C (OpenMP), built into
                oracle/liboracle.so by oracle/Makefile; bench.py times it as
                the CPU baseline.

Every function cites the reference file:line it restates.  How each one is
pinned (closed forms, library routines, brute force, the reference's own
known-answer tests) is in tests/test_oracle_*.py; no function here is left
"parity unpinned".
"""
