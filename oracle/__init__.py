"""CPU oracle for torchpp's transformer-inference kernel set.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py may import this package, and only as the checker
(or the timed CPU baseline). The product package `torchplusplus_amd` never
imports it and has no CPU fallback.

Each function restates the reference's algorithm in PyTorch-CPU / numpy
(fp32 where the reference computes in fp32, fp64 for the closed forms that
pin the restatements) and cites the reference file:line it follows. How each
one is pinned (library routine, closed form, invariant, brute force) is
tested in tests/test_oracle.py.

The reference's native code is CUDA/CUTLASS-only (inline PTX, __shfl_*_sync
with 32-lane masks, CUTLASS/CuTe headers that are absent here), so there is
no buildable `oracle/_ref`.
"""
from .ops import *  # noqa: F401,F403
