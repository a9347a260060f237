"""CPU oracle for the xvllm decode hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in numpy (float64 where the reference computes in
fp32), in multi-threaded torch (the decode attention, for the CPU baseline)
and in plain C (the sampler, whose integer fixed-point arithmetic must
match bit for bit), what xixi-vllm's hot-path ops compute.  Each function
cites the reference file:line it follows.  Only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` leg may
import it, and only as the checker or as the timed CPU baseline; the product
path (``xvllm``) never calls into it.

Pinning (how each function is checked against something other than itself)
is listed in tests/test_oracle.py; nothing here is "parity unpinned" except
what that file's header names.
"""
