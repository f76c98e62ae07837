"""The oracle: a CPU restatement of FuryKernel's arithmetic, reductions,
planned kernels and f64 program evaluator.

TEST INFRASTRUCTURE.  Only ``tests/``, ``__graft_entry__.smoke()`` and
``bench.py``'s ``cpu_baseline`` leg import this package, as the checker of the
HIP path and as the CPU baseline; the product never does.
"""
