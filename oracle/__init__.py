"""CPU oracle for the decode hot path.

TEST INFRASTRUCTURE ONLY. This package restates, on the CPU, the arithmetic of
the reference's decode operators (the Metal kernels under
ios_kernels/kernels/*/kernels.metal and the step order of their Swift hosts),
and is the checker the GPU library is compared against. Only tests/,
__graft_entry__.smoke() and bench.py's cpu_baseline leg may import it, and only
as the checker or the timed CPU baseline; the product package never imports it.

Modules:
    hashrng  -- NumPy restatement of the synthetic-weight generator
    ops      -- NumPy restatement of each operator, fp64 inside an op
    model    -- the Gemma-2B-shaped decode step composed from ops (small configs)
    batch    -- one Llama-shaped int8 layer stepping a ragged batch
    native   -- ctypes binding of the C restatement (liboracle.so) for
                full-size decode runs and CPU timing

How each function is pinned (closed forms, library routines, brute force,
HF transformers' Gemma model and Llama decoder layer, the llama3 rope
initialiser) is in tests/test_oracle.py; every oracle function has at least
one such check.
"""
