"""CPU oracle for the EXL3 trellis hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the shipped library imports, links or
executes this package.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may use it, and only as the checker (or the
timed CPU baseline), never as a path that produces library results.

Contents
--------
``codec``   ring-window extraction, the three procedural codebooks and the
            16x16 tile permutation (restates python/strix_trellis/codec.py and
            docs/FORMAT.md:42-101 of the reference).
``linear``  the FP64 algebraic layer and the staged FP32/RN16 production
            contract (restates python/strix_trellis/linear.py and
            docs/NUMERICS.md:30-126).
``moe``     the routed-expert (SwiGLU + ordered weighted top-k) block on top of
            ``linear`` (restates docs/TP_RANK.md:64-76 and
            include/strix_trellis.h:197-233).
``native``  ctypes loader for the C restatement in ``oracle/c`` (a faster
            decode and a scalar FP32 core of the same contract), used where
            the NumPy forms would be too slow for a test.
"""
