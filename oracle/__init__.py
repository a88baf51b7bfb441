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
``_ref``    (built, not committed) ``libstrix_ref.so``: the reference's own
            scalar host oracle (src/host_reference.hpp) compiled from the
            reference tree by ``make -C oracle ref``; tests use it to pin
            ``codec`` state by state.
"""
