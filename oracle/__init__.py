"""CPU oracle for the Gated DeltaNet hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in the product package imports this
directory; only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` use it, and only as the checker (or as
the timed CPU baseline), never as a compute path of the library.

``oracle.gdn`` restates the floating-point math of the reference's torch /
Triton operators in plain torch on the CPU; ``oracle.metadata`` restates the
integer host logic (packed indices, checkpoint placement, verify groups,
Marconi block mapping, speculative commit) bit-exactly.  Every function cites
the reference file:line it follows.  How each function is pinned (closed
forms, invariants, known answers from the reference's own tests) is recorded
in the module headers.
"""
