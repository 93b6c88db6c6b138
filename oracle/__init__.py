"""CPU oracle for PURIN's Chambolle--Pock projection path.

TEST INFRASTRUCTURE ONLY.  This package is a NumPy (and plain C) restatement of
the reference algorithm, used as the checker for the HIP implementation in
``purin_amd``.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product package never
does, and has no CPU fallback that routes here.

Parity status per function (what pins it) is stated in each module header.
"""
