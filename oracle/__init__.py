"""TEST INFRASTRUCTURE -- the CPU oracle of the Block AttnRes operator.

Nothing in the product (``blackwell-switchyard_amd/switchyard``) imports this
package. Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg use it, and only as the checker or the timed CPU
baseline -- never as the code path being measured or shipped.

Contents
--------
``reference``
    A float64 torch restatement of the reference's oracle module
    (``src/switchyard/reference.py``) and eager formulations
    (``src/switchyard/baselines.py``), with the parity metric of
    ``bench/harness.py:295-358``.
``c_oracle``
    ctypes binding of ``attnres_oracle.c``: an independent double-precision
    C restatement (forward, closed-form backward, stats, merge, batched).

Pinning. The reference ships no golden vectors (its tests draw seeded random
inputs and compare against an on-the-fly float64 oracle). The two
restatements here are pinned against each other, against every semantic
property ``tests/test_reference.py`` asserts, against hand-derived closed
forms, against ``torch.autograd`` and central differences for the backward,
and against committed fixtures (``tests/golden``) -- see
``tests/test_oracle.py``, which also plants mistakes in the oracle to show
that those checks catch them.
"""
