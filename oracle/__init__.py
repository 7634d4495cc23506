"""CPU oracle of the ThetaScan scan hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU (torch float64/float32), the reference
algorithms the MI355X kernels must reproduce.  It is the checker: only the
test-suite, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import it.  The product package ``thetascan_amd`` never
imports anything from here and has no CPU path of its own.

Every function cites the reference file:line it follows.  How each one is
pinned (golden vectors written from the reference, closed forms, brute force)
is listed in each module header; a function with no such check says
"parity unpinned".
"""
