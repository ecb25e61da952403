"""CPU oracle of the compressed-KV attention path.

TEST INFRASTRUCTURE ONLY.  Nothing here is part of the product: only the
tests, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` import it, and only as the reference results a test compares
against or as the CPU baseline.

``hc_oracle.py`` is a numpy restatement of the reference's algorithm (each
function cites the reference file:line it follows); ``hc_oracle.c`` restates
the two loops that dominate CPU time (decode attention, top-k selection) in
plain C for the CPU baseline and as a second, independent implementation.

Parity pinning (what fixes each function beyond its own formula) is listed
in the header of hc_oracle.py.
"""
