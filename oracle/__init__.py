"""CPU oracle for the SCOPE attention hot path.

TEST INFRASTRUCTURE ONLY.  Nothing in ``scope_amd`` imports this package:
only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` use it, and there only to check results (or as the timed CPU
baseline), never as a fallback for the GPU path.

Modules:

* ``pointer``   – doc starts, reference-mode pointer mask, block-scoring mode,
                  sort/dedupe/pack, NB-wide export, q-list transpose (numpy).
* ``stats``     – forward and mask debug statistics (numpy).
* ``attention`` – dense-masked and block-sparse attention with the spectral
                  bias in token or block offsets, fp64/fp32 (torch on CPU).

Parity status of every function is listed in each module's header.
"""
