"""CPU oracle of the paged-attention hot path — test infrastructure only.

Imported by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU
baseline as the checker; never by the ``infrared_amd`` product package.
"""
