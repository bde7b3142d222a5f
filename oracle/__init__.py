"""CPU oracle for the attention-relation KL path.

Test infrastructure only: imported by ``tests/``, ``__graft_entry__.smoke()``
and ``bench.py``'s ``cpu_baseline`` leg, never by the ``linearard_amd``
package.
"""
