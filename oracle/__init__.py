"""CPU oracle for the attention hot path (test infrastructure only).

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import this package; the shipped ``nitrix_amd``
package never does.
"""
