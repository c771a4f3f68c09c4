"""CPU oracle of the fused PLE path -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, always as the checker or the timed CPU
baseline, never as part of the product path.
"""
