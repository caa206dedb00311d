"""CPU oracle of the FlashMap drafter-attention path.

TEST INFRASTRUCTURE ONLY: imported by ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py``, always as the computation the tests compare
against or the reported CPU baseline, never as a code path of the product
(``flashmap_amd``), which has no CPU fallback.
"""
