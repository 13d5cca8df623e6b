"""CPU oracle of the O(2) tensor-product hot path.

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and
the ``cpu_baseline`` leg of bench.py as the checker / timed CPU baseline.
The product (ictc-o2-hp_amd/) never imports it.
"""
