"""CPU oracle for the int8 MoE layer — TEST INFRASTRUCTURE ONLY.

Only tests/, ``__graft_entry__.smoke()`` and bench.py's ``cpu_baseline`` leg
may import this package, and only as the checker. The product path
(``runntime_amd``) never imports it.
"""
