"""CPU oracle for the attention hot path -- TEST INFRASTRUCTURE ONLY.

Imported only by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg, as the checker.  The product package
(``flash_attn_v100_amd`` / ``flash_attn_v100``) never imports it.
"""
