"""CPU oracle and CPU baseline of the KV-cache data path -- TEST INFRASTRUCTURE ONLY.

Importable by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
CPU-baseline leg, as the checker; never by the ``hexgen2_amd`` product path.
"""
