"""CPU oracle for the fused SDPA forward -- TEST INFRASTRUCTURE ONLY.

Importable by ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg, as the
checker. Nothing in the product package (``fused_attn``) imports it.
"""
