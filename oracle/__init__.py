"""Test infrastructure: CPU restatements of the reference's EWS algorithm, used only as the checker by
``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline leg. The product never imports it."""
