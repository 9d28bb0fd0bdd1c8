"""Parity oracle and CPU baseline -- TEST INFRASTRUCTURE, not product code.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s
``cpu_baseline`` leg may import anything here.  See ``oracle/reference.py``
and ``oracle/quant_ref.py`` for what each function restates and how it is
pinned.
"""
