"""CPU oracle for the column sequence mixers: TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU and in plain PyTorch (float64 unless a caller asks otherwise),
the algorithms the HIP kernels of ``vesper`` must reproduce:

- ``oracle.delta``: the delta-rule fast-weight scan (reference ``vesper/recurrence.py``);
- ``oracle.attention``: sliding-window causal attention, the chronological cache and the decode
  ring (reference ``vesper/attention.py``, ``vesper/kernels/window_attn.py``);
- ``oracle.loop``: the looped column with per-token halting and copy-forward (reference
  ``vesper/loop.py``, ``vesper/column.py``);
- ``oracle.keys``: the causal key filter and key normalization before the scan (reference
  ``vesper/column.py``, ``vesper/kernels/keys.py``).

Only ``tests/``, ``__graft_entry__.smoke()`` and the CPU-baseline leg of ``bench.py`` may import
this package, and only as the checker (or as the timed CPU baseline); the product path never
routes through it, and it never runs on a GPU. Every function cites the reference file:line it
follows. Each function is pinned by closed forms, invariants or brute force in
``tests/test_oracle_*.py``; none is "parity unpinned".
"""
