"""CPU restatement of LoGo's attention hot path -- TEST INFRASTRUCTURE ONLY.

This package is the parity checker for the HIP kernels in ``logo_amd``.  It is
imported only by ``tests/``, by ``__graft_entry__.smoke()`` and by the
``cpu_baseline`` leg of ``bench.py``; the product path (``logo_amd``) never
imports, links or runs anything here.

Modules
-------
``compact``   integer row compaction, tile schedule and dK/dV start blocks
              (numpy, bit-exact semantics of the reference selection helpers).
``attn``      query-sparse causal attention forward/backward, sliding-window
              attention, dense causal reference (numpy, float64 or float32).
``epilogue``  gate threshold, branch RMSNorm and gated fusion, forward and
              backward (numpy, with the reference's bf16 rounding points).
``decode``    one decode step of the LoGo attention branches over a KV cache.
``cpu_path``  the reference's own CPU-capable formulation (dense causal
              attention per packed segment, then row masking) in torch fp32,
              used as the timed CPU baseline.

Every function cites the reference file:line whose behaviour it restates.
How each function is pinned (golden vectors, closed forms, brute force) is
listed in the module docstrings and exercised by ``tests/test_oracle_*.py``.
"""
