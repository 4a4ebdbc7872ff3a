"""One decode step of LoGo's attention branches on the CPU.

Test infrastructure only: see the package docstring.

Restates logo/layers/logo.py:228-249 (decode branch) with the cache of
logo/cache.py:46-124: the global branch attends over every cached key of its
row when the row's gate passes (``gate >= thres``) and is zero otherwise; the
local branch attends over the last ``window + 1`` keys (128 cached plus the new
one, flash-attn window (128, 128) with a 129-key cache, logo/layers/utils.py:
144-147).

Pinning (tests/test_oracle_decode.py): the decode output equals the last row
of the prefill oracle (oracle.attn.sq_attn_fwd) over the same keys, for the
global branch (full causal) and the local branch (window 128).
"""

import numpy as np


def decode_attn(q, k, v, lens, active=None, scale=None, dtype=np.float64):
    """``q [B, HQ, D]``, ``k/v [B, H, T, D]`` (row b valid on ``[0, lens[b])``).

    Returns ``[B, HQ, D]``; inactive rows are zero.
    """
    B, HQ, D = q.shape
    H = k.shape[1]
    G = HQ // H
    if scale is None:
        scale = D ** -0.5
    out = np.zeros((B, HQ, v.shape[3]), dtype=dtype)
    for b in range(B):
        if active is not None and not active[b]:
            continue
        n = int(lens[b])
        for hq in range(HQ):
            K = k[b, hq // G, :n].astype(dtype)
            V = v[b, hq // G, :n].astype(dtype)
            s = (K @ q[b, hq].astype(dtype)) * dtype(scale)
            p = np.exp(s - s.max())
            out[b, hq] = (p @ V) / p.sum()
    return out
