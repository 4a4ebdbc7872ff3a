"""Query-sparse causal attention and sliding-window attention on the CPU.

Test infrastructure only: see the package docstring.

Restates
--------
* forward  -- logo/ops/selected_full_attn.py:33-121 (``sq_full_attn_fwd_kernel``)
  and :449-471 (zero rows for unselected tokens): for a selected row at
  position ``p`` of its segment, ``o = softmax(scale * q K[seg, 0..p]^T) V``;
  ``lse`` is stored in the log2 domain, ``lse = log2(sum_j exp(scale * s_j))``
  (:93-99, :118-119).
* backward -- :124-138 (``delta = rowsum(o * dO)``), :141-228 (dq), :231-337
  (dk, dv) and :444-445 (GQA sum of dk/dv over the query heads of a group):
  ``P = softmax``, ``dP = dO V^T``, ``dS = P * (dP - delta)``,
  ``dq = scale dS K``, ``dk = scale dS^T Q``, ``dv = P^T dO``.
* sliding window -- logo/layers/utils.py:144-147 with flash-attn's
  ``window_size=(w, w)`` + ``causal=True``: keys ``j`` with
  ``p - w <= j <= p`` inside the segment (129 keys for w = 128).
* dense causal reference -- logo/ops/dense_full_attn.py:30-69
  (per-segment causal SDPA with GQA ``repeat_kv``).

Arrays are ``q [N, HQ, D]``, ``k/v [N, H, D]`` (the reference's ``B = 1``
packed layout with the batch axis dropped).  ``selection`` is ``[N]`` (shared
by all heads, the reference API) or ``[N, HQ]`` (per-head extension).

Pinning (tests/test_oracle_attn.py): all-ones selection equals torch's own
``scaled_dot_product_attention`` per segment; row 0 of a segment returns
``v_0``; unselected rows are zero; GQA equals ``repeat_kv``; ``lse`` equals
``logsumexp / ln 2``; the backward equals torch autograd (float64) of an
independently written masked-softmax formulation; windowed attention with
``T <= w + 1`` equals full causal attention and matches a brute-force loop.
"""

import math

import numpy as np

from .compact import _lanes


def _visible(pos, keys, window):
    m = keys[None, :] <= pos[:, None]
    if window is not None and window >= 0:
        m &= keys[None, :] >= (pos[:, None] - window)
    return m


def _rows_by_lane(selection, n_tokens, hq_count):
    """Per query head: bool row mask [N]."""
    if selection is None:
        lanes = np.ones((1, n_tokens), dtype=bool)
    else:
        lanes = _lanes(selection)
    if lanes.shape[0] == 1:
        return [lanes[0]] * hq_count
    assert lanes.shape[0] == hq_count
    return list(lanes)


def sq_attn_fwd(q, k, v, selection, cu_seqlens, scale=None, window=None,
                dtype=np.float64, row_chunk=1024):
    """Forward.  Returns ``o [N, HQ, D]`` and ``lse [N, HQ]`` (log2 domain).

    Unselected rows: ``o = 0`` (logo/ops/selected_full_attn.py:469-471) and
    ``lse = nan`` (the reference never stores them).
    """
    N, HQ, D = q.shape
    H = k.shape[1]
    G = HQ // H
    if scale is None:
        scale = D ** -0.5
    cu = np.asarray(cu_seqlens).astype(np.int64)
    rows_mask = _rows_by_lane(selection, N, HQ)
    o = np.zeros((N, HQ, v.shape[2]), dtype=dtype)
    lse = np.full((N, HQ), np.nan, dtype=dtype)
    for s in range(cu.size - 1):
        bos, eos = int(cu[s]), int(cu[s + 1])
        if eos <= bos:
            continue
        keys = np.arange(eos - bos)
        for hq in range(HQ):
            h = hq // G
            rows = np.flatnonzero(rows_mask[hq][bos:eos]) + bos
            if rows.size == 0:
                continue
            K = k[bos:eos, h].astype(dtype)
            V = v[bos:eos, h].astype(dtype)
            for c0 in range(0, rows.size, row_chunk):
                r = rows[c0:c0 + row_chunk]
                pos = r - bos
                S = (q[r, hq].astype(dtype) @ K.T) * dtype(scale)
                vis = _visible(pos, keys, window)
                S = np.where(vis, S, -np.inf)
                m = S.max(axis=1, keepdims=True)
                P = np.exp(S - m)
                l = P.sum(axis=1, keepdims=True)
                o[r, hq] = (P @ V) / l
                lse[r, hq] = ((m + np.log(l)) / math.log(2.0))[:, 0]
    return o, lse


def sq_attn_bwd(q, k, v, o, do, selection, cu_seqlens, scale=None, window=None,
                dtype=np.float64, row_chunk=1024):
    """Backward.  Returns ``dq [N, HQ, D]``, ``dk [N, H, D]``, ``dv [N, H, D]``.

    ``o`` is the forward output used for ``delta`` (the reference uses the
    stored, rounded output: logo/ops/selected_full_attn.py:135-137).
    Unselected rows get ``dq = 0``; keys seen by no selected row get
    ``dk = dv = 0``; dk/dv of a GQA group are summed over its query heads
    (:444-445).
    """
    N, HQ, D = q.shape
    H = k.shape[1]
    G = HQ // H
    if scale is None:
        scale = D ** -0.5
    cu = np.asarray(cu_seqlens).astype(np.int64)
    rows_mask = _rows_by_lane(selection, N, HQ)
    dq = np.zeros((N, HQ, D), dtype=dtype)
    dk = np.zeros((N, H, D), dtype=dtype)
    dv = np.zeros((N, H, v.shape[2]), dtype=dtype)
    for s in range(cu.size - 1):
        bos, eos = int(cu[s]), int(cu[s + 1])
        if eos <= bos:
            continue
        keys = np.arange(eos - bos)
        for hq in range(HQ):
            h = hq // G
            rows = np.flatnonzero(rows_mask[hq][bos:eos]) + bos
            if rows.size == 0:
                continue
            K = k[bos:eos, h].astype(dtype)
            V = v[bos:eos, h].astype(dtype)
            for c0 in range(0, rows.size, row_chunk):
                r = rows[c0:c0 + row_chunk]
                pos = r - bos
                Q = q[r, hq].astype(dtype)
                dO = do[r, hq].astype(dtype)
                S = (Q @ K.T) * dtype(scale)
                vis = _visible(pos, keys, window)
                S = np.where(vis, S, -np.inf)
                P = np.exp(S - S.max(axis=1, keepdims=True))
                P /= P.sum(axis=1, keepdims=True)
                delta = (o[r, hq].astype(dtype) * dO).sum(axis=1, keepdims=True)
                dP = dO @ V.T
                dS = P * (dP - delta)
                dq[r, hq] = dtype(scale) * (dS @ K)
                dk[bos:eos, h] += dtype(scale) * (dS.T @ Q)
                dv[bos:eos, h] += P.T @ dO
    return dq, dk, dv


def swa_fwd(q, k, v, cu_seqlens, window=128, scale=None, dtype=np.float64):
    """Sliding-window causal attention on every row (logo/layers/utils.py:144-147)."""
    return sq_attn_fwd(q, k, v, None, cu_seqlens, scale=scale, window=window, dtype=dtype)


def sq_flops_fwd(selection, cu_seqlens, n_heads, head_dim):
    """Algorithmic forward FLOPs counted on selected rows only.

    ``F_fwd = 4 * D * sum over heads and selected rows of (p + 1)`` (QK^T plus
    PV over the p + 1 visible keys).  Backward is ``2.5 * F_fwd``.
    """
    cu = np.asarray(cu_seqlens).astype(np.int64)
    lanes = _lanes(selection)
    total = 0
    for lane in lanes:
        for s in range(cu.size - 1):
            bos, eos = int(cu[s]), int(cu[s + 1])
            pos = np.flatnonzero(lane[bos:eos])
            total += int((pos + 1).sum())
    if lanes.shape[0] == 1:
        total *= n_heads
    return 4.0 * head_dim * total
