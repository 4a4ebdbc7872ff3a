"""Row compaction, tile schedule and dK/dV start blocks (integer, bit-exact).

Test infrastructure only: see the package docstring.

Restates
--------
* ``build_selection``        -- logo/ops/common.py:71-107
* ``prepare_chunk_indices``  -- logo/ops/common.py:110-124
* ``compute_q_start_blk``    -- logo/ops/selected_full_attn.py:374-402

Selection "lanes": the reference takes a per-token mask ``[1, N]`` that every
query head shares (logo/ops/selected_full_attn.py:520).  The per-(head, token)
mask ``[1, N, HQ]`` is this build's extension; it is compacted independently
per head, i.e. lane ``h`` is the reference's per-token semantics applied to the
column ``mask[:, h]``.

Pinning: brute-force pure-Python loops on small inputs and the invariants
``cu_q[-1] == Sq == mask.sum()``, ascending ``q_idx``, ``pos`` strictly
increasing inside a segment, zero-length segments allowed
(tests/test_oracle_compact.py).
"""

import numpy as np


def _lanes(selection: np.ndarray) -> np.ndarray:
    """Return the mask as ``[lanes, N]`` bool (lanes = 1 or HQ)."""
    sel = np.asarray(selection).astype(bool)
    if sel.ndim == 1:
        return sel[None, :]
    if sel.ndim == 2:  # [N, HQ] per-head extension
        return np.ascontiguousarray(sel.T)
    raise ValueError("selection must be [N] or [N, HQ]")


def build_selection(selection, cu_seqlens):
    """Compaction metadata per lane.

    Follows logo/ops/common.py:84-96: ``q_idx = nonzero(flat)`` (ascending,
    int64, :90); ``seg = searchsorted(cu, q_idx, right=True) - 1`` (:92);
    ``pos = q_idx - cu[seg]`` (int32, :93); ``cu_q = [0, cumsum(bincount(seg,
    minlength=Nseq))]`` (int32, :94-96).

    Returns a list (one entry per lane) of dicts with ``q_idx`` (int64),
    ``pos_ids`` (int32), ``cu_seqlens_q`` (int32), ``Sq``.
    """
    cu = np.asarray(cu_seqlens).astype(np.int64)
    nseq = cu.size - 1
    out = []
    for lane in _lanes(selection):
        q_idx = np.flatnonzero(lane).astype(np.int64)
        seg = np.searchsorted(cu, q_idx, side="right") - 1
        pos = (q_idx - cu[seg]).astype(np.int32)
        counts = np.bincount(seg, minlength=nseq) if q_idx.size else np.zeros(nseq, np.int64)
        cu_q = np.zeros(nseq + 1, dtype=np.int32)
        cu_q[1:] = np.cumsum(counts[:nseq]).astype(np.int32)
        out.append(dict(q_idx=q_idx, pos_ids=pos, cu_seqlens_q=cu_q, Sq=int(q_idx.size)))
    return out


def prepare_chunk_indices(cu_seqlens, chunk_size: int) -> np.ndarray:
    """``[NT, 2]`` int32 list of (sequence id, local block id).

    Follows logo/ops/common.py:116-124: NT = sum over sequences of
    ceil(len / chunk_size), sequences in order, blocks in order, zero-length
    sequences contribute nothing.
    """
    cu = np.asarray(cu_seqlens).astype(np.int64)
    lens = cu[1:] - cu[:-1]
    nblk = (lens + chunk_size - 1) // chunk_size
    seq = np.repeat(np.arange(lens.size, dtype=np.int32), nblk)
    if seq.size == 0:
        return np.zeros((0, 2), dtype=np.int32)
    starts = np.concatenate([[0], np.cumsum(nblk)[:-1]])
    blk = np.arange(seq.size, dtype=np.int64) - np.repeat(starts, nblk)
    return np.stack([seq, blk.astype(np.int32)], axis=1).astype(np.int32)


def chunk_prefix(cu_seqlens, chunk_size: int) -> np.ndarray:
    """Exclusive prefix of per-sequence block counts, ``[Nseq+1]`` int32.

    The device kernels locate tile ``t`` in sequence ``s`` with
    ``prefix[s] <= t < prefix[s+1]``; enumerating that relation gives exactly
    ``prepare_chunk_indices`` (logo/ops/common.py:110-124).
    """
    cu = np.asarray(cu_seqlens).astype(np.int64)
    lens = cu[1:] - cu[:-1]
    nblk = (lens + chunk_size - 1) // chunk_size
    out = np.zeros(lens.size + 1, dtype=np.int32)
    out[1:] = np.cumsum(nblk).astype(np.int32)
    return out


def compute_q_start_blk(pos_ids, cu_seqlens_q, cu_seqlens_k, block: int, T: int) -> np.ndarray:
    """First compacted-query block each KV block can see.

    Follows logo/ops/selected_full_attn.py:380-402: for KV block ``(n, j)``
    (from ``prepare_chunk_indices(cu_k, block)``) find the first compacted
    query of sequence ``n`` whose position is ``>= j * block`` via a
    searchsorted over ``seg * (T + 1) + pos``, subtract the segment start,
    clamp at 0 and divide by ``block``.
    """
    cu_q = np.asarray(cu_seqlens_q).astype(np.int64)
    chunks = prepare_chunk_indices(cu_seqlens_k, block)
    if chunks.shape[0] == 0:
        return np.zeros(0, dtype=np.int32)
    i_n = chunks[:, 0].astype(np.int64)
    kv0 = chunks[:, 1].astype(np.int64) * block
    big = int(T) + 1
    counts = cu_q[1:] - cu_q[:-1]
    seg = np.repeat(np.arange(counts.size, dtype=np.int64), counts)
    keys = seg * big + np.asarray(pos_ids).astype(np.int64)
    first = np.searchsorted(keys, i_n * big + kv0, side="left")
    local = np.maximum(first - cu_q[i_n], 0)
    return (local // block).astype(np.int32)

