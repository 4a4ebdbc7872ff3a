"""Pin the integer oracle (oracle.compact) by brute force and invariants.

The reference ships no golden vectors for this path (its only test,
tests/test_model.py, has no assertions), so the compaction semantics of
logo/ops/common.py:71-124 and logo/ops/selected_full_attn.py:374-402 are
pinned here against pure-Python loops written from the definitions.
"""

import numpy as np
import pytest

from oracle import compact


def brute_selection(mask, cu):
    q_idx, pos, counts = [], [], [0] * (len(cu) - 1)
    for t, on in enumerate(mask):
        if not on:
            continue
        s = max(i for i in range(len(cu) - 1) if cu[i] <= t)
        q_idx.append(t)
        pos.append(t - cu[s])
        counts[s] += 1
    cu_q = [0]
    for c in counts:
        cu_q.append(cu_q[-1] + c)
    return q_idx, pos, cu_q


def brute_chunks(cu, bt):
    rows = []
    for s in range(len(cu) - 1):
        n = cu[s + 1] - cu[s]
        for b in range(-(-n // bt)):
            rows.append((s, b))
    return rows


def brute_q_start(pos, cu_q, cu_k, bt):
    out = []
    for s, j in brute_chunks(cu_k, bt):
        first = next((r for r in range(cu_q[s], cu_q[s + 1]) if pos[r] >= j * bt), cu_q[s + 1])
        out.append((first - cu_q[s]) // bt)
    return out


CASES = [
    ([0, 7], 0.5),
    ([0, 1, 1, 5, 5, 17], 0.5),      # zero-length segments
    ([0, 64, 130, 300], 0.25),
    ([0, 0, 50], 1.0),
    ([0, 50, 50], 0.0),
    ([0, 1], 1.0),                     # single token
]


@pytest.mark.parametrize("cu,ratio", CASES)
@pytest.mark.parametrize("seed", [0, 1])
def test_build_selection_matches_brute_force(cu, ratio, seed):
    rng = np.random.default_rng(seed)
    n = cu[-1]
    mask = rng.random(n) < ratio
    (res,) = compact.build_selection(mask, cu)
    q_idx, pos, cu_q = brute_selection(mask.tolist(), cu)
    assert res["q_idx"].tolist() == q_idx
    assert res["pos_ids"].tolist() == pos
    assert res["cu_seqlens_q"].tolist() == cu_q
    assert res["Sq"] == int(mask.sum()) == cu_q[-1]
    assert res["q_idx"].dtype == np.int64 and res["pos_ids"].dtype == np.int32
    assert res["cu_seqlens_q"].dtype == np.int32


def test_per_head_lanes_are_independent_columns():
    rng = np.random.default_rng(3)
    cu = [0, 40, 41, 100]
    mask = rng.random((100, 4)) < 0.4
    lanes = compact.build_selection(mask, cu)
    assert len(lanes) == 4
    for h in range(4):
        (single,) = compact.build_selection(mask[:, h], cu)
        for key in ("q_idx", "pos_ids", "cu_seqlens_q"):
            assert np.array_equal(lanes[h][key], single[key])


@pytest.mark.parametrize("cu,ratio", CASES)
@pytest.mark.parametrize("bt", [1, 3, 64, 128])
def test_chunk_indices_and_prefix(cu, ratio, bt):
    got = compact.prepare_chunk_indices(cu, bt)
    want = brute_chunks(cu, bt)
    assert [tuple(r) for r in got.tolist()] == want
    assert got.dtype == np.int32
    pre = compact.chunk_prefix(cu, bt)
    enum = []
    for t in range(int(pre[-1])):
        s = max(i for i in range(len(cu) - 1) if pre[i] <= t)
        enum.append((s, t - int(pre[s])))
    assert enum == want


@pytest.mark.parametrize("cu,ratio", CASES)
@pytest.mark.parametrize("bt", [2, 16, 64])
@pytest.mark.parametrize("seed", [0, 5])
def test_q_start_blk_matches_brute_force(cu, ratio, bt, seed):
    rng = np.random.default_rng(seed)
    mask = rng.random(cu[-1]) < ratio
    (res,) = compact.build_selection(mask, cu)
    got = compact.compute_q_start_blk(res["pos_ids"], res["cu_seqlens_q"], cu, bt, T=cu[-1])
    want = brute_q_start(res["pos_ids"].tolist(), res["cu_seqlens_q"].tolist(), cu, bt)
    assert got.tolist() == want


def test_brute_force_catches_planted_mistake():
    """A searchsorted with side='left' (a plausible slip) must be caught."""
    cu = [0, 5, 5, 12]
    mask = np.ones(12, dtype=bool)
    q_idx = np.flatnonzero(mask)
    wrong_seg = np.searchsorted(np.asarray(cu), q_idx, side="left") - 1
    wrong_pos = (q_idx - np.asarray(cu)[np.maximum(wrong_seg, 0)]).tolist()
    _, pos, _ = brute_selection(mask.tolist(), cu)
    assert wrong_pos != pos
