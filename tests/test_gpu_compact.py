"""Row compaction on the GPU is bit-exact against oracle.compact.

Covers zero-length segments, empty and full selections, single-token
segments, multi-chunk sizes (N > 4096, N not a multiple of the chunk), and
per-head lanes.  Calls go through the C ABI (logo_amd.ops.common).
"""

import numpy as np
import pytest
import torch

from logo_amd import _lib
from logo_amd.ops import build_selection, compute_q_start_blk, prepare_chunk_indices
from logo_amd.ops.common import compact_selection, dense_selection
from oracle import compact

pytestmark = pytest.mark.gpu

CASES = [
    ([0, 7], 0.5),
    ([0, 1, 1, 5, 5, 17], 0.5),
    ([0, 0, 50], 1.0),
    ([0, 50, 50], 0.0),
    ([0, 1], 1.0),
    ([0, 4096], 0.5),
    ([0, 3000, 3000, 9000, 9001, 12345], 0.3),
    ([0, 8192, 16384, 24576, 32768], 0.25),
    ([0, 70000], 0.5),
    ([0, 4096], 0.7),             # the largest one-lane input one workgroup compacts alone
    ([0, 100, 4097], 0.7),        # one token past it: the three-launch path
    ([0, 63, 64, 65, 130], 0.5),  # segment bounds inside and on 64-token groups
]


def _meta_lane(meta, nseq, lane):
    st = _lib.meta_stride(nseq)
    return meta[lane * st:(lane + 1) * st].cpu().numpy()


def _check_lane(dsel, lane, want, cu, n):
    m = _meta_lane(dsel.meta, dsel.nseq, lane)
    nseq = len(cu) - 1
    sq = want["Sq"]
    assert m[0] == sq
    assert m[3] == n and m[4] == nseq
    assert np.array_equal(m[8:8 + nseq + 1], want["cu_seqlens_q"])
    tq = compact.chunk_prefix(want["cu_seqlens_q"], _lib.BQ)
    tk = compact.chunk_prefix(cu, _lib.BKV)
    assert np.array_equal(m[8 + (nseq + 1):8 + 2 * (nseq + 1)], tq)
    assert np.array_equal(m[8 + 2 * (nseq + 1):8 + 3 * (nseq + 1)], tk)
    assert m[1] == tq[-1] and m[2] == tk[-1]
    if sq:
        assert np.array_equal(dsel.q_idx[lane, :sq].cpu().numpy(), want["q_idx"])
        assert np.array_equal(dsel.pos[lane, :sq].cpu().numpy(), want["pos_ids"])


@pytest.mark.parametrize("cu,ratio", CASES)
def test_compaction_bit_exact(gpu, cu, ratio):
    n = cu[-1]
    rng = np.random.default_rng(n)
    mask = rng.random(n) < ratio
    print(f"compaction cu={cu[:4]}.. n={n} ratio={ratio}", flush=True)
    dsel = compact_selection(torch.from_numpy(mask).to(gpu), torch.tensor(cu, dtype=torch.int32))
    (want,) = compact.build_selection(mask, cu)
    _check_lane(dsel, 0, want, cu, n)


@pytest.mark.parametrize("cu,ratio", [([0, 512], 0.5), ([0, 5000, 5000, 8192], 0.5),
                                      ([0, 30000, 65536], 0.3),   # per-head: one workgroup a lane
                                      ([0, 70000], 0.3)])         # past 65536: three launches
def test_per_head_lanes_bit_exact(gpu, cu, ratio):
    n, hq = cu[-1], 4
    rng = np.random.default_rng(7)
    mask = rng.random((n, hq)) < ratio
    dsel = compact_selection(torch.from_numpy(mask).to(gpu), torch.tensor(cu, dtype=torch.int32))
    for lane, want in enumerate(compact.build_selection(mask, cu)):
        _check_lane(dsel, lane, want, cu, n)


def test_build_selection_api(gpu):
    cu = torch.tensor([0, 100, 100, 300], dtype=torch.int64, device=gpu)
    rng = np.random.default_rng(1)
    mask = torch.from_numpy(rng.random(300) < 0.4)
    info = build_selection(mask.view(1, 300).to(gpu), 1, 300, cu)
    (want,) = compact.build_selection(mask.numpy(), cu.cpu().numpy())
    assert info.Sq == want["Sq"] and info.Nseq == 3 and info.T == 300
    assert info.q_idx.dtype == torch.int64 and info.pos_ids.dtype == torch.int32
    assert np.array_equal(info.q_idx.cpu().numpy(), want["q_idx"])
    assert np.array_equal(info.pos_ids.cpu().numpy(), want["pos_ids"])
    assert np.array_equal(info.cu_seqlens_q.cpu().numpy(), want["cu_seqlens_q"])
    assert info.cu_seqlens_k.dtype == torch.int32


@pytest.mark.parametrize("cu", [[0, 7], [0, 1, 1, 5, 5, 17], [0, 300, 301, 1000]])
@pytest.mark.parametrize("bt", [1, 16, 64, 128])
def test_chunk_indices_and_q_start(gpu, cu, bt):
    cut = torch.tensor(cu, dtype=torch.int32, device=gpu)
    got = prepare_chunk_indices(cut, bt).cpu().numpy()
    assert np.array_equal(got, compact.prepare_chunk_indices(cu, bt))
    rng = np.random.default_rng(bt)
    mask = rng.random(cu[-1]) < 0.3
    info = build_selection(torch.from_numpy(mask).view(1, -1).to(gpu), 1, cu[-1], cut)
    ck = prepare_chunk_indices(cut, bt)
    qs = compute_q_start_blk(info.pos_ids, info, ck, bt).cpu().numpy()
    (want,) = compact.build_selection(mask, cu)
    ref = compact.compute_q_start_blk(want["pos_ids"], want["cu_seqlens_q"], cu, bt, T=cu[-1])
    assert np.array_equal(qs, ref)


def test_dense_meta(gpu):
    cu = [0, 5, 5, 300]
    dsel = dense_selection(torch.tensor(cu, dtype=torch.int32), 300, gpu)
    m = _meta_lane(dsel.meta, 3, 0)
    assert m[0] == 300
    assert np.array_equal(m[8:12], cu)
    assert np.array_equal(m[12:16], compact.chunk_prefix(cu, _lib.BQ))


def test_compaction_is_deterministic(gpu):
    rng = np.random.default_rng(11)
    mask = torch.from_numpy(rng.random(50000) < 0.5).to(gpu)
    cu = torch.tensor([0, 20000, 50000], dtype=torch.int32)
    a = compact_selection(mask, cu)
    b = compact_selection(mask, cu)
    sq = a.sq()
    assert sq == int(mask.sum().item())
    assert torch.equal(a.meta, b.meta)
    assert torch.equal(a.q_idx[:, :sq], b.q_idx[:, :sq]) and torch.equal(a.pos[:, :sq], b.pos[:, :sq])
