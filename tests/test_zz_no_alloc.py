"""``logo_compact_noalloc`` (no workspace argument, fixed device scratch) against
``logo_compact`` through the C ABI: bit-identical q_idx, pos and meta, and
equal to the oracle's build_selection, on two calls in a row with the second
smaller than the first (the scratch keeps the first call's counts, which the
second must not see).  Also: a size above the fixed scratch is refused with
LOGO_EINVAL before any launch.
"""

import numpy as np
import pytest
import torch

from logo_amd import _lib
from oracle import compact as oc

pytestmark = pytest.mark.gpu

SENTINEL = -7
LOGO_COMPACT_SCRATCH_INTS = 65536  # include/logo_hip.h


def _outputs(n, lanes, nseq, dev):
    q_idx = torch.full((lanes, max(n, 1)), SENTINEL, dtype=torch.int64, device=dev)
    pos = torch.full((lanes, max(n, 1)), SENTINEL, dtype=torch.int32, device=dev)
    meta = torch.full((lanes * _lib.meta_stride(nseq),), SENTINEL, dtype=torch.int32, device=dev)
    return q_idx, pos, meta


def _call(noalloc, sel, cu, lanes, dev):
    lib = _lib.lib()
    n = sel.shape[0]
    nseq = cu.numel() - 1
    q_idx, pos, meta = _outputs(n, lanes, nseq, dev)
    stream = _lib.stream_of(sel)
    if noalloc:
        rc = lib.logo_compact_noalloc(_lib.ptr(sel), n, lanes, _lib.ptr(cu), nseq, _lib.ptr(q_idx),
                                      _lib.ptr(pos), _lib.ptr(meta), stream)
        _lib.check(rc, "logo_compact_noalloc")
    else:
        ws = torch.empty(lib.logo_compact_workspace_bytes(n, lanes), dtype=torch.uint8, device=dev)
        rc = lib.logo_compact(_lib.ptr(sel), n, lanes, _lib.ptr(cu), nseq, _lib.ptr(q_idx), _lib.ptr(pos),
                              _lib.ptr(meta), _lib.ptr(ws), stream)
        _lib.check(rc, "logo_compact")
    torch.cuda.synchronize()
    return q_idx.cpu(), pos.cpu(), meta.cpu()


def _case(n, lanes, lengths, ratio, seed):
    g = torch.Generator().manual_seed(seed)
    sel = (torch.rand(n, lanes, generator=g) < ratio).to(torch.uint8)
    cu = torch.tensor(np.concatenate([[0], np.cumsum(lengths)]), dtype=torch.int32)
    assert int(cu[-1]) == n
    return sel, cu


def test_noalloc_matches_compact_twice_second_smaller(gpu):
    cases = [
        (300000, 16, [1, 0, 150000, 149999], 0.3, 1),   # 74 chunks x 16 lanes of counts
        (70000, 1, [35000, 0, 35000], 0.5, 2),          # smaller: 18 chunks x 1 lane (above the
                                                        # 65536 tokens one workgroup compacts alone)
    ]
    for n, lanes, lengths, ratio, seed in cases:
        print(f"noalloc compaction n={n} lanes={lanes} segments={len(lengths)}", flush=True)
        sel, cu = _case(n, lanes, lengths, ratio, seed)
        selg, cug = sel.to(gpu).contiguous(), cu.to(gpu)
        ref = _call(False, selg, cug, lanes, gpu)
        got = _call(True, selg, cug, lanes, gpu)
        for name, a, b in zip(("q_idx", "pos", "meta"), got, ref):
            assert torch.equal(a, b), f"{name} differs from logo_compact (n={n}, lanes={lanes})"
        # and both equal the oracle's build_selection on every lane
        stride = _lib.meta_stride(len(lengths))
        for lane in range(lanes):
            o = oc.build_selection(sel[:, lane].numpy().astype(bool), cu.numpy())[0]
            sq = o["q_idx"].size
            m = got[2][lane * stride:(lane + 1) * stride].numpy()
            assert m[0] == sq
            np.testing.assert_array_equal(got[0][lane, :sq].numpy(), o["q_idx"])
            np.testing.assert_array_equal(got[1][lane, :sq].numpy(), o["pos_ids"])
            np.testing.assert_array_equal(m[8:8 + len(lengths) + 1], o["cu_seqlens_q"])


def test_noalloc_refuses_more_than_its_scratch(gpu):
    """One token in 65537 lanes needs 65537 counts, one more than the scratch
    holds.  Every buffer is real and sized for that call, so a regression of
    the guard would launch on valid memory rather than fault."""
    lib = _lib.lib()
    n, lanes = 1, LOGO_COMPACT_SCRATCH_INTS + 1
    sel = torch.ones(n, lanes, dtype=torch.uint8, device=gpu)
    cu = torch.tensor([0, n], dtype=torch.int32, device=gpu)
    q_idx = torch.zeros(lanes, n, dtype=torch.int64, device=gpu)
    pos = torch.zeros(lanes, n, dtype=torch.int32, device=gpu)
    meta = torch.zeros(lanes * _lib.meta_stride(1), dtype=torch.int32, device=gpu)
    rc = lib.logo_compact_noalloc(_lib.ptr(sel), n, lanes, _lib.ptr(cu), 1, _lib.ptr(q_idx), _lib.ptr(pos),
                                  _lib.ptr(meta), _lib.stream_of(sel))
    torch.cuda.synchronize()
    assert rc == 1
    assert "scratch" in lib.logo_last_error().decode()
