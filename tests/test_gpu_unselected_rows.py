"""Sparse mode writes every row of o and dq, through the C ABI.

The forward and dq kernels zero the rows of the tokens no compacted row
writes (the gaps between a lane's selected tokens, the span before its first
and after its last, every row of a lane without selected tokens), so the
caller's buffers need no fill; the forward also zeroes the lse rows past
each lane's rows.  Each call here runs twice, into buffers filled with NaN
and into zero-filled ones: both results must be identical (every row
written, no selected row touched by the zeroing), and the unselected rows
exactly zero.  The compaction likewise writes zero to its row lists past Sq.  Shapes cover the paired 8-wave forward
(one long sequence), long unselected spans at both ends and in the middle,
per-head selections with an empty and a full head, a segment without
selected rows, GQA, the key-range split, a window and fp16.
"""

import pytest
import torch

from logo_amd import _lib
from logo_amd.ops.common import compact_selection
from tests.helpers import gen, markov_selection, randn

pytestmark = pytest.mark.gpu


def _ws(n, nseq, hq, d, dev):
    lib = _lib.lib()
    nbytes = lib.logo_sq_workspace_bytes(n, nseq, hq, d)
    return torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=dev), nbytes


def _fwd(q, k, v, dsel, cu, scale, window, dtype, fill, ws, nbytes):
    lib = _lib.lib()
    n, hq, d = q.shape
    o = torch.full_like(q, fill)
    lse = torch.full((hq, n), fill, dtype=torch.float32, device=q.device)
    rc = lib.logo_sq_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(lse), _lib.ptr(dsel.q_idx),
                         _lib.ptr(dsel.pos), _lib.ptr(dsel.meta), _lib.ptr(cu), n, cu.numel() - 1, hq, k.shape[1], d,
                         d, dsel.lanes, scale, window, dtype, _lib.ptr(ws) if nbytes else None, nbytes,
                         _lib.stream_of(q))
    _lib.check(rc, "logo_sq_fwd")
    return o, lse


def _dq(q, k, v, o, lse, do, dsel, cu, scale, window, dtype, fill, ws, nbytes):
    """delta phase, then dq into a buffer filled with `fill`."""
    lib = _lib.lib()
    n, hq, d = q.shape
    delta = torch.empty(hq, n, dtype=torch.float32, device=q.device)
    q_sel = torch.empty(hq, n, d, dtype=q.dtype, device=q.device)
    do_sel = torch.empty_like(q_sel)
    dq = torch.full_like(q, fill)
    for fn, w, nb in ((lib.logo_sq_bwd_delta, None, 0), (lib.logo_sq_bwd_dq, ws, nbytes)):
        rc = fn(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(do), _lib.ptr(lse), _lib.ptr(delta),
                _lib.ptr(q_sel), _lib.ptr(do_sel), _lib.ptr(dq), None, None, _lib.ptr(dsel.q_idx), _lib.ptr(dsel.pos),
                _lib.ptr(dsel.meta), _lib.ptr(cu), n, cu.numel() - 1, hq, k.shape[1], d, d, dsel.lanes, scale, window,
                dtype, _lib.ptr(w) if nb else None, nb, _lib.stream_of(q))
        _lib.check(rc, "logo_sq_bwd")
    return dq


def _selection(case, n, hq, g):
    if case == "long_spans":
        sel = markov_selection(n, g)
        sel[:3000] = False
        sel[n // 2:n // 2 + 4000] = False
        sel[-5000:] = False
        sel[3000] = True
        return sel
    if case == "per_head":
        sel = torch.rand(n, hq, generator=g) < 0.3
        sel[:, 1] = False   # a lane without rows
        sel[:, 2] = True    # a lane with every row
        sel[700:1300, :] = False  # the second segment [700, 1300) selects nothing
        return sel
    return markov_selection(n, g)


CASES = [
    # name, n, hq, h, d, cu, selection, window, split, dtype
    ("paired", 20000, 4, 4, 128, [0, 20000], "long_spans", -1, False, "bf16"),
    ("paired_split", 20000, 4, 4, 128, [0, 20000], "long_spans", -1, True, "bf16"),
    ("per_head_packed", 3000, 8, 2, 128, [0, 700, 1300, 3000], "per_head", -1, True, "bf16"),
    ("window_d64", 4000, 4, 2, 64, [0, 1500, 4000], "markov", 96, False, "bf16"),
    ("fp16", 5000, 4, 4, 128, [0, 5000], "long_spans", -1, False, "f16"),
]


@pytest.mark.parametrize("name,n,hq,h,d,cu,case,window,split,dt", CASES, ids=[c[0] for c in CASES])
def test_every_row_written(gpu, name, n, hq, h, d, cu, case, window, split, dt):
    g = gen(900 + n)
    tdt = torch.float16 if dt == "f16" else torch.bfloat16
    dtype = _lib.DTYPE_F16 if dt == "f16" else _lib.DTYPE_BF16
    q, k, v = (randn((n, x, d), g, 0.5, tdt) for x in (hq, h, h))
    do = randn((n, hq, d), g, 1.0, tdt)
    sel = _selection(case, n, hq, g)
    cu = torch.tensor(cu, dtype=torch.int32)
    scale = d ** -0.5
    print(f"unselected rows: {name} n={n} hq={hq} h={h} d={d} window={window} split={split} {dt}", flush=True)
    qg, kg, vg, dog, cug = (x.to(gpu) for x in (q, k, v, do, cu))
    dsel = compact_selection(sel.to(gpu), cug)
    ws, nbytes = _ws(n, cu.numel() - 1, hq, d, gpu) if split else (None, 0)
    if split:
        assert nbytes > 0, "this device and shape should allow a split"
    nan = float("nan")

    o_nan, lse = _fwd(qg, kg, vg, dsel, cug, scale, window, dtype, nan, ws, nbytes)
    o_zero, lse_zero = _fwd(qg, kg, vg, dsel, cug, scale, window, dtype, 0.0, ws, nbytes)
    dq_nan = _dq(qg, kg, vg, o_zero, lse, dog, dsel, cug, scale, window, dtype, nan, ws, nbytes)
    dq_zero = _dq(qg, kg, vg, o_zero, lse, dog, dsel, cug, scale, window, dtype, 0.0, ws, nbytes)
    torch.cuda.synchronize()

    unsel = ~(sel if sel.dim() == 2 else sel[:, None].expand(n, hq)).to(gpu)
    for label, got, want in (("o", o_nan, o_zero), ("dq", dq_nan, dq_zero)):
        assert not torch.isnan(got).any(), f"{label}: {int(torch.isnan(got).any(-1).sum())} rows left unwritten"
        assert torch.equal(got, want), f"{label}: a NaN-filled and a zero-filled output differ"
        assert int(got[unsel].count_nonzero()) == 0, f"{label}: an unselected row is not zero"
        assert int(got[~unsel].count_nonzero()) > 0
    # lse: rows past each lane's Sq are zero too (the lanes' rows cover Sq)
    assert torch.equal(lse, lse_zero), "lse: a NaN-filled and a zero-filled buffer differ"
    counts = (~unsel).sum(0).cpu()
    for hq_i in range(hq):
        assert int(lse[hq_i, int(counts[hq_i]):].count_nonzero()) == 0
        assert not torch.isnan(lse[hq_i, :int(counts[hq_i])]).any()


@pytest.mark.parametrize("n,lanes", [(3000, 1), (20000, 1), (20000, 4), (70000, 2)])
@pytest.mark.parametrize("noalloc", [False, True])
def test_compaction_zeroes_entries_past_sq(gpu, n, lanes, noalloc):
    """q_idx / pos entries [Sq, N) are written zero (buffers start at -1), on
    the one-launch path (short or per-head inputs) and the three-launch path."""
    lib = _lib.lib()
    g = gen(77 + n + lanes)
    sel = torch.rand((n, lanes) if lanes > 1 else (n,), generator=g) < 0.3
    if lanes > 1:
        sel[:, 0] = False  # a lane without rows
    cu = torch.tensor([0, n // 3, n], dtype=torch.int32)
    print(f"compaction tails: n={n} lanes={lanes} noalloc={noalloc}", flush=True)
    selg, cug = sel.to(gpu).view(torch.uint8).contiguous(), cu.to(gpu)
    q_idx = torch.full((lanes, n), -1, dtype=torch.int64, device=gpu)
    pos = torch.full((lanes, n), -1, dtype=torch.int32, device=gpu)
    meta = torch.empty(lanes * (8 + 3 * cu.numel()), dtype=torch.int32, device=gpu)
    if noalloc:
        rc = lib.logo_compact_noalloc(_lib.ptr(selg), n, lanes, _lib.ptr(cug), cu.numel() - 1, _lib.ptr(q_idx),
                                      _lib.ptr(pos), _lib.ptr(meta), _lib.stream_of(selg))
    else:
        ws = torch.empty(max(lib.logo_compact_workspace_bytes(n, lanes), 1), dtype=torch.uint8, device=gpu)
        rc = lib.logo_compact(_lib.ptr(selg), n, lanes, _lib.ptr(cug), cu.numel() - 1, _lib.ptr(q_idx), _lib.ptr(pos),
                              _lib.ptr(meta), _lib.ptr(ws), _lib.stream_of(selg))
    _lib.check(rc, "logo_compact")
    torch.cuda.synchronize()
    sel2 = sel if lanes > 1 else sel[:, None]
    stride = meta.numel() // lanes
    for lane in range(lanes):
        want = torch.nonzero(sel2[:, lane]).flatten()
        sq = int(meta[lane * stride].item())
        assert sq == want.numel()
        assert torch.equal(q_idx[lane, :sq].cpu(), want)
        assert int(q_idx[lane, sq:].count_nonzero()) == 0 and int(pos[lane, sq:].count_nonzero()) == 0
