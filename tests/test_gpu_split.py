"""Key-range split of the forward and dq kernels, through the C ABI.

With a workspace, a head with few query tiles has each tile's keys cut into
pieces that run as separate workgroups; the last piece of a tile to finish
combines the fp32 partials (the forward rescales them by their row maxima).
Against the same call without a workspace (no split): dq to the rounding of
the final bf16 store (at most one bf16 ulp: its fp32 sums run in another
order; P and dS are recomputed from the same lse, so they round alike); o to
one ulp plus 2^-9 max|v| (each piece rounds P to bf16 relative to its own
running max, which moves P's rounding points: at most 2^-9 relative per
weight of a convex combination of v rows); lse to 1e-4; the arrival counters are zero after every call, and repeated split
calls are bit-identical (the combine order is fixed).  Both are checked
against the oracle at the north-star bound (at 32K tokens, against the fp32
torch reference, which is pinned against the oracle on the CPU).  Shapes: one long sequence with
few selected rows (4 pieces per tile), cfg2's per-head selection (2 pieces),
and packed segments with GQA.
"""

import numpy as np
import pytest
import torch

from logo_amd import _lib
from logo_amd.ops.common import compact_selection
from oracle import attn
from tests.helpers import assert_within, gen, randn, torch_sq_attn

pytestmark = pytest.mark.gpu


def _within_ulp(name, x, ref, extra=0.0):
    """|x - ref| <= one bf16 ulp of ref (2^-7 relative, 2^-14 absolute floor) + extra."""
    x, ref = x.float().cpu(), ref.float().cpu()
    err = (x - ref).abs()
    bad = err > 2.0 ** -7 * ref.abs() + 2.0 ** -14 + extra
    assert not bad.any(), f"{name}: {int(bad.sum())} entries beyond the bound, worst {err.max():.3e}"


def _ws(n, nseq, hq, d, dev):
    lib = _lib.lib()
    nbytes = lib.logo_sq_workspace_bytes(n, nseq, hq, d)
    ws = torch.zeros(max(nbytes, 1), dtype=torch.uint8, device=dev)
    return ws, nbytes, lib.logo_sq_workspace_counter_bytes()


def _fwd(q, k, v, dsel, cu, scale, ws, nbytes):
    lib = _lib.lib()
    n, hq, d = q.shape
    o = torch.zeros_like(q)
    lse = torch.zeros(hq, n, dtype=torch.float32, device=q.device)
    rc = lib.logo_sq_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(lse), _lib.ptr(dsel.q_idx),
                         _lib.ptr(dsel.pos), _lib.ptr(dsel.meta), _lib.ptr(cu), n, cu.numel() - 1, hq, k.shape[1], d,
                         d, dsel.lanes, scale, -1, _lib.DTYPE_BF16, _lib.ptr(ws) if nbytes else None, nbytes,
                         _lib.stream_of(q))
    _lib.check(rc, "logo_sq_fwd")
    return o, lse


def _bwd(q, k, v, o, lse, do, dsel, cu, scale, ws, nbytes):
    """delta phase (no workspace), then dq with or without the split."""
    lib = _lib.lib()
    n, hq, d = q.shape
    delta = torch.zeros(hq, n, dtype=torch.float32, device=q.device)
    q_sel = torch.empty(hq, n, d, dtype=q.dtype, device=q.device)
    do_sel = torch.empty_like(q_sel)
    dq = torch.zeros_like(q)
    for fn, w, nb in ((lib.logo_sq_bwd_delta, None, 0), (lib.logo_sq_bwd_dq, ws, nbytes)):
        rc = fn(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(do), _lib.ptr(lse), _lib.ptr(delta),
                _lib.ptr(q_sel), _lib.ptr(do_sel), _lib.ptr(dq), None, None, _lib.ptr(dsel.q_idx), _lib.ptr(dsel.pos),
                _lib.ptr(dsel.meta), _lib.ptr(cu), n, cu.numel() - 1, hq, k.shape[1], d, d, dsel.lanes, scale, -1,
                _lib.DTYPE_BF16, _lib.ptr(w) if nb else None, nb, _lib.stream_of(q))
        _lib.check(rc, "logo_sq_bwd")
    return dq


@pytest.mark.parametrize("n,hq,h,d,ratio,cu,per_head", [
    (16384, 4, 4, 128, 0.03, [0, 16384], False),       # few tiles: 4 pieces per tile
    (8192, 16, 16, 128, 0.5, [0, 8192], True),         # cfg2's selection: 2 pieces
    (6000, 8, 2, 64, 0.3, [0, 2500, 2501, 6000], False),  # packed segments, GQA
    (32768, 16, 16, 128, 0.14, [0, 32768], False),     # one long sequence, 8-wave forward tiles
])
def test_split_matches_unsplit_and_oracle(gpu, n, hq, h, d, ratio, cu, per_head):
    g = gen(500 + hq)
    q, k, v = (randn((n, x, d), g, 0.5) for x in (hq, h, h))
    do = randn((n, hq, d), g)
    sel = torch.rand((n, hq) if per_head else (n,), generator=g) < ratio
    sel[0] = True
    cu = torch.tensor(cu, dtype=torch.int32)
    scale = d ** -0.5
    print(f"split n={n} hq={hq} h={h} d={d} ratio={ratio} per_head={per_head}", flush=True)
    qg, kg, vg, dog, cug = (x.to(gpu) for x in (q, k, v, do, cu))
    dsel = compact_selection(sel.to(gpu), cug)
    ws, nbytes, cnt_bytes = _ws(n, cu.numel() - 1, hq, d, gpu)
    assert nbytes > 0, "this device and shape should allow a split"

    o0, lse0 = _fwd(qg, kg, vg, dsel, cug, scale, None, 0)
    ws[cnt_bytes:] = 0xFF  # the partials: a split call overwrites some of them
    o1, lse1 = _fwd(qg, kg, vg, dsel, cug, scale, ws, nbytes)
    assert bool((ws[cnt_bytes:] != 0xFF).any()), "the forward did not split"
    assert int(ws[:cnt_bytes].count_nonzero()) == 0, "forward left a counter set"
    o2, lse2 = _fwd(qg, kg, vg, dsel, cug, scale, ws, nbytes)
    assert torch.equal(o1, o2) and torch.equal(lse1, lse2)
    _within_ulp("o split vs unsplit", o1, o0, extra=2.0 ** -9 * float(v.float().abs().max()))
    assert_within("lse split vs unsplit", lse1, lse0.cpu(), max_abs=1e-4, mean_abs=1e-5)

    dq0 = _bwd(qg, kg, vg, o0, lse0, dog, dsel, cug, scale, None, 0)
    ws[cnt_bytes:] = 0xFF
    dq1 = _bwd(qg, kg, vg, o0, lse0, dog, dsel, cug, scale, ws, nbytes)
    assert bool((ws[cnt_bytes:] != 0xFF).any()), "dq did not split"
    assert int(ws[:cnt_bytes].count_nonzero()) == 0, "dq left a counter set"
    dq2 = _bwd(qg, kg, vg, o0, lse0, dog, dsel, cug, scale, ws, nbytes)
    assert torch.equal(dq1, dq2)
    _within_ulp("dq split vs unsplit", dq1, dq0)

    # and against the oracle where it finishes in seconds, else against the
    # fp32 torch reference on the GPU (itself pinned against the oracle)
    if n * n * hq * ratio > 2e8:
        ro, (rdq, _, _) = torch_sq_attn(qg, kg, vg, sel.to(gpu), cu, scale=scale, do=dog)
        assert_within("o split vs fp32 reference", o1, ro)
        assert_within("dq split vs fp32 reference", dq1, rdq)
    else:
        qn, kn, vn = (x.float().numpy() for x in (q, k, v))
        ro, _ = attn.sq_attn_fwd(qn, kn, vn, sel.numpy(), cu.numpy(), scale=scale, dtype=np.float32)
        assert_within("o split vs oracle", o1, ro)
        rdq, _, _ = attn.sq_attn_bwd(qn, kn, vn, ro, do.float().numpy(), sel.numpy(), cu.numpy(), scale=scale,
                                     dtype=np.float32)
        assert_within("dq split vs oracle", dq1, rdq)
