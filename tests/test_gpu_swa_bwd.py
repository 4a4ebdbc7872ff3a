"""The fused sliding-window backward (logo_sq_bwd_dqkv on the local branch:
dense rows, window <= 128, HQ == H): dq, dk and dv in one pass.

Against the oracle (float64, logo/layers/utils.py:144-147 semantics) through
the public swa_attn autograd path, at the north-star bound scaled by
max(1, max |ref|) as in the other window tests (with one or two visible keys
|dK| reaches 2-4, where one bf16 ulp is 1.6e-2): windows 0 .. 128, head dims
64 and 128, packed segments shorter than a block, ragged last blocks.

Against the generic dq and dk/dv phases through the C ABI at sizes where a
workgroup walks several key blocks (its warm-up block, the dQ carried from
block to block, the last two steps of its run left to the next workgroup):
dk and dv bit-identical (the fused kernel computes S, P, dP and dS from the
same operands in the same order and accumulates dK, dV row tile by row
tile as the dk/dv kernel does), dq within one bf16 ulp of the generic
result plus 2^-9 of its largest entry (the two kernels sum dS K in other
orders, and the dq kernel computes its own S and dP), and repeated calls
bit-identical.
"""

import numpy as np
import pytest
import torch

from logo_amd import _lib
from logo_amd.ops import swa_attn
from logo_amd.ops.common import dense_selection
from oracle import attn
from tests.helpers import assert_within, gen, randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("window,d,cu,h", [
    (128, 128, [0, 50, 51, 900], 2),
    (127, 128, [0, 900], 2),
    (100, 64, [0, 300, 301, 1000], 3),
    (64, 128, [0, 1000], 1),
    (33, 64, [0, 17, 700], 2),
    (16, 128, [0, 640, 1280], 2),
    (1, 128, [0, 200, 900], 1),
    (0, 64, [0, 129, 900], 2),
    (128, 128, [0, 3000, 3001, 5000], 2),  # long runs: blocks spread over workgroups
])
def test_fused_window_backward_matches_oracle(gpu, window, d, cu, h):
    n = cu[-1]
    g = gen(40 + window + d + h)
    q, k, v = (randn((n, h, d), g) for _ in range(3))
    do = randn((n, h, d), g)
    cut = torch.tensor(cu, dtype=torch.int32)
    print(f"fused swa bwd window={window} d={d} h={h} cu={cu}", flush=True)
    qg, kg, vg = (x.to(gpu).requires_grad_() for x in (q, k, v))
    o = swa_attn(qg[None], kg[None], vg[None], cut.to(gpu), window=window)[0]
    o.backward(do.to(gpu))
    qn, kn, vn = (x.float().numpy() for x in (q, k, v))
    ro, _ = attn.sq_attn_fwd(qn, kn, vn, None, cu, window=window)
    rdq, rdk, rdv = attn.sq_attn_bwd(qn, kn, vn, ro, do.float().numpy(), None, cu, window=window)
    for name, x, r in (("o", o, ro), ("dq", qg.grad, rdq), ("dk", kg.grad, rdk), ("dv", vg.grad, rdv)):
        assert_within(name, x, r, max_abs=2e-2 * max(1.0, float(np.abs(r).max())))


def _bwd_call(fn, q, k, v, o, lse, do, delta, dsel, cu, window, scale, dq, dk, dv):
    n, hq, d = q.shape
    rc = fn(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(do), _lib.ptr(lse), _lib.ptr(delta),
            None, None, _lib.ptr(dq) if dq is not None else None, _lib.ptr(dk) if dk is not None else None,
            _lib.ptr(dv) if dv is not None else None, None, None, _lib.ptr(dsel.meta), _lib.ptr(cu), n,
            cu.numel() - 1, hq, k.shape[1], d, d, dsel.lanes, scale, window, _lib.DTYPE_BF16, None, 0,
            _lib.stream_of(q))
    _lib.check(rc, "backward")


@pytest.mark.parametrize("n,h,d,window,cu", [
    (32768, 16, 128, 128, [0, 8192, 16384, 24576, 32768]),  # the local branch of the cfg4 layer
    (40000, 2, 128, 16, [0, 40000]),
    (20000, 4, 64, 100, [0, 7000, 7001, 20000]),
    (9000, 3, 128, 128, [0, 100, 4000, 4001, 9000]),
])
def test_fused_equals_generic_phases(gpu, n, h, d, window, cu):
    lib = _lib.lib()
    g = gen(90 + h + d)
    q, k, v, do = (randn((n, h, d), g).to(gpu) for _ in range(4))
    cut = torch.tensor(cu, dtype=torch.int32, device=gpu)
    dsel = dense_selection(cut, n, gpu)
    scale = d ** -0.5
    print(f"fused vs generic n={n} h={h} d={d} window={window}", flush=True)
    o = torch.empty_like(q)
    lse = torch.empty(h, n, dtype=torch.float32, device=gpu)
    rc = lib.logo_sq_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(o), _lib.ptr(lse), None, None,
                         _lib.ptr(dsel.meta), _lib.ptr(cut), n, len(cu) - 1, h, h, d, d, dsel.lanes, scale, window,
                         _lib.DTYPE_BF16, None, 0, _lib.stream_of(q))
    _lib.check(rc, "logo_sq_fwd")
    delta = torch.empty(h, n, dtype=torch.float32, device=gpu)
    args = (q, k, v, o, lse, do, delta, dsel, cut, window, scale)
    _bwd_call(lib.logo_sq_bwd_delta, *args, None, None, None)
    dq0, dk0, dv0 = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    _bwd_call(lib.logo_sq_bwd_dq, *args, dq0, None, None)
    _bwd_call(lib.logo_sq_bwd_dkv, *args, None, dk0, dv0)
    outs = []
    for _ in range(2):
        dq1, dk1, dv1 = torch.full_like(q, float("nan")), torch.full_like(k, float("nan")), torch.full_like(v, 7.0)
        _bwd_call(lib.logo_sq_bwd_dqkv, *args, dq1, dk1, dv1)
        outs.append((dq1, dk1, dv1))
    torch.cuda.synchronize()
    dq1, dk1, dv1 = outs[0]
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b), "repeated fused calls differ"
    assert torch.equal(dk1, dk0), f"dk: max diff {(dk1.float() - dk0.float()).abs().max():.3e}"
    assert torch.equal(dv1, dv0), f"dv: max diff {(dv1.float() - dv0.float()).abs().max():.3e}"
    x, ref = dq1.float(), dq0.float()
    err = (x - ref).abs()
    bound = 2.0 ** -7 * ref.abs() + 2.0 ** -9 * float(ref.abs().max()) + 2.0 ** -14
    bad = ~(err <= bound)
    assert not bool(bad.any()), f"dq: {int(bad.sum())} entries beyond the bound, worst {float(err.max()):.3e}"
