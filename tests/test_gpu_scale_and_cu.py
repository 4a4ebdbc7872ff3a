"""GPU parity for the op's arguments beyond the defaults: an explicit
``scale`` (the reference's optional argument, logo/ops/selected_full_attn.py:
495-527; the sparse path folds it into its pre-scaled q copies, the window
and dense branches into the exp2 argument), on all three branches, with
``cu_seqlens`` passed as int64 (the reference casts it to int32,
logo/ops/common.py:87), against the float64 oracle at the north-star mean
bound.  A larger scale makes the softmax peakier and dq several units large
(5.6-8.9 at scale 0.2, on every branch alike, the window and dense ones
without the sparse path's pre-scaled q): the max bound scales with the
reference's largest magnitude there, as in the other large-value tests."""

import numpy as np
import pytest
import torch

from logo_amd.ops import dense_causal_attn, sq_full_attn, swa_attn
from oracle import attn
from tests.helpers import assert_within, gen, randn

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("branch,scale", [
    ("sparse", 0.05), ("sparse", 0.2), ("window", 0.05), ("window", 0.2), ("dense", 0.2),
])
def test_explicit_scale_and_int64_cu(gpu, branch, scale):
    n, hq, h, d = 900, 4, 2 if branch == "sparse" else 4, 128
    g = gen(1500 + int(scale * 100) + len(branch))
    q, k, v = randn((n, hq, d), g), randn((n, h, d), g), randn((n, h, d), g)
    do = randn((n, hq, d), g)
    cu = torch.tensor([0, 333, 334, 900], dtype=torch.int64)
    print(f"{branch} scale={scale}", flush=True)
    qg, kg, vg = (x.to(gpu).requires_grad_() for x in (q, k, v))
    window = 64 if branch == "window" else None
    sel = None
    if branch == "sparse":
        sel = torch.rand(n, generator=g) < 0.5
        o = sq_full_attn(qg[None], kg[None], vg[None], sel.to(gpu)[None], scale=scale, cu_seqlens=cu.to(gpu))[0]
    elif branch == "window":
        o = swa_attn(qg[None], kg[None], vg[None], cu.to(gpu), window=window, scale=scale)[0]
    else:
        o = dense_causal_attn(qg[None], kg[None], vg[None], cu.to(gpu), scale=scale)[0]
    o.backward(do.to(gpu))
    qn, kn, vn = (x.double().numpy() for x in (q, k, v))
    s = None if sel is None else sel.numpy()
    cun = cu.numpy().astype(np.int32)
    ro, _ = attn.sq_attn_fwd(qn, kn, vn, s, cun, scale=scale, window=window)
    rdq, rdk, rdv = attn.sq_attn_bwd(qn, kn, vn, ro, do.double().numpy(), s, cun, scale=scale, window=window)
    for name, x, r in (("o", o, ro), ("dq", qg.grad, rdq), ("dk", kg.grad, rdk), ("dv", vg.grad, rdv)):
        big = float(np.abs(r).max())
        assert_within(f"{name} {branch} scale={scale} (max |ref| {big:.2f})", x, r, max_abs=2e-2 * max(1.0, big / 2))
