"""Pin ``oracle.cpu_path.dense_then_mask`` (the timed CPU baseline's formula).

It restates the reference's only CPU-capable formulation (per-segment dense
causal SDPA, logo/ops/dense_full_attn.py:30-69, then the row mask of
logo/ops/selected_full_attn.py:469-471).  Pinned here against the numpy
oracle ``oracle.attn`` on small packed inputs with unselected rows, GQA and a
one-token segment: outputs, and torch autograd gradients against
``oracle.attn.sq_attn_bwd``.  A planted mistake (the causal flag dropped)
must fail the same comparison.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attn, cpu_path


def _case(seed, n=70, hq=4, h=2, d=16):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n, hq, d))
    k = rng.standard_normal((n, h, d))
    v = rng.standard_normal((n, h, d))
    do = rng.standard_normal((n, hq, d))
    sel = rng.random(n) < 0.45
    sel[0] = False  # an unselected first row too
    cu = np.array([0, 23, 24, 70], dtype=np.int32)  # includes a one-token segment
    return q, k, v, do, sel, cu


def _run(q, k, v, do, sel, cu, fn=cpu_path.dense_then_mask):
    qt, kt, vt = (torch.tensor(x, dtype=torch.float64, requires_grad=True) for x in (q, k, v))
    o = fn(qt, kt, vt, torch.tensor(sel), torch.tensor(cu))
    dq, dk, dv = torch.autograd.grad(o, (qt, kt, vt), torch.tensor(do))
    return o.detach().numpy(), dq.numpy(), dk.numpy(), dv.numpy()


@pytest.mark.parametrize("seed", [0, 1])
def test_dense_then_mask_matches_oracle(seed):
    q, k, v, do, sel, cu = _case(seed)
    o, dq, dk, dv = _run(q, k, v, do, sel, cu)
    ro, _ = attn.sq_attn_fwd(q, k, v, sel, cu)
    rdq, rdk, rdv = attn.sq_attn_bwd(q, k, v, ro, do, sel, cu)
    np.testing.assert_allclose(o, ro, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dq, rdq, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, rdk, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dv, rdv, rtol=1e-9, atol=1e-11)
    assert not o[~sel].any() and not dq[~sel].any()


def test_dense_then_mask_all_rows_is_dense_causal():
    q, k, v, do, _, cu = _case(2)
    sel = np.ones(q.shape[0], bool)
    o, *_ = _run(q, k, v, do, sel, cu)
    ro, _ = attn.sq_attn_fwd(q, k, v, None, cu)
    np.testing.assert_allclose(o, ro, rtol=1e-10, atol=1e-12)


def test_planted_non_causal_variant_fails():
    """The same formula without the causal flag must not pass the pin."""

    def no_causal(q, k, v, sel, cu, scale=None):
        N, HQ, D = q.shape
        G = HQ // k.shape[1]
        kk, vv = k.repeat_interleave(G, dim=1), v.repeat_interleave(G, dim=1)
        outs = []
        for s in range(len(cu) - 1):
            b, e = int(cu[s]), int(cu[s + 1])
            o = F.scaled_dot_product_attention(q[b:e].transpose(0, 1)[None], kk[b:e].transpose(0, 1)[None],
                                               vv[b:e].transpose(0, 1)[None], scale=D ** -0.5)
            outs.append(o[0].transpose(0, 1))
        return torch.cat(outs, 0) * sel.to(q.dtype)[:, None, None]

    q, k, v, do, sel, cu = _case(3)
    o, *_ = _run(q, k, v, do, sel, cu, fn=no_causal)
    ro, _ = attn.sq_attn_fwd(q, k, v, sel, cu)
    assert np.abs(o - ro).max() > 1e-3
