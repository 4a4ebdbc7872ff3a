"""Pin oracle.epilogue against the reference formulas written as torch code.

The torch side restates logo/modules/layernorm.py:17-22 and
logo/layers/logo.py:180-181, :225-226, :256-258 with torch ops (a separate
implementation from the numpy oracle); autograd gives the backward.
"""

import numpy as np
import pytest
import torch

from oracle import epilogue


def torch_rmsnorm(x, w, eps):
    dt = x.dtype
    xf = x.to(torch.float32) if dt != torch.float64 else x
    var = xf.pow(2).mean(-1, keepdim=True)
    xf = xf * torch.rsqrt(var + eps)
    return w * xf.to(dt)


def torch_epilogue(L, G, gate, thres, w_l, w_g, eps):
    N, H, D = L.shape
    Ln = torch_rmsnorm(L, w_l, eps).reshape(N, H * D)
    Gn = torch_rmsnorm(G, w_g, eps).reshape(N, H * D)
    g = gate[:, None].masked_fill(gate[:, None] < thres, 0.0)
    return (1 - g) * Ln + g * Gn


def _inputs(seed, N=37, H=3, D=16):
    rng = np.random.default_rng(seed)
    L = rng.standard_normal((N, H, D))
    G = rng.standard_normal((N, H, D))
    G[::5] = 0.0  # unselected global rows are exactly zero
    gate = 1 / (1 + np.exp(-rng.standard_normal(N)))
    w_l = 1 + 0.1 * rng.standard_normal(D)
    w_g = 1 + 0.1 * rng.standard_normal(D)
    dout = rng.standard_normal((N, H * D))
    return L, G, gate, w_l, w_g, dout


def test_fwd_bwd_float64_match_autograd():
    L, G, gate, w_l, w_g, dout = _inputs(0)
    thres, eps = 0.5, 1e-5
    out = epilogue.epilogue_fwd(L, G, gate, thres, w_l, w_g, eps, bf16=False)
    tl, tg, tgate, twl, twg = (torch.tensor(x, requires_grad=True) for x in (L, G, gate, w_l, w_g))
    tout = torch_epilogue(tl, tg, tgate, thres, twl, twg, eps)
    np.testing.assert_allclose(out, tout.detach().numpy(), rtol=1e-12, atol=1e-12)
    tout.backward(torch.tensor(dout))
    dL, dG, dgate, dwl, dwg = epilogue.epilogue_bwd(L, G, gate, thres, w_l, w_g, eps, dout)
    np.testing.assert_allclose(dL, tl.grad.numpy(), rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(dG, tg.grad.numpy(), rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(dgate, tgate.grad.numpy(), rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(dwl, twl.grad.numpy(), rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(dwg, twg.grad.numpy(), rtol=1e-10, atol=1e-11)


def test_unselected_rows_take_local_branch_only():
    L, G, gate, w_l, w_g, _ = _inputs(1)
    gate[:] = 0.1
    out = epilogue.epilogue_fwd(L, G, gate, 0.5, w_l, w_g, 1e-5, bf16=False)
    ref = epilogue.rmsnorm(L, w_l, 1e-5, bf16=False).reshape(out.shape)
    np.testing.assert_allclose(out, ref, rtol=0, atol=1e-14)
    assert np.all(epilogue.rmsnorm(np.zeros((2, 3, 16)), w_g, 1e-5, bf16=False) == 0)


@pytest.mark.parametrize("seed", [2, 3])
def test_bf16_forward_matches_eager_bf16(seed):
    L, G, gate, w_l, w_g, _ = _inputs(seed, N=64, H=4, D=32)
    bf = lambda x: torch.tensor(x, dtype=torch.float32).bfloat16()
    Lb, Gb, gb, wlb, wgb = bf(L), bf(G), bf(gate), bf(w_l), bf(w_g)
    thres = torch.tensor([0.5]).bfloat16()
    ref = torch_epilogue(Lb, Gb, gb, thres, wlb, wgb, 1e-5).float().numpy()
    f = lambda t: t.float().numpy()
    out = epilogue.epilogue_fwd(f(Lb), f(Gb), f(gb), 0.5, f(wlb), f(wgb), 1e-5, bf16=True)
    # same rounding points: all but a handful of elements identical, none off by more than 1 ulp
    diff = np.abs(out - ref)
    assert (diff == 0).mean() > 0.99
    assert np.all(diff <= np.abs(ref) * 2 ** -7 + 1e-6)


def test_dropped_gate_term_would_be_caught():
    """Planting `out = Ln + g*Gn` (a dropped (1-g) factor) must break the autograd check."""
    L, G, gate, w_l, w_g, _ = _inputs(4)
    good = epilogue.epilogue_fwd(L, G, gate, 0.5, w_l, w_g, 1e-5, bf16=False)
    Ln = epilogue.rmsnorm(L, w_l, 1e-5, bf16=False)
    Gn = epilogue.rmsnorm(G, w_g, 1e-5, bf16=False)
    g = np.where(gate < 0.5, 0.0, gate)[:, None, None]
    bad = (Ln + g * Gn).reshape(good.shape)
    assert np.abs(bad - good).max() > 1e-3
