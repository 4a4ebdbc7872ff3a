"""GPU parity of the fused epilogue against oracle.epilogue.

Forward: the bf16 output reproduces the reference's eager bf16 rounding chain
(oracle bf16 restatement): >= 99% of elements bit-identical, the rest within
two bf16 ulps at magnitude 1.  Against the exact float64 function the error is bounded by
2e-2 * max(1, |ref|) (max) and 2e-3 (mean): the outputs are RMS-normalised,
so |out| reaches ~5 where one bf16 ulp is 0.03 and an absolute 2e-2 bound is
unattainable for any bf16 result, the reference's included.  Backward: dL, dG
within the same bound of the float64 gradient; dgate and the weight gradients
are sums over 2048 (per token) or N*H (per weight) terms, so their bf16
results are checked with the reference's own relative criterion
(assert_close, logo/ops/common.py:34-41) at ratio 5e-3.
"""

import numpy as np
import pytest
import torch

from logo_amd.ops import assert_close
from logo_amd.ops.epilogue import logo_epilogue
from oracle import epilogue
from tests.helpers import gen


def assert_scaled(name, x, ref, max_rel=2e-2, mean_abs=2e-3):
    got = x.detach().double().cpu().numpy()
    ref = np.asarray(ref, dtype=np.float64)
    err = np.abs(got - ref)
    worst = (err / np.maximum(1.0, np.abs(ref))).max()
    assert worst <= max_rel and err.mean() <= mean_abs, f"{name}: scaled max {worst:.3e}, mean {err.mean():.3e}"


def _inputs(n, H, D, seed, dev):
    g = gen(seed)
    L = torch.randn(n, H, D, generator=g).bfloat16()
    G = torch.randn(n, H, D, generator=g).bfloat16()
    gate = torch.sigmoid(torch.randn(n, generator=g)).bfloat16()
    G[gate < 0.5] = 0  # unselected global rows are zero (sq_full_attn output)
    w_l = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    w_g = (1 + 0.1 * torch.randn(D, generator=g)).bfloat16()
    dout = torch.randn(n, H * D, generator=g).bfloat16()
    return L, G, gate, w_l, w_g, dout


@pytest.mark.gpu
@pytest.mark.parametrize("n,H,D", [(333, 16, 128), (64, 4, 64), (8192, 16, 128)])
def test_epilogue_fwd_bwd(gpu, n, H, D):
    L, G, gate, w_l, w_g, dout = _inputs(n, H, D, n + D, gpu)
    thres = torch.tensor([0.5], dtype=torch.bfloat16, device=gpu)
    eps = 1e-5
    Lg, Gg, gg, wl, wg = (x.to(gpu).requires_grad_() for x in (L, G, gate, w_l, w_g))
    out = logo_epilogue(Lg, Gg, gg, thres, wl, wg, eps)
    out.backward(dout.to(gpu))
    f = lambda t: t.float().numpy()
    ref_bf = epilogue.epilogue_fwd(f(L), f(G), f(gate), 0.5, f(w_l), f(w_g), eps, bf16=True)
    ref64 = epilogue.epilogue_fwd(f(L), f(G), f(gate), 0.5, f(w_l), f(w_g), eps, bf16=False)
    got = out.detach().float().cpu().numpy()
    assert (got == ref_bf).mean() > 0.99
    # off-by-one roundings upstream (rsqrt, sum order) can flip one rounding of a
    # term of A + B; under cancellation that is up to one ulp of max(|A|, |B|)
    assert np.all(np.abs(got - ref_bf) <= 2 ** -6 * np.maximum(1.0, np.abs(ref_bf)))
    assert_scaled("out", out, ref64)
    dL, dG, dgate, dwl, dwg = epilogue.epilogue_bwd(f(L), f(G), f(gate), 0.5, f(w_l), f(w_g), eps, f(dout))
    assert_scaled("dL", Lg.grad, dL)
    assert_scaled("dG", Gg.grad, dG)
    t = lambda x: torch.as_tensor(x, dtype=torch.float64)
    assert_close("dgate", t(dgate), gg.grad.double().cpu(), 5e-3)
    assert_close("dw_l", t(dwl), wl.grad.double().cpu(), 5e-3)
    assert_close("dw_g", t(dwg), wg.grad.double().cpu(), 5e-3)
    assert torch.all(gg.grad[gate.to(gpu) < 0.5] == 0)


@pytest.mark.gpu
def test_epilogue_all_unselected_is_local_norm(gpu):
    L, G, gate, w_l, w_g, _ = _inputs(100, 4, 128, 3, gpu)
    gate = torch.full_like(gate, 0.25)
    thres = torch.tensor([0.5], dtype=torch.bfloat16, device=gpu)
    out = logo_epilogue(L.to(gpu), G.to(gpu), gate.to(gpu), thres, w_l.to(gpu), w_g.to(gpu), 1e-5)
    f = lambda t: t.float().numpy()
    ref = epilogue.rmsnorm(f(L), f(w_l), 1e-5, bf16=True).reshape(100, -1)
    assert (out.float().cpu().numpy() == ref).mean() > 0.99
