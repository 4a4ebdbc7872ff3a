"""Gate threshold, branch RMSNorm and gated fusion (forward and backward).

Test infrastructure only: see the package docstring.

Restates
--------
* RMSNorm -- logo/modules/layernorm.py:17-22: ``x`` to fp32, ``variance =
  mean(x^2)``, ``x * rsqrt(variance + eps)``, cast back to the input dtype,
  then ``weight * x`` (a second rounding in bf16).
* context norms -- logo/layers/logo.py:180-181 (local), :225-226 (global),
  one ``[D]`` weight shared by every head.
* gate mask and fusion -- :256 ``gate.masked_fill(gate < thres, 0)`` and
  :258 ``(1 - gate) * local + gate * global``, each eager bf16 op rounding its
  result.

``epilogue_fwd(..., bf16=True)`` reproduces every eager rounding point (inputs
are bf16-valued float arrays); ``bf16=False`` is the exact float64 function.
``epilogue_bwd`` is the float64 gradient of the exact function.

Pinning (tests/test_oracle_epilogue.py): the float64 forward and backward
equal torch autograd (float64) of the reference formulas written as torch
modules; unselected rows give exactly RMSNorm_local(L); zero global rows stay
zero; the bf16 forward equals the same torch modules run in bf16 eagerly.
"""

import numpy as np
import torch


def _bf16(x):
    return torch.from_numpy(np.ascontiguousarray(x, dtype=np.float32)).bfloat16().float().numpy()


def rmsnorm(x, w, eps, bf16=True):
    """``x [..., D]``, ``w [D]``."""
    if bf16:
        xf = x.astype(np.float32)
        var = (xf * xf).mean(-1, keepdims=True, dtype=np.float32)
        n = _bf16(xf * (np.float32(1.0) / np.sqrt(var + np.float32(eps))))
        return _bf16(w.astype(np.float32) * n)
    xd = x.astype(np.float64)
    var = (xd * xd).mean(-1, keepdims=True)
    return w.astype(np.float64) * (xd / np.sqrt(var + eps))


def epilogue_fwd(L, G, gate, thres, w_l, w_g, eps, bf16=True):
    """``L, G [N, H, D]``, ``gate [N]`` (post-sigmoid), ``thres`` scalar.

    Returns ``out [N, H*D]``.
    """
    N, H, D = L.shape
    Ln = rmsnorm(L, w_l, eps, bf16)
    Gn = rmsnorm(G, w_g, eps, bf16)
    g = np.where(gate < thres, 0.0, gate)[:, None, None]
    if bf16:
        g = g.astype(np.float32)
        a = _bf16(np.float32(1.0) - g)
        out = _bf16(_bf16(a * Ln) + _bf16(g * Gn))
    else:
        out = (1.0 - g) * Ln + g * Gn
    return out.reshape(N, H * D)


def _rmsnorm_bwd(x, w, eps, dy):
    """Gradient of y = w * x * rsqrt(mean(x^2) + eps) (float64)."""
    D = x.shape[-1]
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    n = x * r
    dn = dy * w
    dx = r * (dn - n * (dn * n).sum(-1, keepdims=True) / D)
    dw = (dy * n).reshape(-1, D).sum(0)
    return dx, dw


def epilogue_bwd(L, G, gate, thres, w_l, w_g, eps, dout):
    """Float64 gradients ``dL, dG [N, H, D]``, ``dgate [N]``, ``dw_l, dw_g [D]``.

    ``dgate`` is zero where ``gate < thres`` (the masked_fill at
    logo/layers/logo.py:256 blocks the gradient there).
    """
    N, H, D = L.shape
    L = L.astype(np.float64)
    G = G.astype(np.float64)
    dout = dout.astype(np.float64).reshape(N, H, D)
    w_l = w_l.astype(np.float64)
    w_g = w_g.astype(np.float64)
    Ln = rmsnorm(L, w_l, eps, bf16=False)
    Gn = rmsnorm(G, w_g, eps, bf16=False)
    sel = ~(gate < thres)
    g = np.where(sel, gate, 0.0)[:, None, None]
    dLn = dout * (1.0 - g)
    dGn = dout * g
    dgate = np.where(sel, (dout * (Gn - Ln)).sum(axis=(1, 2)), 0.0)
    dL, dw_l = _rmsnorm_bwd(L, w_l, eps, dLn)
    dG, dw_g = _rmsnorm_bwd(G, w_g, eps, dGn)
    return dL, dG, dgate, dw_l, dw_g
