"""The reference's CPU-capable formulation, timed as the CPU baseline.

Test/bench infrastructure only: see the package docstring.

The reference's Triton path has no CPU implementation; its only formulation
that runs on a CPU is dense causal attention per packed segment through
torch SDPA (``sdpa_causal_ref``, logo/ops/dense_full_attn.py:30-69) with the
unselected rows then zeroed (logo/ops/selected_full_attn.py:469-471).  This
restates that in torch fp32 and differentiates it with autograd.
"""

import time

import torch
import torch.nn.functional as F


def dense_then_mask(q, k, v, sel, cu, scale=None):
    """q [N, HQ, D], k/v [N, H, D] fp32 CPU tensors, sel bool [N]; -> o [N, HQ, D]."""
    N, HQ, D = q.shape
    G = HQ // k.shape[1]
    if scale is None:
        scale = D ** -0.5
    kk = k.repeat_interleave(G, dim=1)
    vv = v.repeat_interleave(G, dim=1)
    outs = []
    cul = [int(x) for x in cu]
    for s in range(len(cul) - 1):
        b, e = cul[s], cul[s + 1]
        o = F.scaled_dot_product_attention(q[b:e].transpose(0, 1)[None], kk[b:e].transpose(0, 1)[None],
                                           vv[b:e].transpose(0, 1)[None], is_causal=True, scale=scale)
        outs.append(o[0].transpose(0, 1))
    o = torch.cat(outs, dim=0)
    return o * sel.to(o.dtype)[:, None, None]


def time_fwd_bwd(q, k, v, sel, cu, do, threads, repeats=1):
    """Seconds per fwd+bwd of dense_then_mask (autograd), best of ``repeats``."""
    torch.set_num_threads(threads)
    best = float("inf")
    for _ in range(repeats):
        qq, kk, vv = (x.detach().clone().requires_grad_() for x in (q, k, v))
        t0 = time.perf_counter()
        o = dense_then_mask(qq, kk, vv, sel, cu)
        torch.autograd.grad(o, (qq, kk, vv), do)
        best = min(best, time.perf_counter() - t0)
    return best
