"""Fused gate-threshold / branch-RMSNorm / gated-fusion epilogue.

One HIP kernel replaces the reference's eager chain (logo/layers/logo.py:180-181
``context_norm_local``, :225-226 ``context_norm_global``, :256
``gate.masked_fill(gate < gate_thres, 0)``, :258 ``(1 - gate) * local +
gate * global``; RMSNorm from logo/modules/layernorm.py:17-22), and one kernel
pair its backward.
"""

import torch

from .. import _lib, _torch_ops

__all__ = ["logo_epilogue", "LogoEpilogueFunction"]


class LogoEpilogueFunction(torch.autograd.Function):
    @staticmethod
    def forward(ctx, L, G, gate, thres, w_l, w_g, eps):
        shape = L.shape  # [..., H, D]
        H, D = shape[-2], shape[-1]
        n = L.numel() // (H * D)
        Lc = L.contiguous().view(n, H, D)
        Gc = G.contiguous().view(n, H, D)
        gc = gate.contiguous().view(n)
        th, _ = _lib.thres_arg(thres)
        out = _torch_ops.timed("logo_epilogue_fwd", _torch_ops.ops().epilogue_fwd, Lc, Gc, gc, th, w_l, w_g,
                               float(eps))
        # the threshold is read in place; the backward keeps its own copy (the
        # buffer may be stepped by the budget controller in between)
        ctx.save_for_backward(Lc, Gc, gc, th.clone() if any(ctx.needs_input_grad) else th, w_l, w_g)
        ctx.eps = eps
        ctx.shapes = (shape, gate.shape)
        return out.view(*shape[:-2], H * D)

    @staticmethod
    def backward(ctx, dout):
        Lc, Gc, gc, th, w_l, w_g = ctx.saved_tensors
        (shape, gshape) = ctx.shapes
        n, H, D = Lc.shape
        do = dout.contiguous().to(Lc.dtype).view(n, H * D)
        dL, dG, dgate, dwl, dwg = _torch_ops.timed("logo_epilogue_bwd", _torch_ops.ops().epilogue_bwd, Lc, Gc, gc,
                                                   th, w_l, w_g, do, float(ctx.eps))
        return dL.view(shape), dG.view(shape), dgate.view(gshape), None, dwl, dwg, None


def logo_epilogue(L, G, gate, thres, w_l, w_g, eps: float):
    """``L``/``G``: branch outputs ``[..., H, D]`` (bf16); ``gate``: post-sigmoid
    gate with one value per token (``[...]`` or ``[..., 1]``); ``thres``: the
    threshold buffer; ``w_l``/``w_g``: ``[D]`` context-norm weights.
    Returns ``[..., H*D]``."""
    _lib.require_gpu(L, G, gate, w_l, w_g)
    for t in (L, G, gate, w_l, w_g):
        if t.dtype != torch.bfloat16:
            raise TypeError("logo_epilogue takes bf16 tensors")
    if L.shape != G.shape or gate.numel() * L.shape[-2] * L.shape[-1] != L.numel():
        raise ValueError("shape mismatch between branches and gate")
    return LogoEpilogueFunction.apply(L, G, gate, thres, w_l.contiguous(), w_g.contiguous(), eps)
