"""Fused gate-threshold / branch-RMSNorm / gated-fusion epilogue.

One HIP kernel replaces the reference's eager chain (logo/layers/logo.py:180-181
``context_norm_local``, :225-226 ``context_norm_global``, :256
``gate.masked_fill(gate < gate_thres, 0)``, :258 ``(1 - gate) * local +
gate * global``; RMSNorm from logo/modules/layernorm.py:17-22), and one kernel
pair its backward.
"""

import torch

from .. import _lib

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
        th, th_dt = _lib.thres_arg(thres)
        out = torch.empty(n, H * D, dtype=L.dtype, device=L.device)
        lib = _lib.lib()
        _lib.launch("logo_epilogue_fwd", lib.logo_epilogue_fwd, _lib.ptr(Lc), _lib.ptr(Gc), _lib.ptr(gc),
                    _lib.ptr(th), th_dt, _lib.ptr(w_l), _lib.ptr(w_g), _lib.ptr(out), n, H, D, float(eps),
                    _lib.DTYPE_BF16, _lib.stream_of(L))
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
        do = dout.contiguous().to(Lc.dtype)
        dL = torch.empty_like(Lc)
        dG = torch.empty_like(Gc)
        dgate = torch.empty_like(gc)
        dwl = torch.empty_like(w_l)
        dwg = torch.empty_like(w_g)
        lib = _lib.lib()
        ws_bytes = lib.logo_epilogue_bwd_workspace_bytes(n, H, D)
        ws = torch.empty((ws_bytes + 3) // 4, dtype=torch.float32, device=Lc.device)
        _lib.launch("logo_epilogue_bwd", lib.logo_epilogue_bwd, _lib.ptr(Lc), _lib.ptr(Gc), _lib.ptr(gc),
                    _lib.ptr(th), _lib.thres_arg(th)[1], _lib.ptr(w_l), _lib.ptr(w_g), _lib.ptr(do), _lib.ptr(dL),
                    _lib.ptr(dG),
                    _lib.ptr(dgate), _lib.ptr(dwl), _lib.ptr(dwg), n, H, D, float(ctx.eps), _lib.ptr(ws),
                    _lib.DTYPE_BF16, _lib.stream_of(Lc))
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
