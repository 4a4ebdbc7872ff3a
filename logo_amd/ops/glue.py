"""Fused RoPE and RMSNorm launches (``csrc/glue.hip``) for the layer and model glue.

``rope_apply_`` rotates q, k and the global q, k in place in one launch with
the eager bf16 rounding of logo/modules/rotary.py:81-106; ``rope`` is the
differentiable form (new outputs, one launch forward and one backward, both
bit-identical to eager autograd through ``apply_rotary_pos_emb``);
``rms_norm`` computes logo/modules/layernorm.py:17-22 in one launch.  Both run only on ROCm tensors
and raise otherwise (the modules that call them keep plain torch math for CPU
tensors).
"""

import torch
import torch.nn.functional as F

from .. import _lib

__all__ = ["rope_apply_", "rope", "RopeFunction", "rms_norm", "head_proj", "add_rms_norm", "silu_mul",
           "head_linear", "HeadLinearFunction", "head_linear_grad_acc", "attn_inputs", "AttnInputsFunction"]


def _rope_checked(tensors, cos, sin, what):
    if not 1 <= len(tensors) <= 4:
        raise ValueError(f"{what} takes one to four tensors")
    _lib.require_gpu(*tensors, cos, sin)
    D = tensors[0].shape[-1]
    n = tensors[0][..., 0, 0].numel()
    for t in tensors:
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.shape[-1] != D or t[..., 0, 0].numel() != n:
            raise ValueError(f"{what} needs contiguous bf16 [..., T, H, D] tensors of one shape prefix")
    cos = cos.to(torch.bfloat16).contiguous()
    sin = sin.to(torch.bfloat16).contiguous()
    if cos.numel() != n * D or sin.numel() != n * D:
        raise ValueError("cos / sin must be [..., T, D] matching the tensors")
    return cos, sin, n, D


def rope_apply_(tensors, cos, sin):
    """Rotate each ``[..., T, H_i, D]`` bf16 tensor of ``tensors`` (up to four,
    contiguous, all with the same leading ``[..., T]``) in place with
    ``cos/sin [..., T, D]``."""
    tensors = [t for t in tensors if t is not None]
    cos, sin, n, D = _rope_checked(tensors, cos, sin, "rope_apply_")
    args = []
    for i in range(4):
        if i < len(tensors):
            args += [_lib.ptr(tensors[i]), tensors[i].shape[-2]]
        else:
            args += [None, 0]
    lib = _lib.lib()
    _lib.launch("logo_rope_apply", lib.logo_rope_apply, *args, _lib.ptr(cos), _lib.ptr(sin), n, D,
                _lib.DTYPE_BF16, _lib.stream_of(tensors[0]))
    return tensors


def _rope_launch(xs, cos, sin, n, D, inverse):
    ys = [torch.empty_like(x) for x in xs]
    args = []
    for i in range(4):
        if i < len(xs):
            args += [_lib.ptr(xs[i]), _lib.ptr(ys[i]), xs[i].shape[-2]]
        else:
            args += [None, None, 0]
    lib = _lib.lib()
    _lib.launch("logo_rope", lib.logo_rope, *args, _lib.ptr(cos), _lib.ptr(sin), n, D, int(inverse),
                _lib.DTYPE_BF16, _lib.stream_of(xs[0]))
    return ys


class RopeFunction(torch.autograd.Function):
    """RoPE of up to four tensors as one autograd node: the forward rotation
    and, for the backward, the transposed rotation of the incoming gradients,
    each one HIP launch (eager autograd through logo/modules/rotary.py:81-106
    takes about six element-wise passes per tensor each way)."""

    @staticmethod
    def forward(ctx, cos, sin, *xs):
        cos, sin, n, D = _rope_checked(list(xs), cos, sin, "rope")
        ctx.set_materialize_grads(False)  # unused outputs: no zero gradients to rotate
        ctx.save_for_backward(cos, sin)
        ctx.nd = (n, D)
        return tuple(_rope_launch(list(xs), cos, sin, n, D, inverse=False))

    @staticmethod
    def backward(ctx, *gys):
        cos, sin = ctx.saved_tensors
        n, D = ctx.nd
        live = [i for i, g in enumerate(gys) if g is not None]
        gxs = [None] * len(gys)
        if live:
            gin = [gys[i].to(torch.bfloat16).contiguous() for i in live]
            for i, gx in zip(live, _rope_launch(gin, cos, sin, n, D, inverse=True)):
                gxs[i] = gx
        return (None, None, *gxs)


def rope(tensors, cos, sin):
    """Differentiable RoPE of up to four contiguous bf16 ``[..., T, H_i, D]``
    tensors with ``cos/sin [..., T, D]``; returns new tensors."""
    return list(RopeFunction.apply(cos, sin, *tensors))


def rms_norm(x, weight, eps):
    """RMSNorm over the last dimension of bf16 ``x`` with bf16 ``weight``."""
    _lib.require_gpu(x, weight)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("rms_norm takes bf16 tensors")
    xc = x.contiguous()
    cols = xc.shape[-1]
    y = torch.empty_like(xc)
    lib = _lib.lib()
    _lib.launch("logo_rmsnorm", lib.logo_rmsnorm, _lib.ptr(xc), _lib.ptr(weight.contiguous()), _lib.ptr(y),
                xc.numel() // cols, cols, float(eps), _lib.DTYPE_BF16, _lib.stream_of(xc))
    return y


def head_proj(xs, ws):
    """Per-head projections ``x_i [..., H_i, D] @ w_i [H_i, D, E]`` of up to
    three bf16 tensors sharing their leading ``[...]`` (at most 4096 tokens),
    one HIP launch; returns ``[..., H_i, E]`` tensors."""
    if not 1 <= len(xs) == len(ws) <= 3:
        raise ValueError("head_proj takes one to three (x, w) pairs")
    _lib.require_gpu(*xs, *ws)
    D, E = xs[0].shape[-1], ws[0].shape[-1]
    n = xs[0][..., 0, 0].numel()
    xs = [x.contiguous() for x in xs]
    ws = [w.to(torch.bfloat16).contiguous() for w in ws]
    for x, w in zip(xs, ws):
        if x.dtype != torch.bfloat16 or x.shape[-1] != D or x[..., 0, 0].numel() != n:
            raise ValueError("head_proj needs bf16 [..., H, D] inputs of one shape prefix")
        if w.shape != (x.shape[-2], D, E):
            raise ValueError("each weight must be [H, D, E] for its input's H")
    ys = [torch.empty(*x.shape[:-1], E, dtype=torch.bfloat16, device=x.device) for x in xs]
    args = []
    for i in range(3):
        if i < len(xs):
            args += [_lib.ptr(xs[i]), _lib.ptr(ws[i]), _lib.ptr(ys[i]), xs[i].shape[-2]]
        else:
            args += [None, None, None, 0]
    lib = _lib.lib()
    _lib.launch("logo_head_proj", lib.logo_head_proj, *args, n, D, E, _lib.DTYPE_BF16, _lib.stream_of(xs[0]))
    return ys


def add_rms_norm(residual, x, weight, eps):
    """``s = residual + x`` and ``RMSNorm(s)`` (bf16, last dimension) in one
    launch; returns ``(s, normed)``."""
    _lib.require_gpu(residual, x, weight)
    for t in (residual, x, weight):
        if t.dtype != torch.bfloat16:
            raise ValueError("add_rms_norm takes bf16 tensors")
    r = residual.contiguous()
    xc = x.contiguous()
    if r.shape != xc.shape:
        raise ValueError("residual and x must have one shape")
    cols = r.shape[-1]
    s = torch.empty_like(r)
    y = torch.empty_like(r)
    lib = _lib.lib()
    _lib.launch("logo_add_rmsnorm", lib.logo_add_rmsnorm, _lib.ptr(r), _lib.ptr(xc), _lib.ptr(weight.contiguous()),
                _lib.ptr(s), _lib.ptr(y), r.numel() // cols, cols, float(eps), _lib.DTYPE_BF16, _lib.stream_of(r))
    return s, y


def silu_mul(gu):
    """``silu(g) * u`` for ``gu [..., 2 * I]`` holding ``[g | u]`` (a stacked
    gate / up projection), bf16; returns ``[..., I]``."""
    _lib.require_gpu(gu)
    if gu.dtype != torch.bfloat16:
        raise ValueError("silu_mul takes bf16 tensors")
    lead = gu.shape[:-1]
    I2 = gu.shape[-1]
    g2 = gu.reshape(-1, I2)
    if g2.stride(-1) != 1 or g2.stride(0) % 8 != 0:
        g2 = g2.contiguous()
    cols = I2 // 2
    y = torch.empty(g2.shape[0], cols, dtype=torch.bfloat16, device=gu.device)
    lib = _lib.lib()
    _lib.launch("logo_silu_mul", lib.logo_silu_mul, _lib.ptr(g2), g2.stride(0), _lib.ptr(y), g2.shape[0], cols,
                _lib.DTYPE_BF16, _lib.stream_of(g2))
    return y.view(*lead, cols)


def _rows(x):
    """``x [..., H, D]`` as (tensor, token count, row stride) with the head and
    dim axes dense; other layouts are copied."""
    H, D = x.shape[-2], x.shape[-1]
    if not (x.stride(-1) == 1 and x.stride(-2) == D):
        x = x.contiguous()
    x2 = x.reshape(-1, H, D) if x.dim() != 3 else x
    if x2.dim() != 3 or x2.stride(-1) != 1 or x2.stride(-2) != D or x2.stride(0) % 8 != 0 or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    return x2, x2.shape[0], x2.stride(0)


def _head_linear_launch(x, w, transpose_w: bool):
    x2, n, ldx = _rows(x)
    H, D = x2.shape[1], x2.shape[2]
    y = torch.empty(n, H, D, dtype=torch.bfloat16, device=x.device)
    lib = _lib.lib()
    _lib.launch("logo_head_linear", lib.logo_head_linear, _lib.ptr(x2), ldx, _lib.ptr(w), _lib.ptr(y), H * D, n, H, D,
                int(transpose_w), _lib.DTYPE_BF16, _lib.stream_of(x2))
    return y.view(x.shape)


def _head_linear_dw(x, dy):
    """``dw[h] = sum_n x[n, h, :]^T dy[n, h, :]`` as bf16 ``[H, D, D]``."""
    x2, n, ldx = _rows(x)
    d2, _, ldy = _rows(dy)
    H, D = x2.shape[1], x2.shape[2]
    lib = _lib.lib()
    ws = torch.empty((lib.logo_head_linear_dw_workspace_bytes(n, H, D) + 3) // 4, dtype=torch.float32,
                     device=x.device)
    dw = torch.empty(H, D, D, dtype=torch.bfloat16, device=x.device)
    _lib.launch("logo_head_linear_dw", lib.logo_head_linear_dw, _lib.ptr(x2), ldx, _lib.ptr(d2), ldy,
                _lib.ptr(dw), _lib.ptr(ws), n, H, D, _lib.DTYPE_BF16, _lib.stream_of(x2))
    return dw


def head_linear_grad_acc(dy, w, add, out):
    """``out = bf16(bf16(dy @ w^T) + add)`` per head: the input gradient of
    ``head_linear`` summed with another gradient ``add`` of the same tensor,
    rounded exactly as the two-pass chain (the product, then an eager bf16
    add).  ``dy``, ``add`` ``[N, H, D]`` bf16 with dense heads; ``out`` a
    ``[N, H, D]`` view with dense heads and any 8-aligned row stride (for
    instance a column slice of a wider buffer), or ``add`` itself."""
    _lib.require_gpu(dy, w, add, out)
    d2, n, lddy = _rows(dy)
    a2, na, ldadd = _rows(add)
    H, D = d2.shape[1], d2.shape[2]
    if out.dim() != 3 or tuple(out.shape) != (n, H, D) or out.stride(2) != 1 or out.stride(1) != D \
            or out.stride(0) % 8 or out.data_ptr() % 16 or out.dtype != torch.bfloat16:
        raise ValueError("head_linear_grad_acc: out must be a bf16 [N, H, D] view with dense heads")
    if na != n or a2.shape[1:] != d2.shape[1:] or tuple(w.shape) != (H, D, D):
        raise ValueError("head_linear_grad_acc: dy, add and w shapes disagree")
    lib = _lib.lib()
    _lib.launch("logo_head_linear_grad_acc", lib.logo_head_linear_grad_acc, _lib.ptr(d2), lddy,
                _lib.ptr(w), _lib.ptr(a2), ldadd, _lib.ptr(out), out.stride(0), n, H, D, _lib.DTYPE_BF16,
                _lib.stream_of(d2))
    return out


class HeadLinearFunction(torch.autograd.Function):
    """``y[..., h, :] = x[..., h, :] @ w[h]`` with its gradients, every pass on
    the ``[..., H, D]`` layout in place (no head-major copies)."""

    @staticmethod
    def forward(ctx, x, w):
        wc = w.contiguous()
        ctx.save_for_backward(x, wc)
        return _head_linear_launch(x, wc, False)

    @staticmethod
    def backward(ctx, dy):
        x, w = ctx.saved_tensors
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dx = _head_linear_launch(dy, w, True)
        if ctx.needs_input_grad[1]:
            dw = _head_linear_dw(x, dy).to(w.dtype)
        return dx, dw


def head_linear(x, w):
    """``x [..., H, D] @ w [H, D, D]`` per head (bf16 ROCm tensors, D = 128 for
    the weight gradient), differentiable."""
    _lib.require_gpu(x, w)
    if x.dtype != torch.bfloat16 or w.dtype != torch.bfloat16:
        raise ValueError("head_linear takes bf16 tensors")
    H, D = x.shape[-2], x.shape[-1]
    if tuple(w.shape) != (H, D, D):
        raise ValueError(f"head_linear: weight {tuple(w.shape)} does not match heads {H}, dim {D}")
    return HeadLinearFunction.apply(x, w)


class AttnInputsFunction(torch.autograd.Function):
    """The attention inputs of a LoGo layer (linear_proj form) from its hidden
    states, as one autograd node (logo/layers/logo.py:86-94, :112-158):

        q, k, v    = h Wq^T + bq, h Wk^T + bk, h Wv^T + bv   (hipBLASLt GEMMs)
        logit      = h wg^T + bg                            (the gate, before its sigmoid)
        gq, gk, gv = per-head maps of q, k, v               (head_linear)
        returns      rope(q), rope(k), v, rope(gq), rope(gk), gv, logit   (one RoPE launch)

    The forward launches exactly the ops of the unfused chain.  The backward
    differs in where sums happen, not in the products: q, k and v each feed
    the local branch and their global map, and h feeds four projections, so
    autograd would add gradient pairs in separate passes.  Here the RoPE
    backward runs once over the four rotated gradients, the global maps' input
    gradients are written by ``head_linear_grad_acc`` together with the local
    gradients (the same bf16 values as the separate add) straight into one
    ``[N, (H + 2 HK) D + 8]`` buffer whose last columns hold the gate logit's
    gradient and seven zeros, and dh is one GEMM of that buffer with the
    stacked projection weights (seven zero rows pad K to a multiple of 8),
    and the q / k / v weight gradients one GEMM of the buffer's first
    columns with h.  dh is therefore summed in fp32 before one rounding,
    where the chain rounds each projection's share first; each weight
    gradient is the chain's product (same operands, one GEMM launch)."""

    @staticmethod
    def forward(ctx, h, wq, bq, wk, bk, wv, bv, wg, bg, gwq, gwk, gwv, cos, sin, heads, kv_heads):
        B, T, C = h.shape
        D = gwq.shape[-1]
        q = F.linear(h, wq, bq).view(B, T, heads, D)
        k = F.linear(h, wk, bk).view(B, T, kv_heads, D)
        v = F.linear(h, wv, bv).view(B, T, kv_heads, D)
        logit = F.linear(h, wg, bg)
        gws = [w.contiguous() for w in (gwq, gwk, gwv)]
        gq, gk, gv = (_head_linear_launch(x, w, False) for x, w in zip((q, k, v), gws))
        cos, sin, n, _ = _rope_checked([q, k, gq, gk], cos, sin, "attn_inputs")
        qr, kr, gqr, gkr = _rope_launch([q, k, gq, gk], cos, sin, n, D, inverse=False)
        ctx.save_for_backward(h, wq, wk, wv, wg, q, k, v, *gws, cos, sin)
        ctx.dims = (B, T, C, heads, kv_heads, D, n)
        return qr, kr, v, gqr, gkr, gv, logit

    @staticmethod
    def backward(ctx, dqr, dkr, dv, dgqr, dgkr, dgv, dlogit):
        h, wq, wk, wv, wg, q, k, v, gwq, gwk, gwv, cos, sin = ctx.saved_tensors
        B, T, C, H, HK, D, n = ctx.dims
        need = ctx.needs_input_grad
        bf = lambda g: g.to(torch.bfloat16).contiguous()  # noqa: E731
        dqr, dkr, dv, dgqr, dgkr, dgv = (bf(g) for g in (dqr, dkr, dv, dgqr, dgkr, dgv))
        dqa, dka, dgq, dgk = _rope_launch([dqr, dkr, dgqr, dgkr], cos, sin, n, D, inverse=True)
        cols = (H * D, HK * D, HK * D, 8)
        dy = torch.empty(n, sum(cols), dtype=torch.bfloat16, device=h.device)
        outs = dy.split(cols, dim=1)
        for g, w, a, o, nh in zip((dgq, dgk, dgv), (gwq, gwk, gwv), (dqa, dka, dv), outs, (H, HK, HK)):
            head_linear_grad_acc(g.view(n, nh, D), w, a.view(n, nh, D), o.view(n, nh, D))
        outs[3].zero_()
        outs[3][:, 0].copy_(dlogit.reshape(n))
        dgw = [_head_linear_dw(x, g).to(w.dtype) if need[9 + i] else None
               for i, (x, g, w) in enumerate(zip((q, k, v), (dgq, dgk, dgv), (gwq, gwk, gwv)))]
        h2 = h.reshape(n, C)
        dh = None
        if need[0]:
            wcat = torch.cat([wq, wk, wv, wg, wg.new_zeros(7, C)], dim=0)
            dh = torch.mm(dy, wcat).view(B, T, C)
        # q / k / v weight gradients as one GEMM over the buffer's first
        # (H + 2 HK) D columns (read in place), split into the three weights:
        # at B = 4, T = 8192 ~725 us against 3 x ~280 us, where each 2048 x 2048 product
        # fills half the GPU; the gate's column stays out of it (with it, M =
        # 6152 takes ~1000 us) and is a GEMV of its own
        if need[1] and need[3] and need[5]:
            dws = list(torch.mm(dy[:, :sum(cols[:3])].t(), h2).split(cols[:3], dim=0))
        else:
            dws = [torch.mm(o.t(), h2) if need[1 + 2 * i] else None for i, o in enumerate(outs[:3])]
        dws.append(torch.mm(dlogit.reshape(n, 1).to(h2.dtype).t(), h2) if need[7] else None)
        dbs = [None] * 4
        if need[2] or need[4] or need[6] or need[8]:
            dbs = [g if need[2 + 2 * i] else None for i, g in enumerate(dy.sum(0).split(cols))]
            if dbs[3] is not None:
                dbs[3] = dbs[3][:1]
        return (dh, dws[0], dbs[0], dws[1], dbs[1], dws[2], dbs[2], dws[3], dbs[3], *dgw, None, None, None, None)


def attn_inputs(h, q_proj, k_proj, v_proj, gate_proj, global_projs, cos, sin, heads, kv_heads):
    """``(rope(q), rope(k), v, rope(gq), rope(gk), gv, gate_logit)`` of hidden
    states ``h [B, T, C]`` through the ``nn.Linear`` projections (the gate's
    with one output) and the per-head global maps ``global_projs = (Wgq, Wgk,
    Wgv)`` (each ``[H_i, D, D]``), with ``cos/sin [B, T, D]``: ``[B, T, H_i,
    D]`` tensors and the logit ``[B, T, 1]``; bf16 ROCm tensors, D = 128."""
    _lib.require_gpu(h, cos, sin, *global_projs)
    lins = (q_proj, k_proj, v_proj, gate_proj)
    ws = (*(m.weight for m in lins), *global_projs)
    if h.dtype != torch.bfloat16 or any(w.dtype != torch.bfloat16 for w in ws):
        raise ValueError("attn_inputs takes bf16 tensors")
    D = global_projs[0].shape[-1]
    if D != 128 or tuple(global_projs[0].shape) != (heads, D, D) or tuple(global_projs[1].shape) != (kv_heads, D, D):
        raise ValueError("attn_inputs: global maps must be [H, 128, 128] / [HK, 128, 128]")
    if gate_proj.weight.shape[0] != 1:
        raise ValueError("attn_inputs: the gate projection has one output")
    args = [t for m in lins for t in (m.weight, m.bias)]
    return AttnInputsFunction.apply(h, *args, *global_projs, cos, sin, heads, kv_heads)
