"""Query-sparse causal attention (``sq_full_attn``) on the HIP kernels.

Drop-in for logo/ops/selected_full_attn.py:495-527: same signature, the same
``AssertionError`` checks (:518-522), default ``scale = K ** -0.5`` (:523-524),
zero output rows for unselected tokens (:469-471) and gradients for q, k, v
only (:492).  The same kernels, in dense mode with a window, give the local
sliding-window branch (``swa_attn``) and the dense causal global branch
(``dense_causal_attn``).
"""

import functools
import os
from typing import Optional

import torch
import torch.nn.functional as F

from .. import _lib, _torch_ops
from .common import DeviceSelection, compact_selection, dense_selection

__all__ = ["sq_full_attn", "swa_attn", "dense_causal_attn", "SQFullAttentionFunction"]

_custom_fwd = functools.partial(torch.amp.custom_fwd, device_type="cuda")
_custom_bwd = functools.partial(torch.amp.custom_bwd, device_type="cuda")


# Head dims the gfx950 kernels are compiled for: 64 and 128 on the tuned
# kernels, 256 on the generic ones.  A call with other K, V <= 256 (V != K
# included, as the reference allows: its V is a separate constexpr and K fits
# one block of <= 256, logo/ops/selected_full_attn.py:341-351, :344) runs on
# the next compiled dim with q, k and v zero-padded: zero columns add nothing
# to q.k, and they give zero output and gradient columns, which are sliced off.
KERNEL_HEAD_DIMS = (64, 128, 256)


def kernel_head_dim(K: int, V: int) -> int:
    """The compiled head dim a call with key dim K and value dim V runs on."""
    assert K <= 256, "K must fit in a single block (<=256)"
    assert 0 < K and 0 < V <= 256, "the gfx950 kernels take head dims K, V in [1, 256]"
    m = max(K, V)
    return 64 if m <= 64 else 128 if m <= 128 else 256


def kernel_dtype(q, k, v, sparse: bool, window: int) -> torch.dtype:
    """The element type a call computes in (fp32 accumulation either way).

    The reference's Triton dots run in the input dtype
    (logo/ops/selected_full_attn.py:80, :93-99, :108).  On the query-sparse
    path (no window): fp32 inputs (any of q, k, v) run on the fp32 kernels,
    all three in fp32 (the others are widened, exactly), and fp16 q, k, v on
    the fp16 kernels.  Everything else runs in bf16: bf16 inputs, mixed 16-bit
    inputs, and the dense / sliding-window branches (the reference's flash-attn
    branches take 16-bit inputs only); outputs are cast back to v's dtype."""
    if sparse and window < 0:
        if torch.float32 in (q.dtype, k.dtype, v.dtype):
            return torch.float32
        if q.dtype == k.dtype == v.dtype == torch.float16:
            return torch.float16
    return torch.bfloat16


def _to_kernel(t: torch.Tensor, d: int, dtype: torch.dtype = torch.bfloat16) -> torch.Tensor:
    """[B, T, H, X] -> contiguous [B*T, H, d] of ``dtype``, zero-padded along X."""
    B, T, H, X = t.shape
    t = t.reshape(B * T, H, X)
    if X != d:
        t = F.pad(t, (0, d - X))
    return t.contiguous() if t.dtype == dtype else t.to(dtype).contiguous()


def _fwd(q, k, v, dsel: DeviceSelection, scale: float, window: int):
    """o [N, HQ, D] (unselected rows zero) and lse [HQ, N] (log2 domain)."""
    return _torch_ops.timed("logo_sq_fwd", _torch_ops.ops().sq_fwd, q, k, v, dsel.q_idx, dsel.pos, dsel.meta,
                            dsel.cu, dsel.lanes, float(scale), int(window))


_side_streams = {}


def _side_stream(dev: torch.device) -> torch.cuda.Stream:
    """One extra stream per device, at the default priority, for the dk / dv
    launch of packed backward calls."""
    s = _side_streams.get(dev.index)
    if s is None:
        s = _side_streams[dev.index] = torch.cuda.Stream(device=dev)
    return s


def _overlap_dkv(dsel: DeviceSelection) -> bool:
    """Whether dk / dv runs on the side stream beside dq: opt-in
    (LOGO_BWD_OVERLAP=1), for calls that pack more than one sequence.  It
    pays where sequences of unequal length leave the heaviest tiles of the
    longest one running alone at the end of each kernel's grid (four packed
    sequences of 2.8K-12.5K tokens, 16 heads, D = 128, r = 0.25: fwd + bwd
    1.49 -> 1.44 ms), and costs where the grids are balanced (the LoGo
    layer at B = 4, T = 8192, four sequences of 8192 tokens: 7.33 -> 7.40
    ms per step); the lengths are on the device, so the choice is the
    caller's.  A single sequence keeps one stream either way
    (its heaviest-first tile order balances each grid; T = 32K at r = 0.125,
    0.25, 0.5 measured the same), and so does a backward traced by
    torch.compile."""
    return (dsel.cu.numel() > 2 and os.environ.get("LOGO_BWD_OVERLAP", "0") == "1"
            and not torch.compiler.is_compiling())


def _bwd(q, k, v, o, lse, do, dsel: DeviceSelection, scale: float, window: int):
    """dq (unselected rows zero), dk, dv: the delta phase (with the compacted
    q / dO copies of sparse mode), then dq and dk / dv as two launches, or
    as the one fused pass of the sliding-window branch (dense rows, window
    <= 128, HQ == H; the library picks the kernels, this only keeps the two
    launches separately timed where they are separate).

    dq and dk / dv read only the delta phase's outputs and q, k, v, so with
    the overlap switched on (``_overlap_dkv``) dk / dv is launched first, on
    a side stream, and dq behind it on the caller's stream: dq's workgroups
    take the CUs that dk / dv's tail leaves idle.  The caller's stream waits
    for the side stream before returning (graph capture forks and joins the
    same way), and dk / dv are marked as used on the caller's stream for the
    caching allocator."""
    ops = _torch_ops.ops()
    args = (q, k, v, o, lse, do, dsel.q_idx, dsel.pos, dsel.meta, dsel.cu, dsel.lanes, float(scale), int(window))
    ws = _torch_ops.timed("logo_sq_bwd_delta", ops.sq_bwd_delta, *args)
    if dsel.q_idx is None and 0 <= window <= 128 and q.shape[1] == k.shape[1]:
        return _torch_ops.timed("logo_sq_bwd_dqkv", ops.sq_bwd_dqkv, *args, *ws)
    if _overlap_dkv(dsel):
        main = torch.cuda.current_stream(q.device)
        side = _side_stream(q.device)
        side.wait_stream(main)
        with torch.cuda.stream(side):
            dk, dv = _torch_ops.timed("logo_sq_bwd_dkv", ops.sq_bwd_dkv, *args, *ws)
        dq = _torch_ops.timed("logo_sq_bwd_dq", ops.sq_bwd_dq, *args, *ws)
        main.wait_stream(side)
        dk.record_stream(main)
        dv.record_stream(main)
        return dq, dk, dv
    dq = _torch_ops.timed("logo_sq_bwd_dq", ops.sq_bwd_dq, *args, *ws)
    dk, dv = _torch_ops.timed("logo_sq_bwd_dkv", ops.sq_bwd_dkv, *args, *ws)
    return dq, dk, dv


class SQFullAttentionFunction(torch.autograd.Function):
    """Autograd wrapper (logo/ops/selected_full_attn.py:449-492)."""

    @staticmethod
    @_custom_fwd
    def forward(ctx, q, k, v, scale, dsel: DeviceSelection, window: int = -1):
        B, T, HQ, K = q.shape
        H = k.shape[2]
        V = v.shape[3]
        d = kernel_head_dim(K, V)
        in_dtypes = (q.dtype, k.dtype, v.dtype)
        kt = kernel_dtype(q, k, v, dsel.q_idx is not None, window)
        qf, kf, vf = _to_kernel(q, d, kt), _to_kernel(k, d, kt), _to_kernel(v, d, kt)
        o, lse = _fwd(qf, kf, vf, dsel, scale, window)
        ctx.save_for_backward(qf, kf, vf, o, lse)
        ctx.dsel = dsel
        ctx.scale = scale
        ctx.window = window
        ctx.shapes = (B, T, HQ, H, K, V)
        ctx.in_dtypes = in_dtypes
        out = o.view(B, T, HQ, d)
        if V != d:
            out = out[..., :V].contiguous()
        # the output has v's dtype (logo/ops/selected_full_attn.py:349)
        return out if v.dtype == kt else out.to(v.dtype)

    @staticmethod
    @_custom_bwd
    def backward(ctx, do):
        qf, kf, vf, o, lse = ctx.saved_tensors
        B, T, HQ, H, K, V = ctx.shapes
        d = qf.shape[2]
        dof = _to_kernel(do, d, qf.dtype)
        dq, dk, dv = _bwd(qf, kf, vf, o, lse, dof, ctx.dsel, ctx.scale, ctx.window)
        tq, tk, tv = ctx.in_dtypes
        dq = dq.view(B, T, HQ, d)[..., :K].to(tq)
        dk = dk.view(B, T, H, d)[..., :K].to(tk)
        dv = dv.view(B, T, H, d)[..., :V].to(tv)
        return dq, dk, dv, None, None, None


def _check_shapes(q, k, v):
    """The reference's rank and GQA checks (logo/ops/selected_full_attn.py:518-519)
    plus the shape agreement its kernels assume; all before any launch."""
    assert q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q/k/v must be [B, T, H, D]"
    B, T, HQ, K = q.shape
    H = k.shape[2]
    assert HQ % H == 0, "HQ must be a multiple of H (GQA)"
    assert tuple(k.shape[:2]) == (B, T) and tuple(v.shape[:2]) == (B, T), "q/k/v must share [B, T]"
    assert v.shape[2] == H, "k and v must have the same number of heads"
    assert k.shape[3] == K, "q and k must have the same head dim K"
    kernel_head_dim(K, v.shape[3])
    return B, T, HQ, H, K


def _check_qkv(q, k, v):
    B, T, HQ, H, K = _check_shapes(q, k, v)
    _lib.require_gpu(q, k, v)
    return B, T, HQ, H, K


def sq_full_attn(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    selection: torch.Tensor,
    scale: Optional[float] = None,
    cu_seqlens: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    r"""Selected-query full causal attention.

    Args:
        q: queries `[1, total_tokens, HQ, K]`.
        k: keys    `[1, total_tokens, H, K]` (GQA when HQ % H == 0).
        v: values  `[1, total_tokens, H, V]`.
        selection: per-token bool mask `[1, total_tokens]`, or the per-head
            extension `[1, total_tokens, HQ]`.
        scale: attention scale; defaults to `K ** -0.5`.
        cu_seqlens: required `[Nseq+1]` int tensor for packed varlen input.

    Returns:
        o: `[1, total_tokens, HQ, V]`; rows for unselected query tokens are 0.
    """
    assert q.dim() == 4 and k.dim() == 4 and v.dim() == 4, "q/k/v must be [B, T, H, D]"
    B, T, HQ, K = q.shape
    H = k.shape[2]
    assert HQ % H == 0, "HQ must be a multiple of H (GQA)"
    per_head = selection.dim() == 3
    assert selection.dtype == torch.bool and (
        selection.shape == (B, T) or (per_head and selection.shape == (B, T, HQ))
    ), "selection must be a bool mask [B, T]"
    assert B == 1, "sq_full_attn only supports B=1 packed-varlen input"
    assert cu_seqlens is not None, "sq_full_attn requires explicit cu_seqlens"
    _check_shapes(q, k, v)
    if scale is None:
        scale = K ** -0.5
    _lib.require_gpu(q, k, v, selection)
    if T == 0:
        return q.new_zeros(B, T, HQ, v.shape[3])
    dsel = compact_selection(selection.reshape(B * T, *selection.shape[2:]), cu_seqlens)
    dsel.B, dsel.T = B, T
    return SQFullAttentionFunction.apply(q, k, v, scale, dsel, -1)


def swa_attn(q, k, v, cu_seqlens: torch.Tensor, window: int = 128,
             scale: Optional[float] = None) -> torch.Tensor:
    """Causal sliding-window attention over every row: keys ``[p - window, p]``
    of the row's own segment (flash-attn ``window_size=(w, w)``, ``causal=True``
    as used by logo/layers/utils.py:144-147, :166-178).  ``q [1, N, HQ, D]``."""
    B, T, HQ, H, K = _check_qkv(q, k, v)
    assert B == 1, "swa_attn takes packed [1, N, H, D] input"
    if scale is None:
        scale = K ** -0.5
    if T == 0:
        return q.new_zeros(B, T, HQ, v.shape[3])
    dsel = dense_selection(cu_seqlens, B * T, q.device)
    return SQFullAttentionFunction.apply(q, k, v, scale, dsel, int(window))


def dense_causal_attn(q, k, v, cu_seqlens: torch.Tensor, scale: Optional[float] = None) -> torch.Tensor:
    """Dense causal attention over every row (the ``"flash"`` global branch,
    logo/layers/logo.py:211-224), on the same kernels without compaction."""
    B, T, HQ, H, K = _check_qkv(q, k, v)
    assert B == 1, "dense_causal_attn takes packed [1, N, H, D] input"
    if scale is None:
        scale = K ** -0.5
    if T == 0:
        return q.new_zeros(B, T, HQ, v.shape[3])
    dsel = dense_selection(cu_seqlens, B * T, q.device)
    return SQFullAttentionFunction.apply(q, k, v, scale, dsel, -1)
