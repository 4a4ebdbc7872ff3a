"""Dense references exported by the reference's op package.

Mirrors logo/ops/dense_full_attn.py: ``sq_full_attn_dense_ref`` is the sparse
op with an all-ones selection (:12-22) and ``sdpa_causal_ref`` is per-segment
causal attention with GQA ``repeat_kv`` through torch's SDPA (:25-69).  These
are reference utilities of the public API, not part of the HIP hot path.
"""

from typing import Optional

import torch
import torch.nn.functional as F

from .sq_attn import sq_full_attn

__all__ = ["sq_full_attn_dense_ref", "sdpa_causal_ref"]


def sq_full_attn_dense_ref(q, k, v, scale: Optional[float] = None,
                           cu_seqlens: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Full causal attention via the sparse kernels (selection = all ones)."""
    B, T, HQ, K = q.shape
    selection = torch.ones(B, T, dtype=torch.bool, device=q.device)
    return sq_full_attn(q, k, v, selection, scale=scale, cu_seqlens=cu_seqlens)


def _repeat_kv(x: torch.Tensor, g: int) -> torch.Tensor:
    B, T, H, D = x.shape
    return x[:, :, :, None, :].expand(B, T, H, g, D).reshape(B, T, H * g, D)


def sdpa_causal_ref(q, k, v, scale: Optional[float] = None,
                    cu_seqlens: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal attention per packed segment using torch SDPA; ``[B,T,HQ,V]``."""
    B, T, HQ, K = q.shape
    H = k.shape[2]
    G = HQ // H
    if scale is None:
        scale = K ** -0.5
    qh = q.transpose(1, 2)
    kh = _repeat_kv(k, G).transpose(1, 2)
    vh = _repeat_kv(v, G).transpose(1, 2)
    if cu_seqlens is None:
        o = F.scaled_dot_product_attention(qh, kh, vh, is_causal=True, scale=scale)
        return o.transpose(1, 2).contiguous()
    assert B == 1
    cu = cu_seqlens.tolist()
    outs = []
    for s in range(len(cu) - 1):
        bos, eos = cu[s], cu[s + 1]
        outs.append(F.scaled_dot_product_attention(
            qh[:, :, bos:eos], kh[:, :, bos:eos], vh[:, :, bos:eos], is_causal=True, scale=scale))
    o = torch.cat(outs, dim=2)
    return o.transpose(1, 2).contiguous()
