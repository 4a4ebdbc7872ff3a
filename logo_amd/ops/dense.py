"""Dense references exported by the op package (logo/ops/__init__.py:14-23).

``sq_full_attn_dense_ref`` is the query-sparse op with every row selected,
which the reference defines as its dense baseline (logo/ops/dense_full_attn.py:12-22).
``sdpa_causal_ref`` is causal attention over each packed segment
(logo/ops/dense_full_attn.py:25-69), written here as one masked attention per
block of query rows: the block's rows see the keys from the start of their
first row's segment up to its last row, and a mask built from segment ids
and positions keeps each row inside its own segment and causal.  Memory stays
at one [rows, keys] score block per call, whatever the sequence length, and
the arithmetic runs in fp32 (results are cast back to q's dtype).  Neither
function is part of the HIP hot path; both run on CPU or GPU tensors.
"""

from typing import Optional

import torch
import torch.nn.functional as F

from .sq_attn import sq_full_attn

__all__ = ["sq_full_attn_dense_ref", "sdpa_causal_ref"]

# query rows per masked-attention call of sdpa_causal_ref
_ROW_BLOCK = 1024


def sq_full_attn_dense_ref(q, k, v, scale: Optional[float] = None,
                           cu_seqlens: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Dense causal attention through the sparse kernels: every row selected."""
    everything = torch.ones(q.shape[:2], dtype=torch.bool, device=q.device)
    return sq_full_attn(q, k, v, everything, scale=scale, cu_seqlens=cu_seqlens)


def _segment_ids(cu: torch.Tensor, n: int) -> torch.Tensor:
    """Segment index of each of the n packed tokens (empty segments skipped)."""
    tok = torch.arange(n, device=cu.device, dtype=cu.dtype)
    return torch.searchsorted(cu, tok, right=True) - 1


def _packed_causal(q, k, v, seg, scale):
    """q [N, HQ, K], k/v [N, H, *] fp32, seg [N] -> [N, HQ, V] fp32."""
    n, hq, _ = q.shape
    g = hq // k.shape[1]
    tok = torch.arange(n, device=q.device)
    # first token of each token's segment
    first = torch.zeros(n, dtype=torch.long, device=q.device)
    if n:
        starts = torch.ones(n, dtype=torch.bool, device=q.device)
        starts[1:] = seg[1:] != seg[:-1]
        first = torch.cummax(torch.where(starts, tok, torch.zeros_like(tok)), dim=0).values
    out = q.new_empty(n, hq, v.shape[2])
    for r0 in range(0, n, _ROW_BLOCK):
        r1 = min(n, r0 + _ROW_BLOCK)
        k0 = int(first[r0])
        rows, keys = tok[r0:r1], tok[k0:r1]
        allowed = (keys[None, :] <= rows[:, None]) & (seg[k0:r1][None, :] == seg[r0:r1][:, None])
        o = F.scaled_dot_product_attention(
            q[r0:r1].transpose(0, 1), k[k0:r1].transpose(0, 1), v[k0:r1].transpose(0, 1),
            attn_mask=allowed, scale=scale, enable_gqa=g > 1)
        out[r0:r1] = o.transpose(0, 1)
    return out


def sdpa_causal_ref(q, k, v, scale: Optional[float] = None,
                    cu_seqlens: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Causal attention per packed segment (GQA when HQ % H == 0): ``[B, T, HQ, V]``.

    With ``cu_seqlens`` the input is one packed batch (B = 1); without it each
    batch row is its own sequence."""
    B, T, HQ, K = q.shape
    if scale is None:
        scale = K ** -0.5
    if cu_seqlens is None:
        cu = torch.arange(0, (B + 1) * T, T, device=q.device)
    else:
        assert B == 1, "packed varlen input (cu_seqlens) must have B == 1"
        cu = cu_seqlens.to(device=q.device, dtype=torch.long)
    n = B * T
    seg = _segment_ids(cu.to(torch.long), n)
    flat = lambda x: x.reshape(n, x.shape[2], x.shape[3]).float()  # noqa: E731
    o = _packed_causal(flat(q), flat(k), flat(v), seg, scale)
    return o.reshape(B, T, HQ, v.shape[3]).to(q.dtype)
