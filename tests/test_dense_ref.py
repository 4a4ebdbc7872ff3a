"""``sdpa_causal_ref`` (logo/ops/dense_full_attn.py:25-69) against the oracle, on the CPU.

Packed input with empty and one-token segments and segments that straddle
the 1024-row blocks of the implementation, GQA, V != K, and the batched form
without ``cu_seqlens`` (each batch row its own sequence).
"""

import numpy as np
import pytest
import torch

from logo_amd.ops import sdpa_causal_ref
from oracle import attn


@pytest.mark.parametrize("cu,hq,h,K,V", [
    ([0, 5, 5, 6, 1500, 2100], 4, 2, 16, 16),
    ([0, 1024, 1025, 2049], 2, 2, 8, 12),
    ([0, 37], 3, 1, 8, 8),
])
def test_packed_matches_oracle(cu, hq, h, K, V):
    n = cu[-1]
    g = torch.Generator().manual_seed(n + hq)
    q = torch.randn(1, n, hq, K, generator=g, dtype=torch.float64)
    k = torch.randn(1, n, h, K, generator=g, dtype=torch.float64)
    v = torch.randn(1, n, h, V, generator=g, dtype=torch.float64)
    o = sdpa_causal_ref(q, k, v, cu_seqlens=torch.tensor(cu, dtype=torch.int32))
    ro, _ = attn.sq_attn_fwd(q[0].numpy(), k[0].numpy(), v[0].numpy(), None, cu)
    assert o.shape == (1, n, hq, V) and o.dtype == torch.float64
    # the reference computes in fp32
    np.testing.assert_allclose(o[0].numpy(), ro, rtol=0, atol=2e-5)


def test_batched_without_cu_seqlens_and_scale():
    g = torch.Generator().manual_seed(3)
    B, T = 2, 40
    q = torch.randn(B, T, 2, 8, generator=g)
    k = torch.randn(B, T, 2, 8, generator=g)
    v = torch.randn(B, T, 2, 8, generator=g)
    o = sdpa_causal_ref(q, k, v, scale=0.2)
    for b in range(B):
        ro, _ = attn.sq_attn_fwd(q[b].numpy(), k[b].numpy(), v[b].numpy(), None, [0, T], scale=0.2)
        np.testing.assert_allclose(o[b].numpy(), ro, rtol=0, atol=2e-5)


def test_planted_cross_segment_leak_fails():
    """Treating the whole pack as one sequence must not pass the same check."""
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(1, 30, 2, 8, generator=g) for _ in range(3))
    cu = [0, 12, 30]
    leaked = sdpa_causal_ref(q, k, v, cu_seqlens=torch.tensor([0, 30]))
    ro, _ = attn.sq_attn_fwd(q[0].numpy(), k[0].numpy(), v[0].numpy(), None, cu)
    assert np.abs(leaked[0].numpy() - ro).max() > 1e-2
