"""Pin the float64 torch layer reference's attention core to oracle.attn (CPU)."""

import numpy as np
import torch

from oracle import attn
from tests.layer_ref import _attn


def test_attention_core_matches_oracle():
    rng = np.random.default_rng(0)
    N, H, HK, D = 90, 4, 2, 16
    q = rng.standard_normal((N, H, D))
    k = rng.standard_normal((N, HK, D))
    v = rng.standard_normal((N, HK, D))
    cu = [0, 40, 90]
    seg = torch.tensor(np.searchsorted(cu, np.arange(N), side="right") - 1)
    pos = torch.arange(N) - torch.tensor(cu)[seg]
    sel = rng.random(N) < 0.5
    got = _attn(torch.tensor(q), torch.tensor(k), torch.tensor(v), seg, pos, torch.tensor(sel), None).numpy()
    ref, _ = attn.sq_attn_fwd(q, k, v, sel, cu, scale=D ** -0.5)
    np.testing.assert_allclose(got, ref, rtol=1e-10, atol=1e-12)
    got_w = _attn(torch.tensor(q), torch.tensor(k), torch.tensor(v), seg, pos, None, 5).numpy()
    ref_w, _ = attn.swa_fwd(q, k, v, cu, window=5, scale=D ** -0.5)
    np.testing.assert_allclose(got_w, ref_w, rtol=1e-10, atol=1e-12)
