"""Pin oracle.decode: a decode step equals the prefill oracle's last row."""

import numpy as np

from oracle import attn, decode


def test_decode_equals_last_prefill_row_global_and_local():
    rng = np.random.default_rng(0)
    B, HQ, H, D, T = 3, 4, 2, 16, 300
    k = rng.standard_normal((B, H, T, D))
    v = rng.standard_normal((B, H, T, D))
    q_seq = rng.standard_normal((B, T, HQ, D))
    lens = [300, 17, 129]
    q = np.stack([q_seq[b, lens[b] - 1] for b in range(B)])
    active = [True, False, True]
    got = decode.decode_attn(q, k, v, lens, active)
    for b in range(B):
        n = lens[b]
        sel = np.zeros(n, bool)
        sel[n - 1] = True
        o, _ = attn.sq_attn_fwd(q_seq[b, :n], k[b].transpose(1, 0, 2)[:n], v[b].transpose(1, 0, 2)[:n], sel, [0, n])
        if active[b]:
            np.testing.assert_allclose(got[b], o[n - 1], rtol=1e-12, atol=1e-12)
        else:
            assert np.all(got[b] == 0)
    # local branch: the last window+1 keys equal the windowed prefill's last row
    w = 128
    b = 0
    n = lens[b]
    lo = n - (w + 1)
    got_l = decode.decode_attn(q[b:b + 1], k[b:b + 1, :, lo:n], v[b:b + 1, :, lo:n], [w + 1])
    o, _ = attn.swa_fwd(q_seq[b, :n], k[b].transpose(1, 0, 2)[:n], v[b].transpose(1, 0, 2)[:n], [0, n], window=w)
    np.testing.assert_allclose(got_l[0], o[n - 1], rtol=1e-12, atol=1e-12)
