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


def test_torch_decode_reference_matches_oracle():
    """tests.helpers.torch_decode_attn (the full-size GPU decode checks' fp32
    reference) equals oracle.decode on ragged lengths, GQA, inactive rows and a
    one-key row; a reference that attended one key too far would fail."""
    import torch

    from tests.helpers import torch_decode_attn

    rng = np.random.default_rng(3)
    B, HQ, H, D, T = 4, 6, 2, 16, 70
    q = rng.standard_normal((B, HQ, D)).astype(np.float32)
    k = rng.standard_normal((B, H, T, D)).astype(np.float32)
    v = rng.standard_normal((B, H, T, D)).astype(np.float32)
    lens = [70, 1, 33, 64]
    active = [True, True, False, True]
    ref = decode.decode_attn(q, k, v, lens, active)
    got = torch_decode_attn(torch.tensor(q), torch.tensor(k), torch.tensor(v), lens, torch.tensor(active))
    np.testing.assert_allclose(got.numpy(), ref, rtol=1e-5, atol=1e-6)
    assert np.all(got.numpy()[2] == 0)
    got_all = torch_decode_attn(torch.tensor(q), torch.tensor(k), torch.tensor(v), lens)
    np.testing.assert_allclose(got_all.numpy(), decode.decode_attn(q, k, v, lens), rtol=1e-5, atol=1e-6)
    # planted off-by-one in the key range (one key too many) must be visible
    wrong = torch_decode_attn(torch.tensor(q), torch.tensor(k), torch.tensor(v), lens[:3] + [lens[3] + 1])
    assert np.abs(wrong.numpy()[3] - ref[3]).max() > 1e-3
