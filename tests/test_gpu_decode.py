"""GPU parity of the gate-aware decode kernel and the preallocated cache."""

import numpy as np
import pytest
import torch

from logo_amd.ops.decode import LogoKVCache, cache_append, decode_attn
from oracle import decode
from tests.helpers import assert_within, gen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,HQ,H,D,lens", [
    (4, 16, 16, 128, [1, 257, 4096, 3000]),
    (3, 8, 2, 64, [5000, 128, 700]),
])
def test_decode_matches_oracle(gpu, B, HQ, H, D, lens):
    g = gen(B * D)
    t_cap = max(lens) + 64
    q = torch.randn(B, HQ, D, generator=g).bfloat16()
    k = (torch.randn(B, H, t_cap, D, generator=g) * 0.5).bfloat16()
    v = torch.randn(B, H, t_cap, D, generator=g).bfloat16()
    gate = torch.tensor([0.7, 0.2, 0.5, 0.9][:B]).bfloat16()
    thres = torch.tensor([0.5], dtype=torch.bfloat16, device=gpu)
    lens_t = torch.tensor(lens, dtype=torch.int32, device=gpu)
    out = decode_attn(q.to(gpu), k.to(gpu), v.to(gpu), lens_t, gate.to(gpu), thres, max_len=max(lens))
    active = (gate.float() >= 0.5).numpy()
    f = lambda t: t.float().numpy()
    ref = decode.decode_attn(f(q), f(k), f(v), lens, active)
    assert_within("decode", out, ref)
    out_all = decode_attn(q.to(gpu), k.to(gpu), v.to(gpu), lens_t, max_len=max(lens))
    assert_within("decode all rows", out_all, decode.decode_attn(f(q), f(k), f(v), lens, None))


def test_cache_ring_and_local_decode(gpu):
    B, H, D, W = 2, 4, 128, 128
    T = 300
    g = gen(5)
    kl = torch.randn(B, H, T + 1, D, generator=g).bfloat16()
    vl = torch.randn(B, H, T + 1, D, generator=g).bfloat16()
    kg = torch.randn(B, H, T + 1, D, generator=g).bfloat16()
    vg = torch.randn(B, H, T + 1, D, generator=g).bfloat16()
    q = torch.randn(B, H, D, generator=g).bfloat16()
    cache = LogoKVCache(1, B, H, D, max_len=T + 8, window=W, device=gpu)
    cache.prefill(0, kl[:, :, :T].to(gpu), vl[:, :, :T].to(gpu), kg[:, :, :T].to(gpu), vg[:, :, :T].to(gpu))
    cache.set_length(T)
    cache.append(0, kl[:, :, T].to(gpu), vl[:, :, T].to(gpu), kg[:, :, T].to(gpu), vg[:, :, T].to(gpu))
    len_g, len_l = cache.lengths()
    out_l = decode_attn(q.to(gpu), cache.local_k[0], cache.local_v[0], len_l, max_len=W + 1)
    out_g = decode_attn(q.to(gpu), cache.global_k[0], cache.global_v[0], len_g, max_len=T + 1)
    f = lambda t: t.float().numpy()
    ref_l = decode.decode_attn(f(q), f(kl[:, :, T - W:T + 1]), f(vl[:, :, T - W:T + 1]), [W + 1] * B)
    ref_g = decode.decode_attn(f(q), f(kg), f(vg), [T + 1] * B)
    assert_within("local", out_l, ref_l)
    assert_within("global", out_g, ref_g)
    assert torch.equal(cache.global_k[0][:, :, :T + 1].cpu(), kg)
