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
    (4, 16, 4, 128, [2000, 1, 256, 9000]),  # GQA groups of 4 share one cache read
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


@pytest.mark.parametrize("B,H,HK,D", [(32, 16, 16, 128), (5, 4, 2, 64)])
def test_decode_qkv_equals_step_by_step(gpu, B, H, HK, D):
    """The fused decode q / k / v transform is bit-identical to the separate
    launches it replaces (global projection, RoPE of q, k, gq, gk, cache
    appends into the local ring and the global cache) on the same stacked
    projection rows."""
    from logo_amd.layers import rope_cos_sin
    from logo_amd.ops.decode import decode_qkv
    from logo_amd.ops.glue import head_proj, rope_apply_

    g = gen(B + H + D)
    ldq = (H + 2 * HK) * D + 8
    qkv = torch.randn(B, ldq, generator=g).bfloat16().to(gpu)
    ws = [(torch.eye(D) + 0.05 * torch.randn(h, D, D, generator=g)).bfloat16().to(gpu) for h in (H, HK, HK)]
    T = 300
    cache_a = LogoKVCache(1, B, HK, D, max_len=T + 4, window=128, device=gpu)
    cache_b = LogoKVCache(1, B, HK, D, max_len=T + 4, window=128, device=gpu)
    for c in (cache_a, cache_b):
        for t in (c.global_k[0], c.global_v[0], c.local_k[0], c.local_v[0]):
            t.zero_()
        c.set_length(T)
    cos, sin = rope_cos_sin(torch.full((B, 1), T, device=gpu), D, 10000.0, torch.bfloat16)
    gate_col = (H + 2 * HK) * D  # first column past the stacked q | k | v
    qkv[:B, gate_col] = torch.linspace(-12, 12, B, device=gpu).bfloat16()
    q, gq, gate = decode_qkv(qkv, *ws, cos, sin, cache_a, 0, H, HK, gate_col=gate_col)
    # the gate against torch's sigmoid of the same bf16 logits: equal up to the
    # last bf16 bit (both round an fp32 1 / (1 + exp(-z)))
    ref_gate = torch.sigmoid(qkv[:, gate_col])
    diff = (gate.float() - ref_gate.float()).abs()
    assert (diff <= ref_gate.float().abs() * 2.0 ** -8).all()
    assert (gate == ref_gate).float().mean().item() >= 0.99
    # step by step
    qv = qkv[:, :H * D].reshape(B, 1, H, D).contiguous()
    kv = qkv[:, H * D:(H + HK) * D].reshape(B, 1, HK, D).contiguous()
    vv = qkv[:, (H + HK) * D:(H + 2 * HK) * D].reshape(B, 1, HK, D).contiguous()
    gqr, gkr, gvr = head_proj((qv, kv, vv), ws)
    rope_apply_([qv, kv, gqr, gkr], cos, sin)
    cache_b.append(0, kv[:, 0], vv[:, 0], gkr[:, 0], gvr[:, 0])
    torch.cuda.synchronize()
    assert torch.equal(q, qv[:, 0]) and torch.equal(gq, gqr[:, 0])
    for name in ("global_k", "global_v", "local_k", "local_v"):
        assert torch.equal(getattr(cache_a, name)[0], getattr(cache_b, name)[0]), name


@pytest.mark.parametrize("B,HQ,H,D,lens_g,lens_l,thres_dtype", [
    (4, 16, 16, 128, [1, 257, 4096, 3000], [1, 129, 129, 129], torch.bfloat16),
    (3, 8, 2, 64, [200, 128, 37], [129, 128, 37], torch.float32),
])
def test_decode_attn_fused_equals_separate_calls(gpu, B, HQ, H, D, lens_g, lens_l, thres_dtype):
    """Both branches and the epilogue in two launches give, bit for bit, what
    decode_attn (local), decode_attn (global, gate-aware) and logo_epilogue
    give; inactive rows, a single-split global branch (every length <= 256)
    and grouped heads included."""
    from logo_amd.ops.decode import decode_attn_fused
    from logo_amd.ops.epilogue import logo_epilogue

    g = gen(B * D + 7)
    W1 = 129
    tg = max(lens_g) + 32
    dev = lambda t: t.to(gpu)
    q_l = dev(torch.randn(B, HQ, D, generator=g).bfloat16())
    q_g = dev(torch.randn(B, HQ, D, generator=g).bfloat16())
    k_l = dev((torch.randn(B, H, W1, D, generator=g) * 0.5).bfloat16())
    v_l = dev(torch.randn(B, H, W1, D, generator=g).bfloat16())
    k_g = dev((torch.randn(B, H, tg, D, generator=g) * 0.5).bfloat16())
    v_g = dev(torch.randn(B, H, tg, D, generator=g).bfloat16())
    gate = dev(torch.tensor([0.7, 0.2, 0.5, 0.9][:B]).bfloat16())
    thres = torch.tensor([0.5], device=gpu).to(thres_dtype)
    w_l = dev((1 + 0.1 * torch.randn(D, generator=g)).bfloat16())
    w_g = dev((1 + 0.1 * torch.randn(D, generator=g)).bfloat16())
    len_l = torch.tensor(lens_l, dtype=torch.int32, device=gpu)
    len_g = torch.tensor(lens_g, dtype=torch.int32, device=gpu)
    eps = 1e-5
    for _ in range(2):  # the second call reuses nothing from the first
        out = decode_attn_fused(q_l, k_l, v_l, len_l, max(lens_l), q_g, k_g, v_g, len_g, max(lens_g), gate, thres,
                                w_l, w_g, eps)
        local = decode_attn(q_l, k_l, v_l, len_l, max_len=max(lens_l))
        glob = decode_attn(q_g, k_g, v_g, len_g, gate, thres, max_len=max(lens_g))
        ref = logo_epilogue(local.view(B, 1, HQ, D), glob.view(B, 1, HQ, D), gate.view(B, 1), thres, w_l, w_g, eps)
        torch.cuda.synchronize()
        assert torch.equal(out.view(B, 1, HQ * D), ref)
    inactive = (gate.float() < 0.5).nonzero().flatten()
    assert inactive.numel() > 0
