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


def _small_layer(seed=0):
    from logo_amd.layers import LoGoConfig

    cfg = LoGoConfig(hidden_size=128, num_attention_heads=2, num_hidden_layers=1, gate_thres_init=0.5)
    g = torch.Generator().manual_seed(seed)
    C, H, D = 128, 2, cfg.head_dim
    p = {
        "q_proj.weight": torch.randn(C, C, generator=g) * 0.05, "k_proj.weight": torch.randn(C, C, generator=g) * 0.05,
        "v_proj.weight": torch.randn(C, C, generator=g) * 0.05, "o_proj.weight": torch.randn(C, C, generator=g) * 0.05,
        "gate_proj.weight": torch.randn(1, C, generator=g) * C ** -0.5,
        "q_global_proj": torch.eye(D).repeat(H, 1, 1) + 0.05 * torch.randn(H, D, D, generator=g),
        "k_global_proj": torch.eye(D).repeat(H, 1, 1) + 0.05 * torch.randn(H, D, D, generator=g),
        "v_global_proj": torch.eye(D).repeat(H, 1, 1) + 0.05 * torch.randn(H, D, D, generator=g),
        "context_norm_local.weight": 1 + 0.1 * torch.randn(D, generator=g),
        "context_norm_global.weight": 1 + 0.1 * torch.randn(D, generator=g),
    }
    p = {k: v.bfloat16().double().requires_grad_() for k, v in p.items()}
    h = torch.randn(1, 150, C, generator=g).bfloat16().double().requires_grad_()
    sel = torch.rand(1, 150, generator=g) < 0.5
    return cfg, p, h, sel


def test_store_mode_float64_is_the_plain_reference():
    from tests.layer_ref import logo_layer_ref

    cfg, p, h, sel = _small_layer()
    a = logo_layer_ref(h, p, cfg, sel)
    b = logo_layer_ref(h, p, cfg, sel, store_dtype=torch.float64)
    np.testing.assert_allclose(a.detach().numpy(), b.detach().numpy(), rtol=0, atol=1e-12)


def test_store_mode_bf16_rounds_outputs_and_gradients_only():
    """bf16 storage: the output and dh are bf16 values, within bf16 storage
    error of the float64 reference; a storage point dropped from the backward
    (plain float64 gradients) gives different gradients."""
    from tests.layer_ref import logo_layer_ref

    cfg, p, h, sel = _small_layer(1)
    dout = torch.randn(1, 150, 128, generator=torch.Generator().manual_seed(2)).bfloat16().double()
    ref = logo_layer_ref(h, p, cfg, sel)
    ref.backward(dout)
    dh64 = h.grad.clone()
    h.grad = None
    out = logo_layer_ref(h, p, cfg, sel, store_dtype=torch.bfloat16)
    out.backward(dout)
    assert torch.equal(out, out.bfloat16().double()) and torch.equal(h.grad, h.grad.bfloat16().double())
    scale = ref.abs().max().item()
    assert (out - ref).abs().max().item() <= 2 ** -5 * scale
    assert (out - ref).abs().mean().item() > 0  # the storage points are applied
    assert (h.grad - dh64).abs().max().item() <= 2 ** -5 * dh64.abs().max().item()
    assert not torch.equal(h.grad, dh64)


def test_rounded_attention_core_backward():
    """The explicit backward of the P / dS-rounding attention core equals torch
    autograd of the plain core when nothing is rounded (float64 'rounding'),
    windowed and GQA included; with bf16 rounding it stays within bf16 error."""
    from tests.layer_ref import _AttnRounded

    rng = np.random.default_rng(3)
    N, H, HK, D = 70, 4, 2, 8
    cu = [0, 30, 70]
    seg = torch.tensor(np.searchsorted(cu, np.arange(N), side="right") - 1)
    pos = torch.arange(N) - torch.tensor(cu)[seg]
    do = torch.tensor(rng.standard_normal((N, H, D)))
    for window in (None, 6):
        base = [torch.tensor(rng.standard_normal(s), requires_grad=True) for s in ((N, H, D), (N, HK, D), (N, HK, D))]
        ref = _attn(*base, seg, pos, None, window)
        ref.backward(do)
        for dtype, tol in ((torch.float64, 1e-12), (torch.bfloat16, 2e-2)):
            xs = [t.detach().clone().requires_grad_() for t in base]
            got = _attn(*xs, seg, pos, None, window, round_dtype=dtype)
            got.backward(do)
            np.testing.assert_allclose(got.detach().numpy(), ref.detach().numpy(), rtol=0, atol=tol)
            for x, b in zip(xs, base):
                np.testing.assert_allclose(x.grad.numpy(), b.grad.numpy(), rtol=0, atol=tol)
