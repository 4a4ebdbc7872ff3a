"""GPU checks of the fused RoPE and RMSNorm kernels against the eager torch ops."""

import pytest
import torch
import torch.nn.functional as F

from logo_amd.layers import apply_rope, rope_cos_sin
from logo_amd.ops.glue import rms_norm, rope, rope_apply_
from tests.helpers import gen

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("D", [64, 128])
def test_rope_bitwise_equal_to_eager(gpu, D):
    g = gen(D)
    B, T, H, HK = 2, 37, 4, 2
    pos = torch.randint(0, 20000, (B, T), generator=g).to(gpu)
    cos, sin = rope_cos_sin(pos, D, 10000.0, torch.bfloat16)
    xs = [torch.randn(B, T, h, D, generator=g).bfloat16().to(gpu) for h in (H, HK, H, HK)]
    ref = [apply_rope(x, cos, sin) for x in xs]
    got = [x.clone() for x in xs]
    rope_apply_(got, cos, sin)
    for r, o in zip(ref, got):
        assert torch.equal(r, o)
    # fewer tensors, and a one-token decode shape
    one = [torch.randn(32, 1, 16, D, generator=g).bfloat16().to(gpu)]
    c1, s1 = rope_cos_sin(torch.full((32, 1), 16400, device=gpu), D, 10000.0, torch.bfloat16)
    ref1 = apply_rope(one[0], c1, s1)
    rope_apply_(one, c1, s1)
    assert torch.equal(ref1, one[0])


@pytest.mark.parametrize("D", [64, 128])
def test_rope_autograd_bitwise_equal_to_eager_autograd(gpu, D):
    """The differentiable fused RoPE: outputs and input gradients equal eager
    autograd through apply_rope bit for bit, with one output unused (no
    gradient) and a non-contiguous upstream gradient."""
    g = gen(D + 1)
    B, T, H, HK = 2, 45, 4, 2
    pos = torch.randint(0, 30000, (B, T), generator=g).to(gpu)
    cos, sin = rope_cos_sin(pos, D, 10000.0, torch.bfloat16)
    xs = [torch.randn(B, T, h, D, generator=g).bfloat16().to(gpu) for h in (H, HK, H, HK)]
    dys = [torch.randn(B, T, h, D, generator=g).bfloat16().to(gpu) for h in (H, HK, H)]
    dys[1] = torch.randn(B, T, D, HK, generator=g).bfloat16().to(gpu).transpose(-1, -2)
    ref_in = [x.clone().requires_grad_() for x in xs]
    ref_out = [apply_rope(x, cos, sin) for x in ref_in]
    torch.autograd.backward(ref_out[:3], dys)
    got_in = [x.clone().requires_grad_() for x in xs]
    got_out = rope(got_in, cos, sin)
    torch.autograd.backward(got_out[:3], dys)
    for r, o in zip(ref_out, got_out):
        assert torch.equal(r.detach(), o.detach())
    for r, o in zip(ref_in[:3], got_in[:3]):
        assert torch.equal(r.grad, o.grad)
    assert got_in[3].grad is None or not got_in[3].grad.any()


@pytest.mark.parametrize("rows,cols", [(7, 2048), (64, 128), (3, 4096), (5, 200)])
def test_rmsnorm_matches_eager(gpu, rows, cols):
    g = gen(rows * cols)
    x = (torch.randn(rows, cols, generator=g) * 3).bfloat16().to(gpu)
    w = (1 + 0.1 * torch.randn(cols, generator=g)).bfloat16().to(gpu)
    eps = 1e-5
    xf = x.float()
    eager = w * (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(torch.bfloat16)
    got = rms_norm(x, w, eps)
    same = (got == eager).float().mean().item()
    diff = (got.float() - eager.float()).abs()
    assert same >= 0.99, f"only {same:.4f} of outputs bit-identical to the eager sequence"
    assert (diff <= 2 ** -7 * eager.float().abs().clamp(min=1)).all()
    ref64 = w.double() * (x.double() / torch.sqrt(x.double().pow(2).mean(-1, keepdim=True) + eps))
    assert (got.double() - ref64).abs().max().item() <= 2e-2 * ref64.abs().max().item()


@pytest.mark.parametrize("T,H,HK,D", [(32, 16, 16, 128), (13, 8, 2, 128), (5, 4, 4, 64)])
def test_head_proj_matches_fp64(gpu, T, H, HK, D):
    """Per-head projection kernel (decode path of the global re-parameterisation)
    against a float64 einsum of the same bf16 inputs, within bf16 rounding."""
    from logo_amd.ops.glue import head_proj

    g = gen(T * H + D)
    xs = [torch.randn(T, h, D, generator=g).bfloat16().to(gpu) for h in (H, HK, HK)]
    ws = [(torch.eye(D) + 0.05 * torch.randn(h, D, D, generator=g)).bfloat16().to(gpu) for h in (H, HK, HK)]
    ys = head_proj(xs, ws)
    for x, w, y in zip(xs, ws, ys):
        ref = torch.einsum("thd,hde->the", x.double(), w.double())
        assert y.shape == ref.shape
        assert ((y.double() - ref).abs() <= 2 ** -8 * ref.abs() + 1e-3).all()


@pytest.mark.parametrize("rows,cols", [(32, 2048), (7, 200), (3, 4096)])
def test_add_rmsnorm_matches_eager(gpu, rows, cols):
    """Fused residual add + RMSNorm: the sum bit-identical to the eager bf16
    add, the norm as the rmsnorm kernel on that sum (bitwise)."""
    from logo_amd.ops.glue import add_rms_norm

    g = gen(rows + cols)
    r = (torch.randn(rows, cols, generator=g) * 2).bfloat16().to(gpu)
    x = torch.randn(rows, cols, generator=g).bfloat16().to(gpu)
    w = (1 + 0.1 * torch.randn(cols, generator=g)).bfloat16().to(gpu)
    s, y = add_rms_norm(r, x, w, 1e-5)
    assert torch.equal(s, r + x)
    assert torch.equal(y, rms_norm(r + x, w, 1e-5))


@pytest.mark.parametrize("rows,cols", [(32, 5632), (5, 64)])
def test_silu_mul_matches_eager(gpu, rows, cols):
    """SwiGLU activation on a stacked [g | u] row against eager
    F.silu(g) * u in bf16 (at least 99.9% of elements bit-identical, the rest
    one bf16 rounding apart)."""
    from logo_amd.ops.glue import silu_mul

    g = gen(rows * 3 + cols)
    gu = (torch.randn(rows, 2 * cols, generator=g) * 3).bfloat16().to(gpu)
    got = silu_mul(gu)
    ref = torch.nn.functional.silu(gu[:, :cols]) * gu[:, cols:]
    assert (got == ref).float().mean().item() >= 0.999
    assert ((got.float() - ref.float()).abs() <= 2 ** -7 * ref.float().abs() + 1e-6).all()


@pytest.mark.parametrize("N,H,D,pad", [(300, 4, 128, 0), (2500, 2, 128, 24), (77, 3, 64, 0)])
def test_head_linear_fwd_bwd_matches_fp32(gpu, N, H, D, pad):
    """The per-head linear map on the [N, H, D] layout (strided rows
    included) against fp32 autograd through einsum: forward and input gradient
    within bf16 rounding, weight gradient (D = 128) within an fp32 sum's; two
    runs bit-identical."""
    from logo_amd.ops.glue import head_linear

    g = gen(N + H + D + pad)
    base = torch.randn(N, H * D + pad, generator=g).bfloat16().to(gpu)
    x = base[:, pad:].view(N, H, D) if pad == 0 else base[:, pad:].unflatten(1, (H, D))
    w = (torch.eye(D) + 0.05 * torch.randn(H, D, D, generator=g)).bfloat16().to(gpu)
    dy = torch.randn(N, H, D, generator=g).bfloat16().to(gpu)
    wgrad = D == 128
    xa = x.detach().clone().requires_grad_(True)
    wa = w.detach().clone().requires_grad_(wgrad)
    y = head_linear(xa, wa)
    y.backward(dy)
    xr = x.detach().float().requires_grad_(True)
    wr = w.detach().float().requires_grad_(wgrad)
    yr = torch.einsum("nhd,hde->nhe", xr, wr)
    yr.backward(dy.float())

    def close(a, b, rel):
        b = b.float()
        return ((a.float() - b).abs() <= rel * b.abs() + 2e-3 * b.abs().max()).all()

    assert close(y, yr.detach(), 2.0 ** -7)
    assert close(xa.grad, xr.grad, 2.0 ** -7)
    if wgrad:
        assert close(wa.grad, wr.grad, 2.0 ** -7)
    y2 = head_linear(x, w)
    assert torch.equal(y2, y.detach())


@pytest.mark.parametrize("N,H,D,layout", [(2500, 4, 128, "slice"), (77, 3, 64, "inplace"), (513, 2, 128, "dense")])
def test_head_linear_grad_acc_equals_product_then_add(gpu, N, H, D, layout):
    """``head_linear_grad_acc`` is bit-identical to the two-pass chain it
    replaces (the input-gradient product, then an eager bf16 add), written
    into a column slice of a wider buffer (the other columns untouched), in
    place over the addend, or into a dense tensor; token counts off the
    512-row workgroup grid."""
    from logo_amd.ops.glue import _head_linear_launch, head_linear_grad_acc

    g = gen(7 * N + H + D)
    w = (torch.eye(D) + 0.05 * torch.randn(H, D, D, generator=g)).bfloat16().to(gpu)
    dy = torch.randn(N, H, D, generator=g).bfloat16().to(gpu)
    add = torch.randn(N, H, D, generator=g).bfloat16().to(gpu)
    ref = (_head_linear_launch(dy, w, True).float() + add.float()).bfloat16()
    assert torch.equal(ref, _head_linear_launch(dy, w, True) + add)  # the eager add rounds the same way
    if layout == "slice":
        buf = torch.full((N, 3 * H * D), 7.0, dtype=torch.bfloat16, device=gpu)
        out = buf[:, H * D:2 * H * D].view(N, H, D)
        head_linear_grad_acc(dy, w, add, out)
        assert torch.equal(out, ref)
        assert bool((buf[:, :H * D] == 7).all()) and bool((buf[:, 2 * H * D:] == 7).all())
    elif layout == "inplace":
        a2 = add.clone()
        head_linear_grad_acc(dy, w, a2, a2)
        assert torch.equal(a2, ref)
    else:
        out = torch.empty_like(dy)
        head_linear_grad_acc(dy, w, add, out)
        assert torch.equal(out, ref)


def _attn_inputs_chain(h, lin, gws, cos, sin, H, HK):
    """The unfused chain (separate projections, head_linear nodes, one RoPE
    node): the autograd graph that sums gradient pairs in separate adds."""
    from logo_amd.ops.glue import head_linear

    B, T, _ = h.shape
    q, k, v = (F.linear(h, m.weight, m.bias).view(B, T, n, 128) for m, n in zip(lin, (H, HK, HK)))
    logit = F.linear(h, lin[3].weight, lin[3].bias)
    gq, gk, gv = (head_linear(x, w) for x, w in zip((q, k, v), gws))
    qr, kr, gqr, gkr = rope([q, k, gq, gk], cos, sin)
    return qr, kr, v, gqr, gkr, gv, logit


@pytest.mark.parametrize("bias", [False, True])
def test_attn_inputs_matches_unfused_chain(gpu, bias):
    """The one-node layer inputs (q, k, v and gate projections, global maps,
    RoPE): forward outputs and the global maps' weight gradients
    bit-identical to the unfused chain; dh (summed in fp32 before one
    rounding, where the chain rounds each projection's share first) and the
    projections' weight and bias gradients within bf16 rounding of an fp32
    autograd reference, and at least as close to it as the chain's."""
    from logo_amd.ops.glue import attn_inputs

    torch.manual_seed(5)
    B, T, C, H, HK = 2, 300, 512, 4, 2
    g = gen(31 + bias)
    lin = [torch.nn.Linear(C, n, bias=bias).to(gpu).bfloat16() for n in (H * 128, HK * 128, HK * 128, 1)]
    gws = [(torch.eye(128) + 0.05 * torch.randn(n, 128, 128, generator=g)).bfloat16().to(gpu).requires_grad_()
           for n in (H, HK, HK)]
    pos = torch.randint(0, 8000, (B, T), generator=g).to(gpu)
    cos, sin = rope_cos_sin(pos, 128, 10000.0, torch.bfloat16)
    h = (torch.randn(B, T, C, generator=g) * 0.5).bfloat16().to(gpu).requires_grad_()
    gos = [torch.randn(B, T, n, 128, generator=g).bfloat16().to(gpu) for n in (H, HK, HK, H, HK, HK)]
    gos.append(torch.randn(B, T, 1, generator=g).bfloat16().to(gpu))
    params = [h, *[p for m in lin for p in m.parameters()], *gws]

    def grads(fn):
        for p in params:
            p.grad = None
        outs = fn()
        torch.autograd.backward(outs, gos)
        return [o.detach() for o in outs], [p.grad.clone() for p in params]

    fo, fg = grads(lambda: attn_inputs(h, *lin, gws, cos, sin, H, HK))
    assert fo[6].shape == (B, T, 1)
    co, cg = grads(lambda: _attn_inputs_chain(h, lin, gws, cos, sin, H, HK))
    for a, b in zip(fo, co):
        assert torch.equal(a, b)
    for a, b in zip(fg[-3:], cg[-3:]):
        assert torch.equal(a, b)
    # fp32 reference of the same chain
    hr = h.detach().float().requires_grad_()
    lr = [(m.weight.detach().float().requires_grad_(), None if m.bias is None else m.bias.detach().float()
           .requires_grad_()) for m in lin]
    gr = [w.detach().float().requires_grad_() for w in gws]
    q, k, v = (F.linear(hr, w, b).view(B, T, n, 128) for (w, b), n in zip(lr, (H, HK, HK)))
    gq, gk, gv = (torch.einsum("bthd,hde->bthe", x, w) for x, w in zip((q, k, v), gr))
    c32, s32 = cos.float(), sin.float()
    outs = [apply_rope(q, c32, s32), apply_rope(k, c32, s32), v, apply_rope(gq, c32, s32), apply_rope(gk, c32, s32),
            gv, F.linear(hr, *lr[3])]
    torch.autograd.backward(outs, [x.float() for x in gos])
    refs = [hr.grad, *[p.grad for wb in lr for p in wb if p is not None]]
    for i, r in enumerate(refs):
        f, c = fg[i].float(), cg[i].float()
        scale = r.abs().max()
        ef, ec = (f - r).abs().max() / scale, (c - r).abs().max() / scale
        assert ef <= 2e-2, f"grad {i}: fused max rel err {ef:.3e}"
        assert ef <= ec * 1.5 + 1e-3, f"grad {i}: fused {ef:.3e} vs chain {ec:.3e}"
