"""GPU parity over many short packed segments: about 200 segments of 0 to 150
tokens (zero-length and one-token segments among them) packed into one
sequence, forward and backward against the fp32 torch reference at the
north-star bound:

* the query-sparse path with per-token and per-head selections (GQA), where
  every tile and key block looks its segment up among hundreds;
* the sliding-window branch at windows 16 and 128 (HQ = H, the fused window
  backward: most of its key blocks start or end inside a segment of fewer
  than 128 tokens, and its workgroups' runs of blocks cross segment starts);
* the dense causal branch.

Unselected rows of the sparse output and of dq are exactly zero.  The max
bound scales with the reference's largest magnitude (see _check); the mean
bound is the north-star one.
"""

import pytest
import torch

from logo_amd.ops import dense_causal_attn, sq_full_attn, swa_attn
from tests.helpers import assert_within, cu_from_lengths, gen, randn, torch_sq_attn

pytestmark = pytest.mark.gpu


def _lengths(g, count=200, hi=150):
    lens = torch.randint(0, hi + 1, (count,), generator=g)
    lens[::37] = 0   # zero-length segments
    lens[5::41] = 1  # one-token segments
    return [int(x) for x in lens]


def _grads(fn, q, k, v, do, gpu):
    qg, kg, vg = (x.to(gpu).requires_grad_() for x in (q, k, v))
    o = fn(qg[None], kg[None], vg[None])[0]
    o.backward(do.to(gpu))
    return o, qg.grad, kg.grad, vg.grad


def _check(tag, got, ref):
    # one- and few-token segments concentrate the softmax, and dk / dv reach
    # several units there, where one bf16 rounding alone is ~1.6e-2: the max
    # bound scales with the reference's largest magnitude, as for D = 256
    for name, x, r in zip(("o", "dq", "dk", "dv"), got, ref):
        big = float(r.abs().max())
        assert_within(f"{name} {tag} (max |ref| {big:.2f})", x, r, max_abs=2e-2 * max(1.0, big / 2))


@pytest.mark.parametrize("per_head", [False, True])
def test_sparse_many_segments(gpu, per_head):
    g = gen(1200 + per_head)
    lens = _lengths(g)
    n, hq, h, d = sum(lens), 4, 2, 128
    cu = cu_from_lengths(lens)
    q, k, v = randn((n, hq, d), g), randn((n, h, d), g), randn((n, h, d), g)
    do = randn((n, hq, d), g)
    sel = torch.rand((n, hq) if per_head else (n,), generator=g) < 0.5
    print(f"sparse {len(lens)} segments, {n} tokens, per_head={per_head}", flush=True)
    got = _grads(lambda a, b, c: sq_full_attn(a, b, c, sel.to(gpu)[None], cu_seqlens=cu.to(gpu)), q, k, v, do, gpu)
    ro, grads = torch_sq_attn(q.to(gpu), k.to(gpu), v.to(gpu), sel.to(gpu), cu, do=do.to(gpu))
    _check(f"{len(lens)} segments per_head={per_head}", got, (ro, *grads))
    o, dq = got[0], got[1]
    rows = ~sel.to(gpu) if per_head else ~sel.to(gpu)[:, None].expand(n, hq)
    assert int(o[rows].count_nonzero()) == 0 and int(dq[rows].count_nonzero()) == 0


@pytest.mark.parametrize("window", [16, 128, None])
def test_dense_and_window_many_segments(gpu, window):
    g = gen(1300 + (window or 0))
    lens = _lengths(g)
    n, h, d = sum(lens), 4, 128
    cu = cu_from_lengths(lens)
    q, k, v = randn((n, h, d), g), randn((n, h, d), g), randn((n, h, d), g)
    do = randn((n, h, d), g)
    print(f"window={window} {len(lens)} segments, {n} tokens", flush=True)
    cug = cu.to(gpu)
    if window is None:
        fn = lambda a, b, c: dense_causal_attn(a, b, c, cug)  # noqa: E731
    else:
        fn = lambda a, b, c: swa_attn(a, b, c, cug, window=window)  # noqa: E731
    got = _grads(fn, q, k, v, do, gpu)
    allrows = torch.ones(n, dtype=torch.bool, device=gpu)
    ro, grads = torch_sq_attn(q.to(gpu), k.to(gpu), v.to(gpu), allrows, cu, window=window, do=do.to(gpu))
    _check(f"window={window} {len(lens)} segments", got, (ro, *grads))
