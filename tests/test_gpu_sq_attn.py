"""GPU parity of the HIP query-sparse attention against the oracle.

Small and mid sizes compare with oracle.attn (numpy, CPU); the full-size
cases use the fp32 torch reference of tests/helpers.py (pinned against the
oracle in tests/test_oracle_attn.py).  Tolerance: bf16
outputs and gradients within max-abs 2e-2 and mean-abs 2e-3 of the fp32
reference.
"""

import numpy as np
import pytest
import torch

from logo_amd.ops import dense_causal_attn, sq_full_attn, sq_full_attn_dense_ref, swa_attn
from oracle import attn
from tests.helpers import (assert_within, cu_from_lengths, err_stats, gen, markov_selection, randn,
                           torch_sq_attn, varlen_lengths)

pytestmark = pytest.mark.gpu


def _run(q, k, v, sel, cu, dev, do=None, scale=None):
    qg, kg, vg = (x.to(dev).requires_grad_(do is not None) for x in (q, k, v))
    o = sq_full_attn(qg[None], kg[None], vg[None], sel.to(dev)[None], scale=scale, cu_seqlens=cu.to(dev))[0]
    if do is None:
        return o, None
    o.backward(do.to(dev))
    return o, (qg.grad, kg.grad, vg.grad)


def _oracle(q, k, v, sel, cu, do=None, scale=None, window=None, dtype=np.float64):
    qn, kn, vn = (x.float().numpy() for x in (q, k, v))
    o, lse = attn.sq_attn_fwd(qn, kn, vn, None if sel is None else sel.numpy(), cu.numpy(), scale=scale,
                              window=window, dtype=dtype)
    if do is None:
        return o, None
    grads = attn.sq_attn_bwd(qn, kn, vn, o, do.float().numpy(), None if sel is None else sel.numpy(),
                             cu.numpy(), scale=scale, window=window, dtype=dtype)
    return o, grads


@pytest.mark.parametrize("n,hq,h,d,ratio,cu,per_head", [
    (512, 4, 4, 64, 0.5, [0, 512], True),            # cfg1 shape, per-head extension
    (512, 4, 4, 64, 0.5, [0, 512], False),           # cfg1 shape, reference API
    (700, 4, 2, 128, 0.4, [0, 1, 1, 200, 700], False),  # GQA, zero/single-token segments
    (1000, 2, 2, 128, 1.0, [0, 333, 1000], False),   # all selected
    (300, 2, 1, 64, 0.1, [0, 150, 300], True),       # sparse per-head GQA
])
def test_fwd_bwd_matches_oracle(gpu, n, hq, h, d, ratio, cu, per_head):
    g = gen(n + hq)
    q, k, v = randn((n, hq, d), g), randn((n, h, d), g), randn((n, h, d), g)
    do = randn((n, hq, d), g)
    sel = torch.rand((n, hq) if per_head else (n,), generator=g) < ratio
    cu = torch.tensor(cu, dtype=torch.int32)
    print(f"fwd/bwd n={n} hq={hq} h={h} d={d} ratio={ratio} per_head={per_head}", flush=True)
    o, (dq, dk, dv) = _run(q, k, v, sel, cu, gpu, do)
    ro, (rdq, rdk, rdv) = _oracle(q, k, v, sel, cu, do)
    assert_within("o", o, ro)
    assert_within("dq", dq, rdq)
    assert_within("dk", dk, rdk)
    assert_within("dv", dv, rdv)
    rows_off = ~sel if sel.dim() == 1 else ~sel
    if sel.dim() == 1:
        assert torch.all(o[rows_off.to(gpu)] == 0) and torch.all(dq[rows_off.to(gpu)] == 0)


def test_cfg2_forward_per_head(gpu):
    """cfg2: bf16, T=8192, H=16, D=128, per-(head, token) Bernoulli(0.5), token 0 on."""
    n, hq, d = 8192, 16, 128
    g = gen(1)
    q, k, v = (randn((n, hq, d), g, 0.5) for _ in range(3))
    sel = torch.rand(n, hq, generator=g) < 0.5
    sel[0, :] = True
    cu = torch.tensor([0, n], dtype=torch.int32)
    print("cfg2 forward", flush=True)
    o, _ = _run(q, k, v, sel, cu, gpu)
    ro, _ = _oracle(q, k, v, sel, cu, dtype=np.float32)
    assert_within("o", o, ro)


def test_cfg3_varlen_fwd_bwd_full_size(gpu):
    """cfg3: packed varlen ~32K tokens, Markov selection ratio 0.25, dO ~ N(0,1)."""
    g = gen(2)
    lens = varlen_lengths(g)
    n = sum(lens)
    hq = h = 16
    d = 128
    sel = markov_selection(n, g)
    q, k, v = (randn((n, hq, d), g, 0.5) for _ in range(3))
    do = randn((n, hq, d), g)
    cu = cu_from_lengths(lens)
    print(f"cfg3 lens={lens} ratio={sel.float().mean():.3f}", flush=True)
    o, (dq, dk, dv) = _run(q, k, v, sel, cu, gpu, do)
    ro, (rdq, rdk, rdv) = torch_sq_attn(q.to(gpu), k.to(gpu), v.to(gpu), sel.to(gpu), cu,
                                        do=do.to(gpu))
    assert_within("o", o, ro)
    assert_within("dq", dq, rdq)
    assert_within("dk", dk, rdk)
    assert_within("dv", dv, rdv)


def test_empty_selection(gpu):
    n, hq, d = 300, 2, 128
    g = gen(5)
    q, k, v = (randn((n, hq, d), g) for _ in range(3))
    do = randn((n, hq, d), g)
    sel = torch.zeros(n, dtype=torch.bool)
    o, (dq, dk, dv) = _run(q, k, v, sel, torch.tensor([0, 100, 300], dtype=torch.int32), gpu, do)
    assert torch.all(o == 0) and torch.all(dq == 0) and torch.all(dk == 0) and torch.all(dv == 0)


def test_dense_paths_and_dense_ref(gpu):
    n, hq, d = 1100, 4, 128
    g = gen(6)
    q, k, v = (randn((n, hq, d), g) for _ in range(3))
    cu = torch.tensor([0, 100, 1100], dtype=torch.int32)
    ro, _ = _oracle(q, k, v, None, cu)
    o1 = sq_full_attn_dense_ref(q[None].to(gpu), k[None].to(gpu), v[None].to(gpu), cu_seqlens=cu.to(gpu))[0]
    o2 = dense_causal_attn(q[None].to(gpu), k[None].to(gpu), v[None].to(gpu), cu.to(gpu))[0]
    assert_within("dense_ref", o1, ro)
    assert_within("dense", o2, ro)


@pytest.mark.parametrize("window,d", [(128, 128), (16, 128), (0, 64), (1, 128), (33, 64), (64, 128), (100, 64),
                                      (127, 128), (200, 128)])
def test_swa_fwd_bwd_matches_oracle(gpu, window, d):
    """Sliding-window attention (keys [p - w, p]) against the oracle: windows
    up to 128 take the dedicated window forward (whole key window in LDS),
    200 the generic pipelined one; packed segments of 50, 1 and 849 rows
    (ragged last blocks, a segment shorter than the window).  Bound: the
    north-star max-abs 2e-2, scaled by max(1, max |ref|) (with one or two
    visible keys the probabilities are O(1) and dP = dO.v ~ N(0, D), so
    |dK| reaches 2-4, where one bf16 ulp is 1.6e-2), and mean-abs 2e-3."""
    n, hq, h = 900, 4, 2
    g = gen(7 + window + d)
    q, k, v = randn((n, hq, d), g), randn((n, h, d), g), randn((n, h, d), g)
    do = randn((n, hq, d), g)
    cu = torch.tensor([0, 50, 51, 900], dtype=torch.int32)
    print(f"swa window={window} d={d}", flush=True)
    qg, kg, vg = (x.to(gpu).requires_grad_() for x in (q, k, v))
    o = swa_attn(qg[None], kg[None], vg[None], cu.to(gpu), window=window)[0]
    o.backward(do.to(gpu))
    ro, (rdq, rdk, rdv) = _oracle(q, k, v, None, cu, do=do, window=window)
    for name, x, r in (("o", o, ro), ("dq", qg.grad, rdq), ("dk", kg.grad, rdk), ("dv", vg.grad, rdv)):
        assert_within(name, x, r, max_abs=2e-2 * max(1.0, float(np.abs(r).max())))


def test_noncontiguous_and_fp32_inputs(gpu):
    """fp32 inputs (cfg1's dtype), q a non-contiguous view: computed in fp32
    on the generic kernels, fp32 outputs and gradients, compared with the
    oracle fed the same fp32 inputs at the fp32 bound of
    tests/test_gpu_generic.py (max-abs 1e-3, mean-abs 1e-4)."""
    n, hq, d = 512, 4, 64
    g = gen(9)
    base = torch.randn(n, d, hq, generator=g)
    q = base.transpose(1, 2)  # non-contiguous view [n, hq, d]
    k = torch.randn(n, hq, d, generator=g)
    v = torch.randn(n, hq, d, generator=g)
    do = torch.randn(n, hq, d, generator=g)
    sel = torch.rand(n, generator=g) < 0.5
    cu = torch.tensor([0, n], dtype=torch.int32)
    o, (dq, dk, dv) = _run(q, k, v, sel, cu, gpu, do)
    assert o.dtype == dq.dtype == dk.dtype == dv.dtype == torch.float32
    ro, (rdq, rdk, rdv) = _oracle(q, k, v, sel, cu, do)
    for name, x, r in (("o", o, ro), ("dq", dq, rdq), ("dk", dk, rdk), ("dv", dv, rdv)):
        assert_within(name, x, r, max_abs=1e-3, mean_abs=1e-4)


@pytest.mark.parametrize("n,hq,h,d,cu,per_head", [
    (512, 4, 4, 64, [0, 512], False),
    (700, 4, 2, 128, [0, 1, 1, 200, 700], False),     # GQA, zero/single-token segments
    (600, 4, 4, 128, [0, 300, 600], True),            # per-head extension
    (900, 2, 1, 64, [0, 900], True),                  # per-head GQA
])
def test_fp16_inputs_run_in_fp16(gpu, n, hq, h, d, cu, per_head):
    """fp16 q, k, v run on the fp16 kernels (the reference's dots run in the
    input dtype, logo/ops/selected_full_attn.py:80 :95-99 :108): fp16 output
    and gradients against the oracle fed the same fp16 values, within max-abs
    4e-3 / mean-abs 4e-4 (fp16's 11-bit significand: 8x finer than bf16's,
    whose north-star bound is 2e-2 / 2e-3), and with a mean error below half
    of what the bf16 kernels give on the same inputs."""
    g = gen(300 + n + d)
    q, k, v = (randn((n, x, d), g, dtype=torch.float16) for x in (hq, h, h))
    do = randn((n, hq, d), g, dtype=torch.float16)
    sel = torch.rand((n, hq) if per_head else (n,), generator=g) < 0.5
    cu = torch.tensor(cu, dtype=torch.int32)
    print(f"fp16 n={n} hq={hq} h={h} d={d} per_head={per_head}", flush=True)
    o, grads = _run(q, k, v, sel, cu, gpu, do)
    assert o.dtype == torch.float16 and all(x.dtype == torch.float16 for x in grads)
    ro, rgrads = _oracle(q, k, v, sel, cu, do)
    ob, gb = _run(*(x.bfloat16() for x in (q, k, v)), sel, cu, gpu, do.bfloat16())
    for name, x, xb, r in zip(("o", "dq", "dk", "dv"), (o, *grads), (ob, *gb), (ro, *rgrads)):
        _, mean16 = assert_within(name, x, r, max_abs=4e-3, mean_abs=4e-4)
        _, mean_bf = err_stats(xb, r)
        assert mean16 < 0.5 * mean_bf, f"{name}: fp16 mean-abs {mean16:.2e} vs bf16 {mean_bf:.2e}"


def test_fp16_dense_and_window_paths_round_to_bf16(gpu):
    """The dense and sliding-window branches have bf16 kernels only: fp16
    inputs are rounded to bf16 and the outputs cast back to fp16, at the
    bf16 bound."""
    n, hq, d = 400, 2, 64
    g = gen(41)
    q, k, v = (randn((n, hq, d), g, dtype=torch.float16) for _ in range(3))
    cu = torch.tensor([0, 150, 400], dtype=torch.int32)
    for window in (16, None):
        qg, kg, vg = (x.to(gpu)[None] for x in (q, k, v))
        if window is None:
            o = dense_causal_attn(qg, kg, vg, cu.to(gpu))[0]
        else:
            o = swa_attn(qg, kg, vg, cu.to(gpu), window=window)[0]
        assert o.dtype == torch.float16
        ro, _ = _oracle(q, k, v, None, cu, window=window)
        assert_within(f"o window={window}", o, ro)


@pytest.mark.parametrize("K,V,hq,h", [(128, 64, 4, 2), (64, 128, 2, 2), (96, 96, 4, 4), (48, 32, 2, 1),
                                      (80, 112, 2, 2)])
def test_head_dims_off_the_compiled_set(gpu, K, V, hq, h):
    """K, V <= 128 other than K = V in {64, 128} (V != K included) run on the
    next compiled head dim with zero-padded q, k, v; outputs [.., V] and
    gradients match the oracle (default scale K**-0.5) at the north-star
    tolerance, and the unselected rows stay zero."""
    n = 600
    g = gen(70 + K + V)
    q, k, v = randn((n, hq, K), g), randn((n, h, K), g), randn((n, h, V), g)
    do = randn((n, hq, V), g)
    sel = torch.rand(n, generator=g) < 0.4
    cu = torch.tensor([0, 1, 250, 600], dtype=torch.int32)
    print(f"head dims K={K} V={V} hq={hq} h={h}", flush=True)
    o, (dq, dk, dv) = _run(q, k, v, sel, cu, gpu, do)
    assert o.shape == (n, hq, V) and dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
    ro, (rdq, rdk, rdv) = _oracle(q, k, v, sel, cu, do)
    assert_within("o", o, ro)
    assert_within("dq", dq, rdq)
    assert_within("dk", dk, rdk)
    assert_within("dv", dv, rdv)
    assert torch.all(o[~sel.to(gpu)] == 0)


def test_deterministic(gpu):
    n, hq, d = 2048, 4, 128
    g = gen(10)
    q, k, v = (randn((n, hq, d), g) for _ in range(3))
    do = randn((n, hq, d), g)
    sel = torch.rand(n, generator=g) < 0.3
    cu = torch.tensor([0, 1000, 2048], dtype=torch.int32)
    a = _run(q, k, v, sel, cu, gpu, do)
    b = _run(q, k, v, sel, cu, gpu, do)
    assert torch.equal(a[0], b[0])
    for x, y in zip(a[1], b[1]):
        assert torch.equal(x, y)


@pytest.mark.parametrize("per_head,hq,h,d", [(False, 4, 2, 128), (True, 4, 4, 128), (False, 2, 1, 64)])
def test_long_single_sequence_paired_forward(gpu, per_head, hq, h, d, monkeypatch):
    """A single sequence of >= 16K tokens takes the 8-wave two-tile forward
    workgroups; the same tokens as a pack with an extra empty segment take the
    4-wave one-tile workgroups.  Without the key-range split (which cuts the
    two kinds of tiles differently) every row visits the same 64-key tiles in
    the same order either way, so outputs and gradients are bit-identical;
    the shared-selection cases are also checked against the torch fp32
    reference (ragged last tile, GQA; head dims 128 and 64)."""
    monkeypatch.setenv("LOGO_SQ_SPLIT", "0")
    g = gen(16 + hq + int(per_head) + d)
    n = 16384 + 77
    sel = torch.rand((n, hq) if per_head else (n,), generator=g) < 0.3
    if per_head:
        sel[0, :] = True
    q, k, v = (randn((n, hq if i == 0 else h, d), g, 0.5) for i in range(3))
    do = randn((n, hq, d), g)
    one = torch.tensor([0, n], dtype=torch.int32)
    two = torch.tensor([0, n, n], dtype=torch.int32)
    o1, gr1 = _run(q, k, v, sel, one, gpu, do)
    o2, gr2 = _run(q, k, v, sel, two, gpu, do)
    assert torch.equal(o1, o2)
    for a, b in zip(gr1, gr2):
        assert torch.equal(a, b)
    if not per_head:
        ro, rgr = torch_sq_attn(q.to(gpu), k.to(gpu), v.to(gpu), sel.to(gpu), one, do=do.to(gpu))
        assert_within("o", o1, ro)
        for name, a, b in zip(("dq", "dk", "dv"), gr1, rgr):
            assert_within(name, a, b)


def test_long_single_sequence_paired_swa_forward(gpu):
    """Sliding-window attention over a single sequence of >= 16K tokens (the
    8-wave two-tile forward in dense mode with a window) equals, bit for bit,
    the same tokens packed with an extra empty segment (4-wave forward)."""
    n, hq, h, d = 16384 + 200, 4, 2, 128
    g = gen(31)
    q, k, v = randn((n, hq, d), g), randn((n, h, d), g), randn((n, h, d), g)
    do = randn((n, hq, d), g)
    outs = []
    for cu in (torch.tensor([0, n], dtype=torch.int32), torch.tensor([0, n, n], dtype=torch.int32)):
        qg, kg, vg = (x.to(gpu).requires_grad_() for x in (q, k, v))
        o = swa_attn(qg[None], kg[None], vg[None], cu.to(gpu), window=128)[0]
        o.backward(do.to(gpu))
        outs.append((o.detach(), qg.grad, kg.grad, vg.grad))
    for a, b in zip(*outs):
        assert torch.equal(a, b)
