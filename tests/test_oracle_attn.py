"""Pin the floating-point oracle (oracle.attn) on the CPU.

Checks chosen so that a dropped term, a wrong sign, an off-by-one in the
causal/window mask or a transposed operand fails at least one of them:
  * all-ones selection == torch scaled_dot_product_attention (is_causal) per
    segment (an independent implementation);
  * row 0 of each segment returns v_0 exactly; unselected rows are zero;
  * GQA equals the MHA oracle on repeat_kv'd keys/values;
  * lse == logsumexp(scale * s) / ln 2;
  * backward == torch autograd (float64) of a separately written masked
    softmax formulation, for sparse, windowed and GQA cases;
  * windowed attention with every segment <= window + 1 long equals full
    causal attention, and a brute-force loop matches the windowed oracle;
  * the torch fp32 test reference (tests/helpers.py) equals the oracle.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import attn
from tests.helpers import torch_sq_attn


def _inputs(n, hq, h, d, seed, dtype=np.float64):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((n, hq, d)).astype(dtype)
    k = rng.standard_normal((n, h, d)).astype(dtype)
    v = rng.standard_normal((n, h, d)).astype(dtype)
    return q, k, v


def _autograd_ref(q, k, v, sel, cu, do, scale, window=None):
    """Masked softmax attention written with torch ops, differentiated by autograd."""
    qt = torch.tensor(q, requires_grad=True)
    kt = torch.tensor(k, requires_grad=True)
    vt = torch.tensor(v, requires_grad=True)
    N, HQ, D = q.shape
    G = HQ // k.shape[1]
    kk = kt.repeat_interleave(G, dim=1)
    vv = vt.repeat_interleave(G, dim=1)
    seg = np.searchsorted(np.asarray(cu), np.arange(N), side="right") - 1
    seg_t = torch.tensor(seg)
    idx = torch.arange(N)
    same = seg_t[:, None] == seg_t[None, :]
    causal = idx[None, :] <= idx[:, None]
    mask = same & causal
    if window is not None:
        mask &= idx[None, :] >= idx[:, None] - window
    S = torch.einsum("qhd,khd->hqk", qt, kk) * scale
    S = S.masked_fill(~mask[None], float("-inf"))
    P = torch.softmax(S, dim=-1)
    o = torch.einsum("hqk,khd->qhd", P, vv)
    selm = torch.tensor(np.broadcast_to(sel.reshape(N, -1), (N, HQ)).copy())
    o = o * selm[:, :, None]
    o.backward(torch.tensor(do))
    return o.detach().numpy(), qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy()


@pytest.mark.parametrize("cu", [[0, 33], [0, 20, 20, 57, 64]])
def test_all_ones_equals_torch_sdpa(cu):
    q, k, v = _inputs(cu[-1], 2, 2, 16, 0)
    o, _ = attn.sq_attn_fwd(q, k, v, np.ones(cu[-1], bool), cu)
    for s in range(len(cu) - 1):
        b, e = cu[s], cu[s + 1]
        if e == b:
            continue
        ref = F.scaled_dot_product_attention(
            torch.tensor(q[b:e]).transpose(0, 1), torch.tensor(k[b:e]).transpose(0, 1),
            torch.tensor(v[b:e]).transpose(0, 1), is_causal=True).transpose(0, 1).numpy()
        np.testing.assert_allclose(o[b:e], ref, rtol=1e-10, atol=1e-12)


def test_row_zero_unselected_and_lse():
    cu = [0, 10, 25]
    q, k, v = _inputs(25, 3, 3, 8, 1)
    sel = np.zeros(25, bool)
    sel[[0, 3, 10, 11, 24]] = True
    o, lse = attn.sq_attn_fwd(q, k, v, sel, cu)
    np.testing.assert_allclose(o[0], v[0], rtol=0, atol=1e-14)
    np.testing.assert_allclose(o[10], v[10], rtol=0, atol=1e-14)
    assert np.all(o[~sel] == 0)
    assert np.all(np.isnan(lse[~sel]))
    scale = 8 ** -0.5
    t, hq = 24, 2
    s = (k[10:25, hq] @ q[t, hq]) * scale
    want = np.log(np.exp(s).sum()) / math.log(2.0)
    assert abs(lse[t, hq] - want) < 1e-12


def test_gqa_equals_repeat_kv():
    cu = [0, 19, 40]
    q, k, v = _inputs(40, 4, 2, 8, 2)
    sel = np.random.default_rng(2).random(40) < 0.6
    o, lse = attn.sq_attn_fwd(q, k, v, sel, cu)
    o2, lse2 = attn.sq_attn_fwd(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1), sel, cu)
    np.testing.assert_allclose(o, o2, rtol=0, atol=1e-14)
    np.testing.assert_allclose(lse[sel], lse2[sel], rtol=0, atol=1e-13)


@pytest.mark.parametrize("hq,h,window,per_head", [(2, 2, None, False), (4, 2, None, False),
                                                    (2, 1, 5, False), (3, 3, None, True)])
def test_backward_matches_autograd(hq, h, window, per_head):
    cu = [0, 13, 13, 30]
    q, k, v = _inputs(30, hq, h, 8, 3)
    rng = np.random.default_rng(4)
    sel = rng.random((30, hq) if per_head else 30) < 0.5
    do = rng.standard_normal((30, hq, 8))
    scale = 0.3
    o, _ = attn.sq_attn_fwd(q, k, v, sel, cu, scale=scale, window=window)
    dq, dk, dv = attn.sq_attn_bwd(q, k, v, o, do, sel, cu, scale=scale, window=window)
    ro, rdq, rdk, rdv = _autograd_ref(q, k, v, sel, cu, do, scale, window)
    np.testing.assert_allclose(o, ro, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dq, rdq, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, rdk, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dv, rdv, rtol=1e-9, atol=1e-11)


def test_window_reduces_to_causal_and_brute_force():
    cu = [0, 6, 15]
    q, k, v = _inputs(15, 2, 2, 4, 5)
    full, _ = attn.sq_attn_fwd(q, k, v, None, cu)
    win, _ = attn.swa_fwd(q, k, v, cu, window=9)
    np.testing.assert_allclose(win, full, rtol=0, atol=1e-14)
    w = 3
    win, _ = attn.swa_fwd(q, k, v, cu, window=w, scale=0.5)
    for s in range(2):
        b, e = cu[s], cu[s + 1]
        for t in range(b, e):
            for hq in range(2):
                js = list(range(max(b, t - w), t + 1))
                sc = np.array([q[t, hq] @ k[j, hq] * 0.5 for j in js])
                p = np.exp(sc - sc.max())
                p /= p.sum()
                want = sum(pi * v[j, hq] for pi, j in zip(p, js))
                np.testing.assert_allclose(win[t, hq], want, rtol=1e-12, atol=1e-13)


def test_mask_off_by_one_would_be_caught():
    """Planting `key < pos` instead of `key <= pos` must break the row-0 check."""
    cu = [0, 8]
    q, k, v = _inputs(8, 1, 1, 4, 6)
    pos = np.arange(8)
    keys = np.arange(8)
    wrong = keys[None, :] < pos[:, None]
    assert not wrong[0].any()  # row 0 would see no key at all -> NaN, not v_0
    o, _ = attn.sq_attn_fwd(q, k, v, None, cu)
    np.testing.assert_allclose(o[0], v[0], atol=1e-14)


@pytest.mark.parametrize("window", [None, 4])
def test_torch_reference_matches_oracle(window):
    cu = torch.tensor([0, 21, 21, 50], dtype=torch.int32)
    q, k, v = _inputs(50, 4, 2, 16, 7, dtype=np.float32)
    rng = np.random.default_rng(8)
    sel = rng.random((50, 4)) < 0.5
    do = rng.standard_normal((50, 4, 16)).astype(np.float32)
    o_ref, (dq_r, dk_r, dv_r) = torch_sq_attn(torch.tensor(q), torch.tensor(k), torch.tensor(v),
                                             torch.tensor(sel), cu, window=window, do=torch.tensor(do))
    o, _ = attn.sq_attn_fwd(q, k, v, sel, cu.numpy(), window=window)
    dq, dk, dv = attn.sq_attn_bwd(q, k, v, o, do, sel, cu.numpy(), window=window)
    np.testing.assert_allclose(o_ref.numpy(), o, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dq_r.numpy(), dq, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dk_r.numpy(), dk, rtol=1e-4, atol=1e-5)
    np.testing.assert_allclose(dv_r.numpy(), dv, rtol=1e-4, atol=1e-5)


def test_flops_formula_closed_form():
    # single sequence, all rows: sum(p+1) = T(T+1)/2
    T, H, D = 100, 3, 8
    f = attn.sq_flops_fwd(np.ones(T, bool), [0, T], H, D)
    assert f == 4 * D * H * T * (T + 1) // 2


def test_flops_formula_per_head_and_segments_brute_force():
    """Per-head selection [N, HQ] over packed segments: each head counts its
    own rows' visible keys (position within the segment + 1), by brute force
    over every (row, key) pair; a shared [N] mask is every head counting the
    same rows."""
    rng = np.random.default_rng(9)
    cu = [0, 13, 13, 40, 61]
    N, HQ, D = 61, 3, 16
    sel = rng.random((N, HQ)) < 0.4
    want = 0
    for s in range(len(cu) - 1):
        for hq in range(HQ):
            for t in range(cu[s], cu[s + 1]):
                if sel[t, hq]:
                    want += sum(1 for key in range(cu[s], cu[s + 1]) if key <= t)
    assert attn.sq_flops_fwd(sel, cu, HQ, D) == 4 * D * want
    shared = sel[:, 0]
    want1 = sum(t - cu[s] + 1 for s in range(len(cu) - 1) for t in range(cu[s], cu[s + 1]) if shared[t])
    assert attn.sq_flops_fwd(shared, cu, HQ, D) == 4 * D * HQ * want1


@pytest.mark.parametrize("K,V", [(8, 5), (6, 12)])
def test_value_dim_differs_from_key_dim(K, V):
    """V != K (the reference's V is its own constexpr, selected_full_attn.py:341):
    forward and backward against the autograd reference, default scale K**-0.5."""
    cu = [0, 11, 27]
    rng = np.random.default_rng(40 + K)
    q = rng.standard_normal((27, 4, K))
    k = rng.standard_normal((27, 2, K))
    v = rng.standard_normal((27, 2, V))
    do = rng.standard_normal((27, 4, V))
    sel = rng.random(27) < 0.6
    o, _ = attn.sq_attn_fwd(q, k, v, sel, cu)
    assert o.shape == (27, 4, V)
    dq, dk, dv = attn.sq_attn_bwd(q, k, v, o, do, sel, cu)
    ro, rdq, rdk, rdv = _autograd_ref(q, k, v, sel, cu, do, K ** -0.5)
    np.testing.assert_allclose(o, ro, rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dq, rdq, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dk, rdk, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dv, rdv, rtol=1e-9, atol=1e-11)
