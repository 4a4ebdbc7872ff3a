"""Parity on the benchmark's own workload, at full size, and in the
large-logit regime.

* The headline input exactly as bench.py builds it (``bench.headline_inputs``:
  T=32768, HQ=H=16, D=128, one sequence, Markov selection at r=0.25, seed 2)
  through ``sq_full_attn`` forward and backward, as the benchmark calls it.
  o, dq, dk and dv are compared with the fp32 torch reference
  ``tests.helpers.torch_sq_attn`` (pinned against the float64 oracle on the
  CPU in tests/test_oracle_attn.py) at the north-star bound, max-abs 2e-2 and
  mean-abs 2e-3.  At r=0.25 neither the forward nor dq splits its key ranges
  (too many tiles per head); the same generator at r=0.125 gives few enough
  tiles that both split, so that case checks the split path against the
  reference at full size.
* A single sequence of 262,144 tokens with GQA: long row searches, many
  key tiles per row and split key ranges at 8x the headline's length.
* Large logits: a few q / k feature dims of magnitude ~9, so that the scaled
  scores span about +-45 in log2 units and attention is peaked.  The sparse
  kernels round the pre-scaled query ``-scale * log2(e) * q`` to bf16 before
  QK^T (the reference scales the fp32 product instead,
  logo/ops/selected_full_attn.py:93); this case measures what that rounding
  costs where it matters most, against the float64 oracle.  Gradients there
  reach ~10 in magnitude, so errors are scaled by max(1, |ref|).  In this
  regime the reference's own rounding chain (fp32 scores, bf16 P and dS
  operands, fp32 accumulation), run on the same inputs, is itself ~5e-2 from
  float64 in dq's scaled max, above the 2e-2 bound.  So each result must be
  within the north-star bound or within CHAIN_FACTOR times the reference
  chain's own error, whichever is larger.  That factor is the slack the bf16
  query pre-rounding (and the other differences in rounding order) may use.
  Measured on MI355X: dq 4.98e-2 against the chain's 4.97e-2, dk 2.2e-2
  against 1.75e-2; means 1.2-1.5x the chain's and 10x below 2e-3.
"""

import numpy as np
import pytest
import torch

from bench import headline_inputs
from logo_amd.ops import sq_full_attn
from oracle import attn
from tests.helpers import MAX_ABS, MEAN_ABS, assert_within, record, torch_sq_attn

pytestmark = pytest.mark.gpu

KBQ = 128  # compacted query rows per forward / dq tile
CHAIN_FACTOR = 1.5  # allowed error relative to the reference rounding chain's own


def _split_pieces(nt, cap):
    """Pieces per tile of a head with nt tiles (the library's split rule)."""
    if cap <= 0 or nt <= 0 or 4 * nt > 3 * cap:
        return 1
    return min(-(-cap // nt), 4)


@pytest.mark.parametrize("ratio,splits", [(0.25, False), (0.125, True)])
def test_headline_workload_full_size(gpu, ratio, splits):
    T, H, D, seed = 32768, 16, 128, 2
    q, k, v, do, sel_np = headline_inputs(T, H, D, ratio, seed)
    rows = int(sel_np.sum())
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    nt = -(-rows // KBQ)
    fwd_pieces = _split_pieces(-(-nt // 2), 2 * cus * 1 // H)  # paired 8-wave tiles, 1 workgroup per CU
    dq_pieces = _split_pieces(nt, 2 * cus * 2 // H)
    print(f"headline T={T} H={H} D={D} r={ratio} seed={seed}: {rows} rows, fwd pieces {fwd_pieces}, "
          f"dq pieces {dq_pieces}", flush=True)
    assert (fwd_pieces > 1 and dq_pieces > 1) == splits

    qg, kg, vg = (x.to(gpu)[None].requires_grad_() for x in (q, k, v))
    dog = do.to(gpu)[None]
    selg = torch.from_numpy(sel_np).to(gpu)[None]
    cu = torch.tensor([0, T], dtype=torch.int32, device=gpu)
    o = sq_full_attn(qg, kg, vg, selg, cu_seqlens=cu)
    dq, dk, dv = torch.autograd.grad(o, (qg, kg, vg), dog)
    torch.cuda.synchronize()

    ro, (rdq, rdk, rdv) = torch_sq_attn(q.to(gpu), k.to(gpu), v.to(gpu), selg[0], cu.cpu(), do=do.to(gpu))
    tag = f"r={ratio}"
    assert_within(f"o {tag}", o[0], ro)
    assert_within(f"dq {tag}", dq[0], rdq)
    assert_within(f"dk {tag}", dk[0], rdk)
    assert_within(f"dv {tag}", dv[0], rdv)
    # unselected rows are exactly zero
    unsel = ~selg[0]
    assert int(o[0][unsel].count_nonzero()) == 0 and int(dq[0][unsel].count_nonzero()) == 0


def _bf(x):
    return torch.as_tensor(x).to(torch.bfloat16).double()


def _reference_chain(q, k, v, do, sel, scale):
    """The reference kernels' rounding chain on one sequence (float64 host
    arithmetic with its rounding points): scores from the exact product
    rounded to fp32 then scaled, P = exp2(s - lse) rounded to bf16 for PV,
    dS rounded to bf16 for dq and dk, P to bf16 for dv
    (logo/ops/selected_full_attn.py:93-99, :206-207, :220-221, :300-330)."""
    N, HQ, D = q.shape
    qd, kd, vd, dod = (torch.as_tensor(x).double() for x in (q, k, v, do))
    c = scale / np.log(2.0)
    o = torch.zeros(N, HQ, vd.shape[2], dtype=torch.float64)
    dq = torch.zeros_like(qd)
    dk = torch.zeros_like(kd)
    dv = torch.zeros_like(vd)
    keys = torch.arange(N)
    for hq in range(HQ):
        h = hq * kd.shape[1] // HQ
        rows = torch.nonzero(torch.as_tensor(sel)).flatten()
        Q, K, V, dO = qd[rows, hq], kd[:, h], vd[:, h], dod[rows, hq]
        s = (Q @ K.T).float().double() * c
        s = s.masked_fill(keys[None, :] > rows[:, None], float("-inf"))
        m = s.max(1, keepdim=True).values
        p = torch.exp2(s - m)
        lse = m + torch.log2(p.sum(1, keepdim=True))
        p = torch.exp2(s - lse)
        orow = (_bf(p) @ V).float().double()
        o[rows, hq] = orow
        delta = (_bf(orow) * dO).sum(1, keepdim=True)
        ds = p * ((dO @ V.T).float().double() - delta)
        dq[rows, hq] = scale * (_bf(ds) @ K)
        dk[:, h] += scale * (_bf(ds).T @ Q)
        dv[:, h] += _bf(p).T @ dO
    return o, dq, dk, dv


def test_large_logits_against_oracle(gpu):
    n, hq, h, d = 2048, 4, 2, 128
    g = torch.Generator()
    g.manual_seed(77)
    q = torch.randn(n, hq, d, generator=g) * 0.5
    k = torch.randn(n, h, d, generator=g) * 0.5
    q[..., :4] = 9.0 * torch.sign(torch.randn(n, hq, 4, generator=g))
    k[..., :4] = 9.0 * torch.sign(torch.randn(n, h, 4, generator=g))
    q, k = q.bfloat16(), k.bfloat16()
    v = torch.randn(n, h, d, generator=g).bfloat16()
    do = torch.randn(n, hq, d, generator=g).bfloat16()
    sel = torch.rand(n, generator=g) < 0.5
    sel[0] = True
    scale = d ** -0.5
    logits = (q[:, 0].double() @ k[:, 0].double().T) * scale / np.log(2.0)
    span = float(logits.tril().abs().max())
    print(f"large logits: n={n} hq={hq} h={h} d={d}, |scaled score| up to {span:.1f} (log2 units)", flush=True)
    assert 30.0 <= span <= 70.0

    cu = torch.tensor([0, n], dtype=torch.int32)
    qg, kg, vg = (x.to(gpu)[None].requires_grad_() for x in (q, k, v))
    o = sq_full_attn(qg, kg, vg, sel.to(gpu)[None], cu_seqlens=cu.to(gpu))
    dq, dk, dv = torch.autograd.grad(o, (qg, kg, vg), do.to(gpu)[None])

    qn, kn, vn, don = (x.float().numpy() for x in (q, k, v, do))
    ro, _ = attn.sq_attn_fwd(qn, kn, vn, sel.numpy(), cu.numpy(), scale=scale)
    rdq, rdk, rdv = attn.sq_attn_bwd(qn, kn, vn, ro, don, sel.numpy(), cu.numpy(), scale=scale)
    co, cdq, cdk, cdv = _reference_chain(qn, kn, vn, don, sel.numpy(), scale)
    failures = []
    for name, got, ref, chain in (("o", o[0], ro, co), ("dq", dq[0], rdq, cdq), ("dk", dk[0], rdk, cdk),
                                  ("dv", dv[0], rdv, cdv)):
        ref = torch.as_tensor(ref).double()
        err = (got.detach().double().cpu() - ref).abs()
        scaled = (err / ref.abs().clamp_min(1.0)).max().item()
        cerr = (chain - ref).abs()
        cscaled = (cerr / ref.abs().clamp_min(1.0)).max().item()
        print(f"  {name}: scaled max {scaled:.3e} mean {err.mean().item():.3e} | reference chain: scaled max "
              f"{cscaled:.3e} mean {cerr.mean().item():.3e}", flush=True)
        max_bound = max(MAX_ABS, CHAIN_FACTOR * cscaled)
        mean_bound = max(MEAN_ABS, CHAIN_FACTOR * cerr.mean().item())
        record(f"{name} large logits", scaled, err.mean().item(), max_bound, mean_bound,
               kind="max scaled by max(1, |ref|)")
        record(f"{name} large logits, reference rounding chain", cscaled, cerr.mean().item(), None, None,
               kind="max scaled by max(1, |ref|)")
        if scaled > max_bound or err.mean().item() > mean_bound:
            failures.append(f"{name}: scaled max {scaled:.3e} (<= {max_bound:.3e}), mean {err.mean().item():.3e} "
                            f"(<= {mean_bound:.3e})")
    assert not failures, "; ".join(failures)


def test_long_sequence_256k_tokens(gpu):
    """One sequence of 262,144 tokens (8x the headline), GQA (HQ=4, H=2),
    D=128, Markov selection at r=0.03: rows that see up to 4096 key tiles,
    lower-bound searches over ~8K rows per lane, a forward and dq with few
    tiles per head (so both split their key ranges).  o, dq, dk and dv against the fp32 torch reference at the
    north-star bound."""
    from bench import markov_mask

    T, hq, h, d = 262144, 4, 2, 128
    g = torch.Generator()
    g.manual_seed(11)
    sel_np = markov_mask(T, 0.03, 8, g)
    sel_np[0] = True
    q = (torch.randn(T, hq, d, generator=g) * 0.5).to(torch.bfloat16)
    k = (torch.randn(T, h, d, generator=g) * 0.5).to(torch.bfloat16)
    v = (torch.randn(T, h, d, generator=g) * 0.5).to(torch.bfloat16)
    do = torch.randn(T, hq, d, generator=g).to(torch.bfloat16)
    print(f"long sequence T={T} hq={hq} h={h} d={d}: {int(sel_np.sum())} rows", flush=True)
    qg, kg, vg = (x.to(gpu)[None].requires_grad_() for x in (q, k, v))
    selg = torch.from_numpy(sel_np).to(gpu)[None]
    cu = torch.tensor([0, T], dtype=torch.int32, device=gpu)
    o = sq_full_attn(qg, kg, vg, selg, cu_seqlens=cu)
    dq, dk, dv = torch.autograd.grad(o, (qg, kg, vg), do.to(gpu)[None])
    torch.cuda.synchronize()
    ro, (rdq, rdk, rdv) = torch_sq_attn(q.to(gpu), k.to(gpu), v.to(gpu), selg[0], cu.cpu(), do=do.to(gpu),
                                        row_chunk=1024)
    assert_within("o T=256K", o[0], ro)
    assert_within("dq T=256K", dq[0], rdq)
    assert_within("dk T=256K", dk[0], rdk)
    assert_within("dv T=256K", dv[0], rdv)
    unsel = ~selg[0]
    assert int(o[0][unsel].count_nonzero()) == 0 and int(dq[0][unsel].count_nonzero()) == 0
