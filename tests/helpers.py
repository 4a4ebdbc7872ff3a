"""Shared test inputs, tolerances and chunked torch fp32 references.

Inputs follow the benchmark configurations of BASELINE.json (seeded
``torch.Generator``).  ``torch_sq_attn`` and ``torch_decode_attn`` are
plain-PyTorch fp32 restatements of the same semantics as ``oracle.attn`` and
``oracle.decode``, used where the numpy oracle would be too slow (full-size
cases on the GPU); they are themselves pinned against the oracle on the CPU
(tests/test_oracle_attn.py, tests/test_oracle_decode.py).

Every comparison made through ``assert_within`` or ``record`` is kept in
``MARGINS`` (test, tensor, max-abs and mean-abs error, the bounds); with the
environment variable ``LOGO_PARITY_LOG`` set, tests/conftest.py writes them as
JSON lines to that file when the session ends (tests/parity_margins.py renders
the table).
"""

import os

import numpy as np
import torch

# BASELINE.json north_star tolerance for bf16 outputs and gradients against
# the fp32 reference path.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


MARGINS = []
CURRENT_TEST = {"id": None}


def record(name, max_err, mean_err, max_bound, mean_bound, kind="abs"):
    """Keep one comparison's errors and bounds for the parity-margin log."""
    MARGINS.append({"test": CURRENT_TEST["id"], "tensor": name, "kind": kind, "max": float(max_err),
                    "mean": float(mean_err), "max_bound": max_bound, "mean_bound": mean_bound})


def err_stats(x, ref):
    """max-abs and mean-abs of x - ref, in float64 on x's device (no host copy
    of full-size tensors)."""
    x = x.detach()
    ref = torch.as_tensor(ref)
    dev = x.device if x.is_cuda else ref.device
    d = (x.to(dev).double() - ref.to(dev).double()).abs()
    return d.max().item(), d.mean().item()


def assert_within(name, x, ref, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    mx, mn = err_stats(x, ref)
    record(name, mx, mn, max_abs, mean_abs)
    if os.environ.get("LOGO_PARITY_VERBOSE"):
        print(f"  {name}: max-abs {mx:.3e} mean-abs {mn:.3e}", flush=True)
    assert mx <= max_abs and mn <= mean_abs, f"{name}: max-abs {mx:.3e} (<= {max_abs}), mean-abs {mn:.3e} (<= {mean_abs})"
    return mx, mn


def gen(seed):
    g = torch.Generator()
    g.manual_seed(seed)
    return g


def randn(shape, g, scale=1.0, dtype=torch.bfloat16):
    return (torch.randn(*shape, generator=g) * scale).to(dtype)


def markov_selection(n, g, p10=1 / 8, p01=1 / 24):
    """Two-state Markov chain (mean run of 1s = 1/p10), stationary ratio
    p01 / (p01 + p10); initial state from the stationary distribution."""
    u = torch.rand(n, generator=g).numpy()
    ratio = p01 / (p01 + p10)
    out = np.empty(n, dtype=bool)
    state = u[0] < ratio
    out[0] = state
    for i in range(1, n):
        state = (u[i] >= p10) if state else (u[i] < p01)
        out[i] = state
    return torch.from_numpy(out)


def varlen_lengths(g, count=4, lo=2048, hi=16384, total_lo=30720, total_hi=34816):
    while True:
        lens = torch.randint(lo, hi + 1, (count,), generator=g)
        if total_lo <= int(lens.sum()) <= total_hi:
            return [int(x) for x in lens]


def cu_from_lengths(lens):
    cu = [0]
    for n in lens:
        cu.append(cu[-1] + n)
    return torch.tensor(cu, dtype=torch.int32)


def torch_sq_attn(q, k, v, sel_rows, cu, scale=None, window=None, do=None, row_chunk=2048):
    """fp32 reference on whatever device the tensors live on.

    q [N, HQ, D], k/v [N, H, D]; ``sel_rows`` bool [N] or [N, HQ]; returns
    ``o`` and, if ``do`` is given, ``(dq, dk, dv)`` (same formulas as
    oracle.attn.sq_attn_bwd with delta from the fp32 output).
    """
    N, HQ, D = q.shape
    H = k.shape[1]
    G = HQ // H
    if scale is None:
        scale = D ** -0.5
    dev = q.device
    qf, kf, vf = q.float(), k.float(), v.float()
    o = torch.zeros(N, HQ, v.shape[2], device=dev)
    grads = do is not None
    if grads:
        dof = do.float()
        dq = torch.zeros(N, HQ, D, device=dev)
        dk = torch.zeros(N, H, D, device=dev)
        dv = torch.zeros(N, H, v.shape[2], device=dev)
    sel = sel_rows.to(dev)
    cul = [int(x) for x in cu.tolist()]
    for s in range(len(cul) - 1):
        bos, eos = cul[s], cul[s + 1]
        if eos <= bos:
            continue
        keys = torch.arange(eos - bos, device=dev)
        for hq in range(HQ):
            h = hq // G
            m = sel[bos:eos] if sel.dim() == 1 else sel[bos:eos, hq]
            rows = torch.nonzero(m).flatten() + bos
            if rows.numel() == 0:
                continue
            K = kf[bos:eos, h]
            V = vf[bos:eos, h]
            for c0 in range(0, rows.numel(), row_chunk):
                r = rows[c0:c0 + row_chunk]
                pos = r - bos
                S = (qf[r, hq] @ K.T) * scale
                vis = keys[None, :] <= pos[:, None]
                if window is not None and window >= 0:
                    vis &= keys[None, :] >= pos[:, None] - window
                S = S.masked_fill(~vis, float("-inf"))
                P = torch.softmax(S, dim=1)
                orow = P @ V
                o[r, hq] = orow
                if grads:
                    dO = dof[r, hq]
                    delta = (orow * dO).sum(1, keepdim=True)
                    dS = P * (dO @ V.T - delta)
                    dq[r, hq] = scale * (dS @ K)
                    dk[bos:eos, h] += scale * (dS.T @ qf[r, hq])
                    dv[bos:eos, h] += P.T @ dO
    if grads:
        return o, (dq, dk, dv)
    return o


def torch_decode_attn(q, k, v, lens, active=None, scale=None):
    """fp32 decode attention on the tensors' device: ``q [B, HQ, D]``,
    ``k/v [B, H, T, D]`` (row b valid on ``[0, lens[b])``); inactive rows are
    zero (the semantics of oracle.decode.decode_attn)."""
    B, HQ, D = q.shape
    G = HQ // k.shape[1]
    if scale is None:
        scale = D ** -0.5
    out = torch.zeros(B, HQ, v.shape[3], dtype=torch.float32, device=q.device)
    for b in range(B):
        if active is not None and not bool(active[b]):
            continue
        n = int(lens[b])
        K = k[b, :, :n].float().repeat_interleave(G, 0).contiguous()  # [HQ, n, D]
        V = v[b, :, :n].float().repeat_interleave(G, 0).contiguous()
        s = torch.bmm(K, q[b].float()[:, :, None].contiguous())[..., 0] * scale
        p = torch.softmax(s, -1)
        out[b] = torch.bmm(p[:, None, :].contiguous(), V)[:, 0]
    return out
