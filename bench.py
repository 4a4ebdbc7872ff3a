#!/usr/bin/env python3
"""Benchmark of the LoGo query-sparse attention hot path on one MI355X.

Metric: ``sq_full_attn`` forward+backward effective TFLOP/s at
T=32768, H=16, D=128 with a 25% global ratio.  A step is one user-level call
``o = sq_full_attn(q, k, v, selection, cu_seqlens=cu)`` plus its backward
(compaction, forward, delta, dq, dk/dv), on synthetic inputs already resident
in HBM.  Effective FLOPs count selected rows only:
``F = 3.5 * 4 * D * HQ * sum over selected rows of (p + 1)``.

Prints ONE JSON line.  Per-kernel durations come from HIP events recorded on
the launch stream around every operator call that launches the kernel inside
the timed region (the operator's output allocation included; the forward and
dq kernels write the zero rows of unselected tokens themselves); the
dominant kernel's roofline is its algorithmic FLOPs over that duration.  The
CPU baseline times the reference's CPU formulation (dense causal attention per
segment, then row masking, torch fp32 autograd) on a bounded sample of heads.
"""

import argparse
import json
import os
import sys
import time

import numpy as np
import torch

MFMA_BF16_PEAK_TFLOPS = 2516.6  # dense bf16 MFMA, 256 CU x 2.4 GHz x 4096 FLOP/clk
HBM_PEAK_GBS = 8000.0

# Matmul FLOPs per visible (query, key) pair and head dim, per kernel: the
# forward does QK^T and PV; dq recomputes S and dP and forms dQ; dk/dv
# recompute S and dP and form dV and dK.
KERNEL_FLOPS_PER_PAIR_D = {
    "logo_sq_fwd": 4,
    "logo_sq_bwd_dq": 6,
    "logo_sq_bwd_dkv": 8,
}


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles", "traffic.json")


def measured_traffic(kernel, T, H, D, ratio, seed):
    """HBM bytes per launch of ``kernel`` from the committed rocprofv3 counter
    runs (FETCH_SIZE and WRITE_SIZE in KiB per dispatch, each scaled by what the
    same counter reads for a 1 GiB copy), or None when this workload has not
    been profiled."""
    try:
        with open(TRAFFIC_FILE) as f:
            rec = json.load(f)
    except (OSError, ValueError):
        return None
    wl = f"T{T}_H{H}_D{D}_r{ratio}_seed{seed}"
    ent = rec.get("kernels", {}).get(kernel)
    if rec.get("workload") != wl or ent is None:
        return None
    return ent["bytes_per_launch"]


def parse():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--seq-len", type=int, default=32768)
    ap.add_argument("--heads", type=int, default=16)
    ap.add_argument("--head-dim", type=int, default=128)
    ap.add_argument("--ratio", type=float, default=0.25)
    ap.add_argument("--cpu-heads", type=int, default=8, help="heads in the CPU-baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--seed", type=int, default=2)
    ap.add_argument("--no-extra", action="store_true", help="skip the secondary measurements")
    ap.add_argument("--no-decode", action="store_true", help="skip the config-5 model decode measurement")
    ap.add_argument("--decode-layer", action="store_true",
                    help="run only the config-5 global decode branch of one layer (the kernel the "
                         "decode HBM-traffic profile measures) and print its time and bandwidth")
    ap.add_argument("--decode-model", action="store_true",
                    help="run only the config-5 model decode measurement (prefill, then captured decode "
                         "steps) and print its result")
    ap.add_argument("--layer", action="store_true",
                    help="run only the config-4 LoGoAttention layer forward + backward measurement and "
                         "print its result")
    ap.add_argument("--swa", action="store_true",
                    help="run only the config-4 sliding-window (local branch) forward and "
                         "forward + backward measurement and print its result")
    ap.add_argument("--generic", action="store_true",
                    help="run only the generic-kernel measurement (head dim 256 in bf16, fp32 at D=128, "
                         "config 1 in fp32) and print its result")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run one 1 GiB device-to-device copy before the workload (the reference kernel "
                         "for scaling rocprofv3 FETCH_SIZE / WRITE_SIZE counters to bytes)")
    return ap.parse_args()


def markov_mask(n, ratio, mean_run, gen):
    """Selection correlated in spans: two-state Markov chain with mean run of
    ones `mean_run` and stationary ratio `ratio` (initial state stationary)."""
    p10 = 1.0 / mean_run
    p01 = ratio * p10 / (1.0 - ratio)
    u = torch.rand(n, generator=gen).numpy()
    out = np.empty(n, dtype=bool)
    state = u[0] < ratio
    out[0] = state
    for i in range(1, n):
        state = (u[i] >= p10) if state else (u[i] < p01)
        out[i] = state
    return out


def headline_inputs(T, H, D, ratio, seed):
    """The timed step's synthetic input on the host: the selection (Markov
    spans, mean run 8, token 0 selected), then q, k, v ~ N(0, 1) * 0.5 and
    dO ~ N(0, 1) in bf16, [T, H, D], all from one generator seeded ``seed``."""
    gen = torch.Generator()
    gen.manual_seed(seed)
    sel_np = markov_mask(T, ratio, 8, gen)
    sel_np[0] = True
    q = (torch.randn(T, H, D, generator=gen) * 0.5).to(torch.bfloat16)
    k = (torch.randn(T, H, D, generator=gen) * 0.5).to(torch.bfloat16)
    v = (torch.randn(T, H, D, generator=gen) * 0.5).to(torch.bfloat16)
    do = torch.randn(T, H, D, generator=gen).to(torch.bfloat16)
    return q, k, v, do, sel_np


class EventTimer:
    """Launch hook: HIP events on the current stream around each operator call
    that launches a kernel (its output allocation and fills included)."""

    def __init__(self):
        self.pending = {}
        self.pairs = {}
        self.enabled = False

    def __call__(self, name, phase):
        if not self.enabled:
            return
        ev = torch.cuda.Event(enable_timing=True)
        ev.record(torch.cuda.current_stream())
        if phase == "start":
            self.pending[name] = ev
        else:
            self.pairs.setdefault(name, []).append((self.pending.pop(name), ev))

    def averages_ms(self):
        return {k: float(np.mean([a.elapsed_time(b) for a, b in v])) for k, v in self.pairs.items()}

    def counts(self):
        return {k: len(v) for k, v in self.pairs.items()}


def cpu_baseline(q, k, v, sel_np, cu, do, heads, flops_per_head):
    from oracle.cpu_path import time_fwd_bwd

    # every core the process may run on, within the host's CPU share for this
    # GPU when the environment states it (OMP_NUM_THREADS; 16 on the GPU boxes)
    threads = len(os.sched_getaffinity(0))
    share = os.environ.get("OMP_NUM_THREADS", "")
    if share.isdigit() and int(share) > 0:
        threads = min(threads, int(share))
    qs = q[:, :heads].float().cpu()
    ks = k[:, :heads].float().cpu()
    vs = v[:, :heads].float().cpu()
    ds = do[:, :heads].float().cpu()
    sel = torch.from_numpy(sel_np)
    secs = time_fwd_bwd(qs, ks, vs, sel, cu, ds, threads)
    return {
        "value": round(flops_per_head * heads / secs / 1e12, 4),
        "unit": "TFLOP/s",
        "cores": threads,
        "kind": "port",
        "sample": (f"reference CPU formulation (logo/ops/dense_full_attn.py:30-69 dense causal SDPA per "
                   f"segment, then selection mask) in torch fp32 autograd fwd+bwd on {heads} of "
                   f"{q.shape[1]} heads of the same T={q.shape[0]} workload; {secs:.2f} s; effective "
                   f"FLOPs on selected rows as for the GPU value; {threads} threads = the process's CPU "
                   f"affinity capped by OMP_NUM_THREADS"),
    }


def _time_ms(fn, iters, warmup=5):
    """Average GPU time of back-to-back calls: the start event is queued
    behind the warm-up calls (no synchronisation in between), so the first
    timed call's host-side launch latency is not counted as GPU time.  Five
    warm-up calls: the first calls on new shapes (allocator growth, first
    launches) ran slower for several calls (cfg3: 1.59 ms, then 1.49 ms)."""
    torch.cuda.synchronize()
    for _ in range(warmup):
        fn()
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        fn()
    b.record()
    torch.cuda.synchronize()
    return a.elapsed_time(b) / iters


def swa_cfg4_measurement(q, k, v, do, iters=10):
    """The local branch at the cfg4 shape: sliding window 128 over
    [1, 4 x 8192, 16, 128] (four packed sequences), forward alone and
    forward + backward through swa_attn.  Bandwidths are algorithmic bytes:
    forward q, k, v read and o written; backward q, k, v, o, dO read and dq,
    dk, dv written (bf16), over the backward's share of the time; beside
    them, the rate of a plain device-to-device copy of the forward's bytes
    (``copy_gbs``, half read and half written)."""
    from logo_amd.ops import swa_attn
    N4, H, D = 4 * 8192, q.shape[2], q.shape[3]
    dev = q.device
    cu4 = torch.arange(0, N4 + 1, 8192, dtype=torch.int32, device=dev)
    q4, k4, v4 = (x[:, :N4].detach().requires_grad_() for x in (q, k, v))
    with torch.no_grad():
        tsf = _time_ms(lambda: swa_attn(q4, k4, v4, cu4, window=128), iters)

    def swa_fb():
        o = swa_attn(q4, k4, v4, cu4, window=128)
        torch.autograd.grad(o, (q4, k4, v4), do[:, :N4])
    tsb = _time_ms(swa_fb, max(iters // 2, 1))
    io = 4 * N4 * H * D * 2
    # a device-to-device copy of the forward's bytes (half read, half written),
    # the read + write rate the part delivers in practice
    src = torch.empty(io // 4, dtype=torch.bfloat16, device=dev)
    dst = torch.empty_like(src)
    tcp = _time_ms(lambda: dst.copy_(src), iters)
    copy_gbs = io / tcp / 1e6
    del src, dst
    return {"fwd_ms": round(tsf, 4), "fwd_gbs": round(io / tsf / 1e6, 1), "fwd_bwd_ms": round(tsb, 4),
            "bwd_ms": round(tsb - tsf, 4), "bwd_gbs": round(2 * io / (tsb - tsf) / 1e6, 1),
            "copy_gbs": round(copy_gbs, 1), "fwd_of_copy": round(io / tsf / 1e6 / copy_gbs, 3),
            "bwd_of_copy": round(2 * io / (tsb - tsf) / 1e6 / copy_gbs, 3)}


def generic_measurement(dev, gen):
    """The generic kernels (head dim 256; fp32 inputs) on the query-sparse
    path: fwd+bwd effective TFLOP/s (selected rows only, as the headline) at
    T=8192, H=16, Markov r=0.25, for K=V=256 in bf16 and for D=128 in fp32
    (against the fp32 MFMA peak), and config 1 (B=1, H=4, T=512, D=64, fp32,
    Bernoulli 0.5) in ms."""
    from logo_amd.ops import sq_full_attn
    out = {}
    T, H = 8192, 16
    sel_np = markov_mask(T, 0.25, 8, gen)
    sel_np[0] = True
    pairs = float((np.flatnonzero(sel_np) + 1).sum()) * H
    sel = torch.from_numpy(sel_np).to(dev)[None]
    cu = torch.tensor([0, T], dtype=torch.int32, device=dev)
    for name, D, dt in (("d256_bf16", 256, torch.bfloat16), ("d128_fp32", 128, torch.float32)):
        q, k, v = ((torch.randn(1, T, H, D, generator=gen) * 0.5).to(dt).to(dev).requires_grad_() for _ in range(3))
        do = torch.randn(1, T, H, D, generator=gen).to(dt).to(dev)

        def fb():
            o = sq_full_attn(q, k, v, sel, cu_seqlens=cu)
            torch.autograd.grad(o, (q, k, v), do)
        t = _time_ms(fb, 5)
        out[f"{name}_T8192_r0.25_fwd_bwd"] = {"ms": round(t, 3), "tflops": round(3.5 * 4 * D * pairs / t / 1e9, 1)}
        del q, k, v, do
    n1, h1, d1 = 512, 4, 64
    q, k, v = (torch.randn(1, n1, h1, d1, generator=gen).to(dev).requires_grad_() for _ in range(3))
    do = torch.randn(1, n1, h1, d1, generator=gen).to(dev)
    sel1 = (torch.rand(1, n1, generator=gen) < 0.5).to(dev)
    cu1 = torch.tensor([0, n1], dtype=torch.int32, device=dev)

    def fb1():
        o = sq_full_attn(q, k, v, sel1, cu_seqlens=cu1)
        torch.autograd.grad(o, (q, k, v), do)
    out["cfg1_fp32_fwd_bwd_ms"] = round(_time_ms(fb1, 20), 4)
    return out


def extra_measurements(dev):
    """Secondary rows: speed-up vs global ratio, cfg2 forward, cfg3 varlen
    fwd+bwd, SWA and epilogue at cfg4 shapes, gate-aware decode at cfg5 shape.
    All timings are HIP events around the op on the current stream."""
    from logo_amd.ops import dense_causal_attn, sq_full_attn, swa_attn
    from logo_amd.ops.decode import decode_attn
    from logo_amd.ops.epilogue import logo_epilogue

    out = {}
    gen = torch.Generator()
    gen.manual_seed(7)
    T, H, D = 32768, 16, 128
    q = (torch.randn(1, T, H, D, generator=gen) * 0.5).bfloat16().to(dev).requires_grad_()
    k = (torch.randn(1, T, H, D, generator=gen) * 0.5).bfloat16().to(dev).requires_grad_()
    v = (torch.randn(1, T, H, D, generator=gen) * 0.5).bfloat16().to(dev).requires_grad_()
    do = torch.randn(1, T, H, D, generator=gen).bfloat16().to(dev)
    cu = torch.tensor([0, T], dtype=torch.int32, device=dev)

    # speed-up of the sparse path over dense causal attention vs the global ratio
    def fb_dense():
        o = dense_causal_attn(q, k, v, cu)
        torch.autograd.grad(o, (q, k, v), do)
    t_dense = _time_ms(fb_dense, 5)
    sweep = {"dense_ms": round(t_dense, 3)}
    for r in (0.5, 0.25, 0.125):
        sel = torch.from_numpy(markov_mask(T, r, 8, gen)).to(dev)[None]

        def fb_sparse():
            o = sq_full_attn(q, k, v, sel, cu_seqlens=cu)
            torch.autograd.grad(o, (q, k, v), do)
        t = _time_ms(fb_sparse, 10)
        sweep[f"r{r}"] = {"ms": round(t, 3), "speedup": round(t_dense / t, 2), "ideal": round(1 / r, 2)}
    out["fwd_bwd_speedup_vs_dense_T32768"] = sweep

    # cfg2: forward only, T=8192, per-(head, token) Bernoulli(0.5)
    T2 = 8192
    q2, k2, v2 = (x[:, :T2].detach() for x in (q, k, v))
    sel2 = torch.rand(1, T2, H, generator=gen) < 0.5
    sel2[:, 0, :] = True
    pairs = float(sum((np.flatnonzero(sel2[0, :, h].numpy()) + 1).sum() for h in range(H)))
    sel2 = sel2.to(dev)
    cu2 = torch.tensor([0, T2], dtype=torch.int32, device=dev)
    with torch.no_grad():
        t2 = _time_ms(lambda: sq_full_attn(q2, k2, v2, sel2, cu_seqlens=cu2), 10)
    out["cfg2_fwd_T8192_per_head_r0.5"] = {"ms": round(t2, 4), "tflops": round(4 * D * pairs / t2 / 1e9, 1)}

    # cfg3: varlen fwd+bwd, ~32K tokens in 4 sequences, Markov ratio 0.25
    lens = [7210, 12503, 2789, 9871]
    cu3 = torch.tensor(np.concatenate([[0], np.cumsum(lens)]), dtype=torch.int32, device=dev)
    n3 = sum(lens)
    sel3_np = markov_mask(n3, 0.25, 8, gen)
    pos3 = np.concatenate([np.flatnonzero(sel3_np[c0:c0 + L]) for c0, L in zip(np.cumsum([0] + lens[:-1]), lens)])
    sel3 = torch.from_numpy(sel3_np).to(dev)[None]
    q3, k3, v3 = (x[:, :n3].detach().requires_grad_() for x in (q, k, v))

    def fb3():
        o = sq_full_attn(q3, k3, v3, sel3, cu_seqlens=cu3)
        torch.autograd.grad(o, (q3, k3, v3), do[:, :n3])
    t3 = _time_ms(fb3, 20)
    f3 = 3.5 * 4 * D * H * float((pos3 + 1).sum())
    out["cfg3_fwd_bwd_varlen"] = {"lens": lens, "ms": round(t3, 3), "tflops": round(f3 / t3 / 1e9, 1)}

    out["swa_w128_cfg4"] = swa_cfg4_measurement(q, k, v, do)
    out["generic_kernels"] = generic_measurement(dev, gen)
    N4 = 4 * 8192

    # fused epilogue at cfg4 shape: L, G [32768, 16, 128], gate [32768]
    L = (torch.randn(N4, H, D, generator=gen)).bfloat16().to(dev).requires_grad_()
    G = (torch.randn(N4, H, D, generator=gen)).bfloat16().to(dev).requires_grad_()
    gate = torch.sigmoid(torch.randn(N4, generator=gen)).bfloat16().to(dev).requires_grad_()
    thres = torch.tensor([0.5], dtype=torch.bfloat16, device=dev)
    wl = torch.ones(D, dtype=torch.bfloat16, device=dev, requires_grad=True)
    wg = torch.ones(D, dtype=torch.bfloat16, device=dev, requires_grad=True)
    dO = torch.randn(N4, H * D, generator=gen).bfloat16().to(dev)
    with torch.no_grad():
        tef = _time_ms(lambda: logo_epilogue(L, G, gate, thres, wl, wg, 1e-5), 20)
    o_e = logo_epilogue(L, G, gate, thres, wl, wg, 1e-5)
    teb = _time_ms(lambda: torch.autograd.grad(o_e, (L, G, gate, wl, wg), dO, retain_graph=True), 20)
    elem = N4 * H * D * 2
    out["epilogue_cfg4"] = {"fwd_ms": round(tef, 4), "fwd_gbs": round(3 * elem / tef / 1e6, 1),
                            "bwd_ms": round(teb, 4), "bwd_gbs": round(5 * elem / teb / 1e6, 1)}
    del L, G, o_e

    # gate-aware decode attention at cfg5 shape: B=32, H=16, D=128, ctx 16384+1, r=0.5
    B5, ctx = 32, 16385
    kc = (torch.randn(B5, H, ctx, D, generator=gen) * 0.5).bfloat16().to(dev)
    vc = torch.randn(B5, H, ctx, D, generator=gen).bfloat16().to(dev)
    q5 = torch.randn(B5, H, D, generator=gen).bfloat16().to(dev)
    gate5 = torch.tensor([0.75, 0.25] * (B5 // 2), dtype=torch.bfloat16, device=dev)
    lens5 = torch.full((B5,), ctx, dtype=torch.int32, device=dev)
    td = _time_ms(lambda: decode_attn(q5, kc, vc, lens5, gate5, thres, max_len=ctx), 20)
    bytes_active = (B5 // 2) * H * ctx * D * 2 * 2
    td_all = _time_ms(lambda: decode_attn(q5, kc, vc, lens5, max_len=ctx), 20)
    del kc, vc
    rc = read_ceiling_gbs(dev, bytes_active)
    ceiling = rc["best_gbs"]
    out["decode_global_cfg5_layer"] = {
        "active_rows": B5 // 2, "ms": round(td, 4), "gbs": round(bytes_active / td / 1e6, 1),
        "all_rows_ms": round(td_all, 4), "all_rows_gbs": round(2 * bytes_active / td_all / 1e6, 1),
        "hbm_peak_gbs": HBM_PEAK_GBS, "read_ceiling_gbs": ceiling,
        "read_ceiling_ordinary_loads_gbs": rc["ordinary_loads_best_gbs"],
        "of_read_ceiling": round(bytes_active / td / 1e6 / ceiling, 4)}
    return out


def layer_cfg4_measurement(dev, iters=5, seed=3):
    """one LoGo attention layer fwd+bwd at the 1.5B shapes
    (hidden 2048, 16 heads, D=128, window 128, linear_proj global
    re-parameterisation, context norms), B=4, T=8192, bf16.  Linear weights
    ~ N(0, 0.02); the global projections are identity + N(0, 0.02) so the
    branches differ; hidden ~ N(0, 1) and gate_proj std 1/sqrt(2048), so the
    gate logits are ~ N(0, 1) and threshold 0.5 selects about half the tokens.
    A step is the layer forward plus the backward of a random upstream
    gradient into the hidden states and every parameter.  The HIP kernels'
    own durations (HIP events around each launching operator call) are listed beside the
    step time; the remainder is the projections (hipBLASLt through torch)
    and the torch glue (RoPE and norms under autograd)."""
    from logo_amd import _lib
    from logo_amd.layers import LoGoAttention, LoGoConfig

    B, T, hidden, H = 4, 8192, 2048, 16
    D = hidden // H
    cfg = LoGoConfig(hidden_size=hidden, num_attention_heads=H, num_hidden_layers=1, window_size=128,
                     global_qk_param="linear_proj", use_context_norm=True, gate_thres_init=0.5,
                     sparse_full_attn_backend="hip")
    gen = torch.Generator()
    gen.manual_seed(seed)
    layer = LoGoAttention(cfg)
    with torch.no_grad():
        for name, p in layer.named_parameters():
            if name.endswith("_global_proj"):
                p.add_(torch.randn(p.shape, generator=gen) * 0.02)
            elif name == "gate_proj.weight":
                p.copy_(torch.randn(p.shape, generator=gen) / hidden ** 0.5)
            elif p.dim() == 2:
                p.copy_(torch.randn(p.shape, generator=gen) * 0.02)
    layer = layer.to(device=dev, dtype=torch.bfloat16).train()
    h = torch.randn(B, T, hidden, generator=gen).bfloat16().to(dev).requires_grad_()
    dout = torch.randn(B, T, hidden, generator=gen).bfloat16().to(dev)
    params = [p for p in layer.parameters() if p.requires_grad]
    with torch.no_grad():
        sel = (torch.sigmoid(layer.gate_proj(h)) >= layer.gate_thres).reshape(B, T).cpu().numpy()
    pairs = float(sum((np.flatnonzero(sel[b]) + 1).sum() for b in range(B)))

    def step():
        out, _, _ = layer(h)
        torch.autograd.grad(out, [h] + params, dout)

    for _ in range(2):
        step()
    torch.cuda.synchronize()
    timer = EventTimer()
    _lib.set_launch_hook(timer)
    timer.enabled = True
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(iters):
        step()
    b.record()
    torch.cuda.synchronize()
    timer.enabled = False
    _lib.set_launch_hook(None)
    ms = a.elapsed_time(b) / iters
    counts = timer.counts()
    kern = {k_: round(v_ * counts[k_] / iters, 4) for k_, v_ in sorted(timer.averages_ms().items())}
    N = B * T
    proj_flops = 3 * (4 * 2 * N * hidden * hidden + 3 * 2 * N * H * D * D)  # fwd + 2x bwd
    sq_flops = 3.5 * 4 * D * H * pairs
    swa_pairs = sum(min(p, 128) + 1 for p in range(T)) * B
    swa_flops = 3.5 * 4 * D * H * swa_pairs
    return {
        "ms": round(ms, 3),
        "tflops": round((proj_flops + sq_flops + swa_flops) / (ms * 1e-3) / 1e12, 1),
        "flops_per_step": {"projections": proj_flops, "sq_attn": sq_flops, "swa": swa_flops},
        "global_ratio": round(float(sel.mean()), 4),
        "hip_kernel_ms_per_step": kern,
        "hip_kernel_ms_total": round(sum(kern.values()), 3),
        "shape": {"B": B, "T": T, "hidden": hidden, "heads": H, "head_dim": D, "window": 128},
        "data": "synthetic hidden states ~N(0,1), random-init weights",
    }


def decode_layer_only(dev, calls=10):
    """Config 5's global decode branch for one layer (batch 32, 16 heads,
    D=128, 16385 cached tokens, gates alternating 0.75 / 0.25 so 16 rows are
    active), called ``calls`` times; prints one JSON line."""
    from logo_amd.ops.decode import decode_attn

    gen = torch.Generator()
    gen.manual_seed(7)
    B, H, D, ctx = 32, 16, 128, 16385
    kc = (torch.randn(B, H, ctx, D, generator=gen) * 0.5).bfloat16().to(dev)
    vc = torch.randn(B, H, ctx, D, generator=gen).bfloat16().to(dev)
    q = torch.randn(B, H, D, generator=gen).bfloat16().to(dev)
    gate = torch.tensor([0.75, 0.25] * (B // 2), dtype=torch.bfloat16, device=dev)
    thres = torch.tensor([0.5], dtype=torch.bfloat16, device=dev)
    lens = torch.full((B,), ctx, dtype=torch.int32, device=dev)
    ms = _time_ms(lambda: decode_attn(q, kc, vc, lens, gate, thres, max_len=ctx), calls)
    nbytes = (B // 2) * H * ctx * D * 2 * 2
    ceiling = read_ceiling_gbs(dev, nbytes)
    print(json.dumps({"workload": "cfg5 global decode branch, one layer, 16 of 32 rows active",
                      "ms": round(ms, 4), "algorithmic_bytes": nbytes, "gbs": round(nbytes / ms / 1e6, 1),
                      "hbm_peak_gbs": HBM_PEAK_GBS, "read_ceiling_gbs": ceiling,
                      "of_read_ceiling": round(nbytes / ms / 1e6 / ceiling["best_gbs"], 4)}), flush=True)


def read_ceiling_gbs(dev, nbytes, calls=10):
    """The read bandwidth this part delivers in practice: the library's
    streaming-read calibration kernel (logo_read_calibration) over a buffer
    of ``nbytes``, at several grid sizes, with non-temporal loads (as the
    decode kernel's cache reads) and with ordinary ones; best and per-grid
    GB/s of the non-temporal reads, best of the ordinary ones."""
    from logo_amd import _lib
    lib = _lib.lib()
    buf = torch.ones(nbytes // 2, dtype=torch.bfloat16, device=dev)
    sink = torch.zeros(65536, dtype=torch.int32, device=dev)
    st = _lib.stream_of(buf)
    per = {0: {}, 1: {}}
    for nt in (1, 0):
        for grid in (2048, 8192, 16384):
            def run():
                _lib.check(lib.logo_read_calibration(_lib.ptr(buf), nbytes, _lib.ptr(sink), grid, nt, st),
                           "logo_read_calibration")
            per[nt][grid] = round(nbytes / _time_ms(run, calls) / 1e6, 1)
    del buf
    return {"best_gbs": max(per[1].values()), "per_grid_gbs": per[1], "ordinary_loads_best_gbs": max(per[0].values())}


def decode_model_measurement(dev, batch=32, prompt=16384, steps=256, seed=4):
    """the LoGo 1.5B shapes (24 layers, hidden 2048, 16 heads,
    vocab 32000, tied embeddings), random-init bf16, a batch of random-id
    prompts, then greedy decode steps through the preallocated cache and the
    gate-aware decode kernel.  tok/s counts decode steps only (prefill is timed
    separately); every decode step runs the whole model (projections and MLP
    through torch / hipBLASLt, attention, cache and epilogue through this
    package's kernels).  The timed steps replay one captured decode step (HIP
    graph); a few eager, Python-launched steps are timed beside them."""
    from logo_amd.layers import LoGoConfig
    from logo_amd.model import LoGoForCausalLM

    cfg = LoGoConfig(vocab_size=32000, hidden_size=2048, intermediate_size=5632, num_hidden_layers=24,
                     num_attention_heads=16, window_size=128, global_qk_param="linear_proj",
                     use_context_norm=True, gate_thres_init=0.5, sparse_full_attn_backend="hip")
    gen = torch.Generator()
    gen.manual_seed(seed)
    model = LoGoForCausalLM(cfg)
    model.init_weights(gen)
    model = model.to(device=dev, dtype=torch.bfloat16).eval()
    params = sum(p.numel() for p in model.parameters())
    ids = torch.randint(0, cfg.vocab_size, (batch, prompt), generator=gen).to(dev)
    cache = model.new_cache(batch, prompt + steps + 32, device=dev)

    # realised global ratio: gate decisions of every layer at the first decode step
    gates = []
    # the gate of each layer from its input (the fused decode path computes the
    # gate logits inside its stacked projection, not through gate_proj)
    hooks = [layer.self_attn.register_forward_pre_hook(
        lambda m_, args: gates.append(torch.sigmoid(m_.gate_proj(args[0]))))
        for layer in model.model.layers]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    tok = model.prefill(ids, cache).argmax(-1)
    torch.cuda.synchronize()
    prefill_s = time.perf_counter() - t0
    gates.clear()
    tok = model.decode_step(tok, cache).argmax(-1)
    for hk in hooks:
        hk.remove()
    thres = float(cfg.gate_thres_init)
    active = [float((gt.float() >= thres).float().mean()) for gt in gates[:cfg.num_hidden_layers]]
    ratio = float(np.mean(active))
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    # eager steps (Python-launched, for reference)
    eager_steps = 16
    torch.cuda.synchronize()
    a.record()
    for _ in range(eager_steps):
        tok = model.decode_step(tok, cache).argmax(-1)
    b.record()
    torch.cuda.synchronize()
    eager_ms = a.elapsed_time(b) / eager_steps
    # the timed steps: one captured decode step, replayed
    step = model.capture_greedy_decode(tok, cache)
    torch.cuda.synchronize()
    a.record()
    for _ in range(steps):
        step()
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b)
    H, D, L = cfg.num_attention_heads, cfg.head_dim, cfg.num_hidden_layers
    ctx = prompt + 18 + steps // 2  # mean cached length over the timed steps
    per_step_bytes = (L * (batch * H * (cfg.window_size + 1) * D * 2 * 2 + ratio * batch * H * ctx * D * 2 * 2)
                      + 2 * params)
    step_ms = ms / steps
    return {
        "tok_s": round(batch * steps / (ms * 1e-3), 1),
        "ms_per_step": round(step_ms, 3),
        "mode": "one decode step captured in a HIP graph, replayed; greedy argmax between replays",
        "eager_tok_s": round(batch / (eager_ms * 1e-3), 1),
        "eager_ms_per_step": round(eager_ms, 3),
        "prefill_s": round(prefill_s, 3),
        "batch": batch, "prompt": prompt, "steps": steps,
        "global_ratio": round(ratio, 4),
        "params": params,
        "est_hbm_bytes_per_step": int(per_step_bytes),
        "est_gbs": round(per_step_bytes / (step_ms * 1e-3) / 1e9, 1),
        "roofline_tok_s": round(batch / (per_step_bytes / (HBM_PEAK_GBS * 1e9)), 1),
        "data": "synthetic random ids, random-init weights",
    }


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (collectives, sharding) and "
              "each box has a single MI355X; run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    from logo_amd import _lib
    from logo_amd.ops import sq_full_attn

    dev = torch.device("cuda", 0)
    if args.decode_layer:
        if args.copy_calibration:
            src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
            dst = torch.empty_like(src)
            torch.cuda.synchronize()
            dst.copy_(src)
            torch.cuda.synchronize()
            del src, dst
        decode_layer_only(dev)
        return
    if args.decode_model:
        print(json.dumps(decode_model_measurement(dev)), flush=True)
        return
    if args.layer:
        print(json.dumps(layer_cfg4_measurement(dev)), flush=True)
        return
    if args.generic:
        g = torch.Generator()
        g.manual_seed(7)
        print(json.dumps(generic_measurement(dev, g)), flush=True)
        return
    if args.swa:
        g = torch.Generator()
        g.manual_seed(args.seed)
        q, k, v = ((torch.randn(1, 4 * 8192, 16, 128, generator=g) * 0.5).to(torch.bfloat16).to(dev)
                   for _ in range(3))
        do = torch.randn(1, 4 * 8192, 16, 128, generator=g).to(torch.bfloat16).to(dev)
        print(json.dumps(swa_cfg4_measurement(q, k, v, do, iters=20)), flush=True)
        return
    T, H, D = args.seq_len, args.heads, args.head_dim
    q, k, v, do, sel_np = headline_inputs(T, H, D, args.ratio, args.seed)
    pos = np.flatnonzero(sel_np)
    pairs_per_head = float((pos + 1).sum())  # single sequence: p = token index
    f_fwd = 4.0 * D * H * pairs_per_head
    f_step = 3.5 * f_fwd

    qg = q.to(dev)[None].requires_grad_()
    kg = k.to(dev)[None].requires_grad_()
    vg = v.to(dev)[None].requires_grad_()
    dog = do.to(dev)[None]
    selg = torch.from_numpy(sel_np).to(dev)[None]
    cu = torch.tensor([0, T], dtype=torch.int32, device=dev)

    def step():
        o = sq_full_attn(qg, kg, vg, selg, cu_seqlens=cu)
        torch.autograd.grad(o, (qg, kg, vg), dog)

    if args.copy_calibration:
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device=dev)
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    timer = EventTimer()
    _lib.set_launch_hook(timer)
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    timer.enabled = True
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    timer.enabled = False
    _lib.set_launch_hook(None)

    ms_per_step = elapsed * 1e3 / args.steps
    value = f_step / (ms_per_step * 1e-3) / 1e12
    kern_ms = timer.averages_ms()
    flop_kernels = {n: ms for n, ms in kern_ms.items() if n in KERNEL_FLOPS_PER_PAIR_D}
    dom = max(flop_kernels, key=flop_kernels.get)
    dom_flops = KERNEL_FLOPS_PER_PAIR_D[dom] * D * H * pairs_per_head
    achieved = dom_flops / (kern_ms[dom] * 1e-3) / 1e12
    roofline = {
        "kernel": dom,
        "bound": "mfma",
        "achieved": round(achieved, 2),
        "peak": MFMA_BF16_PEAK_TFLOPS,
        "unit": "TFLOP/s",
        "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
        "traffic": measured_traffic(dom, T, H, D, args.ratio, args.seed),
        "flops_per_launch": dom_flops,
        "avg_launch_ms": round(kern_ms[dom], 4),
    }

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline(q, k, v, sel_np, [0, T], do, min(args.cpu_heads, H), f_step / H)

    extra = None if args.no_extra else extra_measurements(dev)
    if not args.no_extra:
        extra["layer_cfg4_fwd_bwd"] = layer_cfg4_measurement(dev)
    if not args.no_extra and not args.no_decode:
        extra["decode_cfg5_model"] = decode_model_measurement(dev)

    line = {
        "metric": "sq_full_attn fwd+bwd effective TFLOP/s @T=32K, 25% global; decode tok/s",
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": "sq_full_attn fwd+bwd, single sequence, selection Markov spans (mean run 8)",
            "T": T, "HQ": H, "H": H, "D": D,
            "global_ratio": round(float(sel_np.mean()), 4),
            "effective_tflop_per_step": round(f_step / 1e12, 4),
            "seed": args.seed,
        },
        "roofline": roofline,
        "cpu_baseline": cpu,
        "kernel_ms": {k_: round(v_, 4) for k_, v_ in sorted(kern_ms.items())},
        "kernel_tflops": {n: round(KERNEL_FLOPS_PER_PAIR_D[n] * D * H * pairs_per_head / (ms * 1e-3) / 1e12, 2)
                          for n, ms in flop_kernels.items()},
        "extra": extra,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
