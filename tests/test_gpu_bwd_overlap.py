"""The packed backward's two-stream form against its one-stream form.

With LOGO_BWD_OVERLAP=1, calls that pack more than one sequence launch
dk / dv on a side stream and dq behind it on the caller's stream
(logo_amd/ops/sq_attn.py ``_bwd``).  The kernels are the same either way,
so outputs and gradients must be bit-identical to the default (every launch
on the caller's stream), eagerly and when the whole forward + backward is
captured in a HIP graph and replayed between eager calls.  The launch hook
checks that the dk / dv launch really ran off the caller's stream with the
switch on, on it by default, and that a single sequence keeps one stream.
"""

import pytest
import torch

from logo_amd import _lib
from logo_amd.ops import dense_causal_attn, sq_full_attn, swa_attn
from tests.helpers import gen, randn

pytestmark = pytest.mark.gpu


class _StreamLog:
    """Launch hook: the stream each entry point was launched on."""

    def __init__(self):
        self.streams = {}

    def __call__(self, name, phase):
        if phase == "start":
            self.streams.setdefault(name, []).append(torch.cuda.current_stream().cuda_stream)


def _grads(op, q, k, v, do):
    qg, kg, vg = (x.clone().requires_grad_() for x in (q, k, v))
    o = op(qg[None], kg[None], vg[None])[0]
    return (o, *torch.autograd.grad(o, (qg, kg, vg), do))


def _inputs(seed, n, hq, h, d, dtype=torch.bfloat16):
    g = gen(seed)
    q, k, v, do = (randn((n, x, d), g, 0.5, dtype=dtype) for x in (hq, h, h, hq))
    return g, q, k, v, do


@pytest.mark.parametrize("case", ["sparse_gqa", "sparse_per_head", "sparse_fp16", "generic_d256", "fp32",
                                  "dense", "swa_gqa"])
def test_two_stream_backward_is_bit_identical(gpu, case, monkeypatch):
    n, hq, h, d, dtype = 3000, 4, 2, 128, torch.bfloat16
    if case == "sparse_per_head":
        d, h = 64, 4
    elif case == "sparse_fp16":
        dtype = torch.float16
    elif case == "generic_d256":
        d = 256
    elif case == "fp32":
        d, dtype = 64, torch.float32
    g, q, k, v, do = _inputs(70 + len(case), n, hq, h, d, dtype)
    q, k, v, do = (x.to(gpu) for x in (q, k, v, do))
    cu = torch.tensor([0, 700, 701, 2100, n], dtype=torch.int32, device=gpu)
    sel = (torch.rand((n, hq) if case == "sparse_per_head" else (n,), generator=g) < 0.3).to(gpu)
    if case == "dense":
        op = lambda q, k, v: dense_causal_attn(q, k, v, cu)  # noqa: E731
    elif case == "swa_gqa":  # HQ != H: the window runs on the dq and dk/dv kernels
        op = lambda q, k, v: swa_attn(q, k, v, cu, window=64)  # noqa: E731
    else:
        op = lambda q, k, v: sq_full_attn(q, k, v, sel[None], cu_seqlens=cu)  # noqa: E731

    monkeypatch.delenv("LOGO_BWD_OVERLAP", raising=False)
    log_one = _StreamLog()
    _lib.set_launch_hook(log_one)
    try:
        one = _grads(op, q, k, v, do)
        torch.cuda.synchronize()
        monkeypatch.setenv("LOGO_BWD_OVERLAP", "1")
        log_two = _StreamLog()
        _lib.set_launch_hook(log_two)
        two = _grads(op, q, k, v, do)
        torch.cuda.synchronize()
    finally:
        _lib.set_launch_hook(None)
    for name, a, b in zip(("o", "dq", "dk", "dv"), one, two):
        assert torch.equal(a, b), name
    assert log_one.streams["logo_sq_bwd_dkv"] == log_one.streams["logo_sq_bwd_dq"]
    assert log_two.streams["logo_sq_bwd_dkv"] != log_two.streams["logo_sq_bwd_dq"]
    assert log_two.streams["logo_sq_bwd_dq"] == log_two.streams["logo_sq_bwd_delta"]


def test_single_sequence_keeps_one_stream(gpu, monkeypatch):
    monkeypatch.setenv("LOGO_BWD_OVERLAP", "1")
    _, q, k, v, do = _inputs(80, 1500, 2, 2, 128)
    q, k, v, do = (x.to(gpu) for x in (q, k, v, do))
    cu = torch.tensor([0, 1500], dtype=torch.int32, device=gpu)
    sel = torch.ones(1, 1500, dtype=torch.bool, device=gpu)
    log = _StreamLog()
    _lib.set_launch_hook(log)
    try:
        _grads(lambda q, k, v: sq_full_attn(q, k, v, sel, cu_seqlens=cu), q, k, v, do)
        torch.cuda.synchronize()
    finally:
        _lib.set_launch_hook(None)
    assert log.streams["logo_sq_bwd_dkv"] == log.streams["logo_sq_bwd_dq"]


def test_two_stream_backward_under_graph_capture(gpu, monkeypatch):
    """sq_full_attn forward + backward on packed sequences captured in a HIP
    graph (the side stream forks from and joins the capturing stream):
    three replays, with eager calls between them, each equal bit for bit to
    the first eager call."""
    monkeypatch.setenv("LOGO_BWD_OVERLAP", "1")
    n, hq, h, d = 4000, 4, 2, 128
    g, q, k, v, do = _inputs(81, n, hq, h, d)
    q, k, v = (x.to(gpu).requires_grad_() for x in (q, k, v))
    do = do.to(gpu)
    cu = torch.tensor([0, 1500, 1501, n], dtype=torch.int32, device=gpu)
    sel = (torch.rand(n, generator=g) < 0.3).to(gpu)

    def step():
        o = sq_full_attn(q[None], k[None], v[None], sel[None], cu_seqlens=cu)[0]
        return (o.detach(), *torch.autograd.grad(o, (q, k, v), do))

    ref = step()
    torch.cuda.synchronize()
    warm = torch.cuda.Stream()
    warm.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(warm):
        for _ in range(2):
            step()
    torch.cuda.current_stream().wait_stream(warm)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = step()
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for name, a, b in zip(("o", "dq", "dk", "dv"), captured, ref):
            assert torch.equal(a, b), f"{name}, replay {rep}"
        eager = step()
        torch.cuda.synchronize()
        for name, a, b in zip(("o", "dq", "dk", "dv"), eager, ref):
            assert torch.equal(a, b), f"{name}, eager call after replay {rep}"
