"""torch.library.opcheck of the logo_hip operators on the GPU: schema, fake
kernel against the real one, and dispatch under AOTAutograd with dynamic
shapes; plus sq_full_attn under torch.compile matching eager."""

import pytest
import torch

from logo_amd import _torch_ops
from logo_amd.ops import sq_full_attn
from logo_amd.ops.common import compact_selection
from tests.helpers import gen, randn

pytestmark = pytest.mark.gpu

_CHECKS = ("test_schema", "test_faketensor", "test_aot_dispatch_dynamic")


def _inputs(dev, n=700, hq=4, h=2, d=128, dtype=torch.bfloat16):
    g = gen(40)
    q, k, v, do = (randn((n, x, d), g, dtype=dtype).to(dev) for x in (hq, h, h, hq))
    sel = (torch.rand(n, generator=g) < 0.4).to(dev)
    cu = torch.tensor([0, 300, n], dtype=torch.int32, device=dev)
    return q, k, v, do, sel, cu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_opcheck_attention_ops(gpu, dtype):
    ops = _torch_ops.ops()
    q, k, v, do, sel, cu = _inputs(gpu, dtype=dtype)
    dsel = compact_selection(sel, cu)
    torch.library.opcheck(ops.compact.default, (sel.view(torch.uint8), cu), test_utils=_CHECKS)
    fwd_args = (q, k, v, dsel.q_idx, dsel.pos, dsel.meta, cu, 1, 0.088, -1)
    torch.library.opcheck(ops.sq_fwd.default, fwd_args, test_utils=_CHECKS)
    o, lse = ops.sq_fwd(*fwd_args)
    bwd_args = (q, k, v, o, lse, do, dsel.q_idx, dsel.pos, dsel.meta, cu, 1, 0.088, -1)
    torch.library.opcheck(ops.sq_bwd.default, bwd_args, test_utils=_CHECKS)
    # the per-phase ops pass workspaces whose rows past Sq are unspecified
    # (q_sel, do_sel): schema and fake kernel only
    phase = ("test_schema", "test_faketensor")
    torch.library.opcheck(ops.sq_bwd_delta.default, bwd_args, test_utils=phase)
    ws = ops.sq_bwd_delta(*bwd_args)
    torch.library.opcheck(ops.sq_bwd_dq.default, (*bwd_args, *ws), test_utils=phase)
    torch.library.opcheck(ops.sq_bwd_dkv.default, (*bwd_args, *ws), test_utils=phase)
    # and the phases give what the whole backward gives
    dq, dk, dv = ops.sq_bwd(*bwd_args)
    assert torch.equal(dq, ops.sq_bwd_dq(*bwd_args, *ws))
    assert all(torch.equal(a, b) for a, b in zip((dk, dv), ops.sq_bwd_dkv(*bwd_args, *ws)))


def test_opcheck_epilogue_and_decode(gpu):
    ops = _torch_ops.ops()
    g = gen(41)
    n, hq, d = 257, 4, 128
    L, G = randn((n, hq, d), g).to(gpu), randn((n, hq, d), g).to(gpu)
    gate = torch.rand(n, generator=g).bfloat16().to(gpu)
    th = torch.tensor([0.5], dtype=torch.bfloat16, device=gpu)
    w = (1 + 0.1 * torch.randn(d, generator=g)).bfloat16().to(gpu)
    torch.library.opcheck(ops.epilogue_fwd.default, (L, G, gate, th, w, w, 1e-5), test_utils=_CHECKS)
    dout = randn((n, hq * d), g).to(gpu)
    torch.library.opcheck(ops.epilogue_bwd.default, (L, G, gate, th, w, w, dout, 1e-5), test_utils=_CHECKS)
    q = randn((3, hq, d), g).to(gpu)
    cache = randn((3, 2, 600, d), g).to(gpu)
    lens = torch.tensor([1, 600, 333], dtype=torch.int32, device=gpu)
    torch.library.opcheck(ops.decode_attn.default, (q, cache, cache, lens, gate[:3].contiguous(), th, 600, 0.088),
                          test_utils=_CHECKS)


def test_sq_full_attn_under_torch_compile(gpu):
    q, k, v, do, sel, cu = _inputs(gpu)

    def f(q, k, v):
        return sq_full_attn(q[None], k[None], v[None], sel[None], cu_seqlens=cu)[0]

    want = f(q, k, v)
    got = torch.compile(f)(q, k, v)
    assert torch.equal(got, want)


def test_split_workspace_under_graph_capture(gpu):
    """sq_fwd and sq_bwd_dq on a shape whose key ranges split, captured in a
    HIP graph and replayed, with eager calls of the same ops (which use the
    per-stream cached workspace) before, between and after the replays: every
    replay and every eager call gives the first eager call's results bit for
    bit.  Under capture the operator takes a fresh workspace from the graph's
    pool with its counters cleared by a recorded fill kernel, so neither side
    depends on the other's buffer or counters."""
    ops = _torch_ops.ops()
    g = gen(45)
    n, hq, h, d = 16384, 4, 4, 128
    q, k, v, do = (randn((n, x, d), g, 0.5).to(gpu) for x in (hq, h, h, hq))
    sel = (torch.rand(n, generator=g) < 0.03).to(gpu)
    sel[0] = True
    cu = torch.tensor([0, n], dtype=torch.int32, device=gpu)
    dsel = compact_selection(sel, cu)
    fwd_args = (q, k, v, dsel.q_idx, dsel.pos, dsel.meta, cu, 1, d ** -0.5, -1)
    o_ref, lse_ref = ops.sq_fwd(*fwd_args)
    bwd_args = (q, k, v, o_ref, lse_ref, do, dsel.q_idx, dsel.pos, dsel.meta, cu, 1, d ** -0.5, -1)
    ws = ops.sq_bwd_delta(*bwd_args)
    dq_ref = ops.sq_bwd_dq(*bwd_args, *ws)
    torch.cuda.synchronize()

    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):  # warm-up on the capture stream (cached workspace)
        ops.sq_fwd(*fwd_args)
        ops.sq_bwd_dq(*bwd_args, *ws)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        o_c, lse_c = ops.sq_fwd(*fwd_args)
        dq_c = ops.sq_bwd_dq(*bwd_args, *ws)
    for rep in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(o_c, o_ref) and torch.equal(lse_c, lse_ref), f"forward replay {rep}"
        assert torch.equal(dq_c, dq_ref), f"dq replay {rep}"
        o_e, lse_e = ops.sq_fwd(*fwd_args)
        dq_e = ops.sq_bwd_dq(*bwd_args, *ws)
        torch.cuda.synchronize()
        assert torch.equal(o_e, o_ref) and torch.equal(dq_e, dq_ref), f"eager call after replay {rep}"
