"""The TORCH_LIBRARY(logo_hip) shim: schemas and fake kernels (CPU, no launch).

The shim (logo_amd/_logo_torch.so, torch_ops/logo_torch_ops.cpp) registers the
hot-path entry points as ``torch.ops.logo_hip`` operators; their fake kernels
give output shapes for torch.library / torch.compile without a GPU.  The real
kernels behind the same schemas are checked with torch.library.opcheck in
tests/test_gpu_torch_ops.py.
"""

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensorMode

from logo_amd import _lib, _torch_ops

OPS = ("compact", "dense_meta", "sq_fwd", "sq_bwd_delta", "sq_bwd_dq", "sq_bwd_dkv", "sq_bwd", "epilogue_fwd",
       "epilogue_bwd", "decode_attn")


def test_every_operator_has_a_schema():
    ops = _torch_ops.ops()
    for name in OPS:
        schema = getattr(ops, name).default._schema
        assert schema.name == f"logo_hip::{name}"


def test_fake_kernels_give_output_shapes():
    ops = _torch_ops.ops()
    n, hq, h, d = 300, 4, 2, 128
    with FakeTensorMode():
        bf = dict(dtype=torch.bfloat16, device="cuda")
        q, k, v = torch.empty(n, hq, d, **bf), torch.empty(n, h, d, **bf), torch.empty(n, h, d, **bf)
        cu = torch.empty(3, dtype=torch.int32, device="cuda")
        sel = torch.empty(n, hq, dtype=torch.uint8, device="cuda")
        q_idx, pos, meta = ops.compact(sel, cu)
        assert q_idx.shape == (hq, n) and q_idx.dtype == torch.int64 and pos.dtype == torch.int32
        assert meta.shape == (hq * _lib.meta_stride(2),)
        o, lse = ops.sq_fwd(q, k, v, q_idx, pos, meta, cu, hq, 0.1, -1)
        assert o.shape == q.shape and o.dtype == q.dtype and lse.shape == (hq, n) and lse.dtype == torch.float32
        delta, q_sel, do_sel = ops.sq_bwd_delta(q, k, v, o, lse, o, q_idx, pos, meta, cu, hq, 0.1, -1)
        assert delta.shape == (hq, n) and q_sel.shape == (hq, n, d) and do_sel.shape == (hq, n, d)
        dense = ops.sq_bwd_delta(q, k, v, o, lse, o, None, None, meta, cu, 1, 0.1, 128)
        assert dense[1].numel() == 0
        dq = ops.sq_bwd_dq(q, k, v, o, lse, o, q_idx, pos, meta, cu, hq, 0.1, -1, delta, q_sel, do_sel)
        dk, dv = ops.sq_bwd_dkv(q, k, v, o, lse, o, q_idx, pos, meta, cu, hq, 0.1, -1, delta, q_sel, do_sel)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == v.shape
        grads = ops.sq_bwd(q, k, v, o, lse, o, q_idx, pos, meta, cu, hq, 0.1, -1)
        assert [x.shape for x in grads] == [q.shape, k.shape, v.shape]
        L = torch.empty(n, hq, d, **bf)
        gate, w = torch.empty(n, **bf), torch.empty(d, **bf)
        th = torch.empty(1, **bf)
        out = ops.epilogue_fwd(L, L, gate, th, w, w, 1e-5)
        assert out.shape == (n, hq * d)
        grads = ops.epilogue_bwd(L, L, gate, th, w, w, out, 1e-5)
        assert [g.shape for g in grads] == [L.shape, L.shape, gate.shape, w.shape, w.shape]
        qd = torch.empty(4, hq, d, **bf)
        cache = torch.empty(4, h, 64, d, **bf)
        lens = torch.empty(4, dtype=torch.int32, device="cuda")
        assert ops.decode_attn(qd, cache, cache, lens, None, None, 64, 0.1).shape == qd.shape


def test_operators_refuse_cpu_tensors():
    ops = _torch_ops.ops()
    cu = torch.tensor([0, 8], dtype=torch.int32)
    with pytest.raises((RuntimeError, NotImplementedError)):
        ops.dense_meta(cu, 8)


@pytest.mark.parametrize("cu,env,want", [
    ([0, 100], None, False), ([0, 100], "1", False),        # a single sequence keeps one stream
    ([0, 40, 100], None, False), ([0, 40, 100], "0", False),  # off by default
    ([0, 40, 100], "1", True), ([0, 0, 40, 100], "1", True),
])
def test_two_stream_backward_policy(cu, env, want, monkeypatch):
    """The packed backward's dk / dv goes to a side stream only when
    LOGO_BWD_OVERLAP=1 and the call packs more than one sequence (the GPU
    side, bit-identical results included, is in tests/test_gpu_bwd_overlap.py)."""
    from logo_amd.ops.common import DeviceSelection
    from logo_amd.ops.sq_attn import _overlap_dkv

    if env is None:
        monkeypatch.delenv("LOGO_BWD_OVERLAP", raising=False)
    else:
        monkeypatch.setenv("LOGO_BWD_OVERLAP", env)
    cu_t = torch.tensor(cu, dtype=torch.int32)
    dsel = DeviceSelection(meta=torch.zeros(1, dtype=torch.int32), cu=cu_t, q_idx=None, pos=None,
                           n_tokens=cu[-1], nseq=len(cu) - 1, lanes=1)
    assert _overlap_dkv(dsel) is want
