"""The C-ABI library loads and exports every symbol include/logo_hip.h declares.

Runs without a GPU: only symbol lookup and argument validation (which returns
before any HIP call) are exercised.
"""

import ctypes

import pytest

from logo_amd import _lib


def test_header_symbols_are_exported():
    names = _lib.header_symbols()
    assert "logo_sq_fwd" in names and "logo_compact" in names
    lib = _lib.lib()
    for name in names:
        assert hasattr(lib, name), f"{name} declared in include/logo_hip.h but not exported"
        assert name in _lib.SIGNATURES, f"{name} has no ctypes signature"


def test_abi_version_and_workspace():
    lib = _lib.lib()
    assert lib.logo_abi_version() == 1
    assert lib.logo_compact_workspace_bytes(4096, 1) == 4
    assert lib.logo_compact_workspace_bytes(4097, 16) == 2 * 16 * 4


@pytest.mark.parametrize("d,hq,h,lanes,msg", [
    (96, 4, 4, 1, "head dim"),
    (128, 6, 4, 1, "multiple"),
    (128, 4, 4, 2, "lanes"),
])
def test_fwd_rejects_bad_shapes_without_touching_gpu(d, hq, h, lanes, msg):
    lib = _lib.lib()
    p = ctypes.c_void_p(1)
    rc = lib.logo_sq_fwd(p, p, p, p, p, None, None, p, p, 128, 1, hq, h, d, lanes, 0.1, -1,
                         _lib.DTYPE_BF16, None)
    assert rc == 1
    assert msg in lib.logo_last_error().decode()


def test_compact_rejects_bad_arguments():
    lib = _lib.lib()
    p = ctypes.c_void_p(1)
    assert lib.logo_compact(p, -1, 1, p, 1, p, p, p, p, None) == 1
    assert lib.logo_compact(p, 16, 0, p, 1, p, p, p, p, None) == 1
    assert "lanes" in lib.logo_last_error().decode()


def test_ops_refuse_cpu_tensors():
    import torch

    from logo_amd.ops import sq_full_attn

    q = torch.zeros(1, 8, 2, 64, dtype=torch.bfloat16)
    sel = torch.ones(1, 8, dtype=torch.bool)
    cu = torch.tensor([0, 8], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        sq_full_attn(q, q, q, sel, cu_seqlens=cu)


def test_reference_assertions_are_kept():
    import torch

    from logo_amd.ops import sq_full_attn

    q = torch.zeros(1, 8, 2, 64)
    k = torch.zeros(1, 8, 2, 64)
    with pytest.raises(AssertionError, match="cu_seqlens"):
        sq_full_attn(q, k, k, torch.ones(1, 8, dtype=torch.bool))
    with pytest.raises(AssertionError, match="bool mask"):
        sq_full_attn(q, k, k, torch.ones(1, 8), cu_seqlens=torch.tensor([0, 8]))
    with pytest.raises(AssertionError, match="B=1"):
        sq_full_attn(torch.zeros(2, 8, 2, 64), torch.zeros(2, 8, 2, 64), torch.zeros(2, 8, 2, 64),
                     torch.ones(2, 8, dtype=torch.bool), cu_seqlens=torch.tensor([0, 8]))
    with pytest.raises(AssertionError, match="GQA"):
        sq_full_attn(torch.zeros(1, 8, 3, 64), k, k, torch.ones(1, 8, dtype=torch.bool),
                     cu_seqlens=torch.tensor([0, 8]))
