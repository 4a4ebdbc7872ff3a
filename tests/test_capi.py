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
    assert lib.logo_abi_version() == 7
    # the generic kernels serve d = 256 and fp32; they never split
    assert [lib.logo_sq_generic(d, t) for d in (64, 128, 256) for t in (_lib.DTYPE_BF16, _lib.DTYPE_F16)] == \
        [0, 0, 0, 0, 1, 1]
    assert all(lib.logo_sq_generic(d, _lib.DTYPE_F32) == 1 for d in (64, 128, 256))
    assert lib.logo_sq_workspace_bytes(32768, 1, 16, 256) == 0
    assert lib.logo_compact_workspace_bytes(4096, 1) == 4
    assert lib.logo_compact_workspace_bytes(4097, 16) == 2 * 16 * 4


@pytest.mark.parametrize("d,v_dim,hq,h,lanes,msg", [
    (96, 96, 4, 4, 1, "head dim"),
    (192, 192, 4, 4, 1, "head dim"),
    (512, 512, 4, 4, 1, "head dim"),
    (256, 128, 4, 4, 1, "value head dim"),
    (128, 128, 6, 4, 1, "multiple"),
    (128, 128, 4, 4, 2, "lanes"),
    (128, 64, 4, 4, 1, "value head dim"),
    (64, 128, 4, 4, 1, "value head dim"),
])
def test_fwd_bwd_reject_bad_shapes_without_touching_gpu(d, v_dim, hq, h, lanes, msg):
    lib = _lib.lib()
    p = ctypes.c_void_p(1)
    rc = lib.logo_sq_fwd(p, p, p, p, p, None, None, p, p, 128, 1, hq, h, d, v_dim, lanes, 0.1, -1,
                         _lib.DTYPE_BF16, None, 0, None)
    assert rc == 1
    assert msg in lib.logo_last_error().decode()
    for fn in (lib.logo_sq_bwd, lib.logo_sq_bwd_delta, lib.logo_sq_bwd_dq, lib.logo_sq_bwd_dkv):
        rc = fn(p, p, p, p, p, p, p, p, p, p, p, p, None, None, p, p, 128, 1, hq, h, d, v_dim, lanes, 0.1, -1,
                _lib.DTYPE_BF16, None, 0, None)
        assert rc == 1
        assert msg in lib.logo_last_error().decode()


@pytest.mark.parametrize("sparse,window,dtype,msg", [
    (False, -1, 2, "fp16 and fp32 are supported on the query-sparse path"),   # dense fp16
    (True, 128, 2, "fp16 and fp32 are supported on the query-sparse path"),   # sliding-window fp16
    (False, -1, 1, "fp16 and fp32 are supported on the query-sparse path"),   # dense fp32
    (True, 64, 1, "fp16 and fp32 are supported on the query-sparse path"),    # sliding-window fp32
    (True, -1, 7, "unsupported"),
])
def test_fwd_bwd_dtype_checks_without_touching_gpu(sparse, window, dtype, msg):
    """fp16 and fp32 run on the query-sparse kernels without a window only;
    other dtypes are refused before any HIP call."""
    lib = _lib.lib()
    p = ctypes.c_void_p(1)
    idx = p if sparse else None
    rc = lib.logo_sq_fwd(p, p, p, p, p, idx, idx, p, p, 128, 1, 4, 4, 128, 128, 1, 0.1, window, dtype, None, 0, None)
    assert rc == 1 and msg in lib.logo_last_error().decode()
    for fn in (lib.logo_sq_bwd, lib.logo_sq_bwd_delta, lib.logo_sq_bwd_dq, lib.logo_sq_bwd_dkv):
        rc = fn(p, p, p, p, p, p, p, p, p, p, p, p, idx, idx, p, p, 128, 1, 4, 4, 128, 128, 1, 0.1, window,
                dtype, None, 0, None)
        assert rc == 1 and msg in lib.logo_last_error().decode()


def test_compact_rejects_bad_arguments():
    lib = _lib.lib()
    p = ctypes.c_void_p(1)
    assert lib.logo_compact(p, -1, 1, p, 1, p, p, p, p, None) == 1
    assert lib.logo_compact(p, 16, 0, p, 1, p, p, p, p, None) == 1
    assert "lanes" in lib.logo_last_error().decode()


def test_head_linear_grad_acc_rejects_bad_arguments():
    """The addend form of the per-head map refuses a null addend, an
    unaligned or too-short addend row stride and unsupported head dims, all
    before any HIP call (pointers are placeholders)."""
    lib = _lib.lib()
    p = ctypes.c_void_p(256)
    args = lambda add, ldadd, d: (p, 4 * d, p, add, ldadd, p, 4 * d, 100, 4, d, _lib.DTYPE_BF16, None)  # noqa: E731
    for add, ldadd, d, msg in ((None, 512, 128, "null"), (p, 500, 128, "addend"), (p, 256, 128, "addend"),
                               (p, 384, 96, "head dim")):
        assert lib.logo_head_linear_grad_acc(*args(add, ldadd, d)) == 1
        assert msg in lib.logo_last_error().decode()


def test_read_calibration_rejects_bad_arguments():
    """The streaming-read calibration refuses null pointers, an unaligned
    buffer or size and grids outside [1, 65536], for either load kind, before
    any HIP call (pointers are placeholders)."""
    lib = _lib.lib()
    p = ctypes.c_void_p(256)
    for nt in (0, 1):
        for buf, nbytes, sink, grid, msg in ((None, 1024, p, 8, "null"), (p, 1024, None, 8, "null"),
                                             (ctypes.c_void_p(264), 1024, p, 8, "aligned"),
                                             (p, 1000, p, 8, "aligned"), (p, 1024, p, 0, "grid"),
                                             (p, 1024, p, 65537, "grid")):
            assert lib.logo_read_calibration(buf, nbytes, sink, grid, nt, None) == 1
            assert msg in lib.logo_last_error().decode()


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


class _LaunchCounter:
    def __init__(self):
        self.n = 0

    def __call__(self, name, when):
        self.n += 1


@pytest.mark.parametrize("qshape,kshape,vshape,msg", [
    ((1, 8, 2, 128), (1, 8, 2, 128), (1, 8, 2, 320), "head dims K, V"),
    ((1, 8, 2, 320), (1, 8, 2, 320), (1, 8, 2, 64), "single block"),
    ((1, 8, 2, 257), (1, 8, 2, 257), (1, 8, 2, 257), "single block"),
    ((1, 8, 2, 128), (1, 8, 2, 64), (1, 8, 2, 128), "same head dim K"),
    ((1, 8, 4, 128), (1, 8, 2, 128), (1, 8, 1, 128), "same number of heads"),
    ((1, 8, 2, 128), (1, 9, 2, 128), (1, 9, 2, 128), "share"),
])
def test_unsupported_shapes_are_rejected_before_any_launch(qshape, kshape, vshape, msg):
    """AssertionError (the reference's error convention) before any launch and
    before the GPU check, for every op that runs the attention kernels."""
    import torch

    from logo_amd.ops import dense_causal_attn, sq_full_attn, swa_attn

    q, k, v = torch.zeros(qshape), torch.zeros(kshape), torch.zeros(vshape)
    cu = torch.tensor([0, qshape[1]], dtype=torch.int32)
    counter = _LaunchCounter()
    _lib.set_launch_hook(counter)
    try:
        with pytest.raises(AssertionError, match=msg):
            sq_full_attn(q, k, v, torch.ones(1, qshape[1], dtype=torch.bool), cu_seqlens=cu)
        with pytest.raises(AssertionError, match=msg):
            swa_attn(q, k, v, cu)
        with pytest.raises(AssertionError, match=msg):
            dense_causal_attn(q, k, v, cu)
    finally:
        _lib.set_launch_hook(None)
    assert counter.n == 0


@pytest.mark.parametrize("K,V,d", [(128, 128, 128), (64, 64, 64), (96, 96, 128), (128, 64, 128),
                                   (64, 128, 128), (48, 32, 64), (1, 1, 64), (256, 256, 256), (192, 160, 256),
                                   (128, 192, 256), (129, 8, 256)])
def test_supported_head_dims_map_to_a_compiled_dim(K, V, d):
    """K, V <= 256 (V != K included, as the reference's single K block of
    <= 256 allows) run on the compiled dim 64, 128 or 256; the GPU parity of
    the padded calls is in tests/test_gpu_sq_attn.py and
    tests/test_gpu_generic.py."""
    import torch

    from logo_amd.ops import sq_full_attn
    from logo_amd.ops.sq_attn import kernel_head_dim

    assert kernel_head_dim(K, V) == d
    q, k, v = torch.zeros(1, 8, 2, K), torch.zeros(1, 8, 2, K), torch.zeros(1, 8, 2, V)
    # shapes pass the checks; the CPU tensors then stop at the no-fallback guard
    with pytest.raises(RuntimeError, match="no CPU fallback"):
        sq_full_attn(q, k, v, torch.ones(1, 8, dtype=torch.bool), cu_seqlens=torch.tensor([0, 8]))
