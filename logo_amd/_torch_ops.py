"""The ``torch.ops.logo_hip`` operators: loader and fake (meta) kernels.

``_logo_torch.so`` registers the hot-path entry points of ``liblogo_hip.so``
as PyTorch operators (``TORCH_LIBRARY(logo_hip)``, torch_ops/logo_torch_ops.cpp),
so ``torch.library`` and ``torch.compile`` see them with schemas; the fake
kernels below give their output shapes and dtypes without running anything.
The ops raise, like the C library, when the shim was not built or a tensor is
not on a ROCm GPU: there is no CPU fallback.
"""

import os

import torch

from . import _lib

SHIM_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "_logo_torch.so")

_ops = None


def ops():
    """``torch.ops.logo_hip`` (loads the shim on first use)."""
    global _ops
    if _ops is None:
        if not os.path.exists(SHIM_PATH):
            raise RuntimeError(f"{SHIM_PATH} is missing: build it with `python -m logo_amd.build`. "
                               "The LoGo HIP ops have no CPU fallback.")
        _lib.lib()
        torch.ops.load_library(SHIM_PATH)
        _register_fakes()
        _ops = torch.ops.logo_hip
    return _ops


def _register_fakes():
    fake = torch.library.register_fake

    @fake("logo_hip::compact")
    def _(selection, cu):
        n = selection.shape[0]
        lanes = selection.shape[1] if selection.dim() == 2 else 1
        stride = _lib.meta_stride(cu.shape[0] - 1)
        return (selection.new_empty((lanes, max(n, 1)), dtype=torch.int64),
                selection.new_empty((lanes, max(n, 1)), dtype=torch.int32),
                selection.new_empty((lanes * stride,), dtype=torch.int32))

    @fake("logo_hip::dense_meta")
    def _(cu, n_tokens):
        return cu.new_empty((_lib.meta_stride(cu.shape[0] - 1),))

    @fake("logo_hip::sq_fwd")
    def _(q, k, v, q_idx, pos, meta, cu, lanes, scale, window):
        return torch.empty_like(q), q.new_empty((q.shape[1], q.shape[0]), dtype=torch.float32)

    @fake("logo_hip::sq_bwd_delta")
    def _(q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window):
        copies = q_idx is not None and not generic_kernels(q.shape[2], q.dtype)
        sel = (q.shape[1], q.shape[0], q.shape[2]) if copies else (0,)
        return q.new_empty((q.shape[1], q.shape[0]), dtype=torch.float32), q.new_empty(sel), q.new_empty(sel)

    @fake("logo_hip::sq_bwd_dq")
    def _(q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window, delta, q_sel, do_sel):
        return torch.empty_like(q)

    @fake("logo_hip::sq_bwd_dkv")
    def _(q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window, delta, q_sel, do_sel):
        return torch.empty_like(k), torch.empty_like(v)

    @fake("logo_hip::sq_bwd_dqkv")
    def _(q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window, delta, q_sel, do_sel):
        return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)

    @fake("logo_hip::sq_bwd")
    def _(q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window):
        return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)

    @fake("logo_hip::epilogue_fwd")
    def _(L, G, gate, thres, w_l, w_g, eps):
        return L.new_empty((L.shape[0], L.shape[1] * L.shape[2]))

    @fake("logo_hip::epilogue_bwd")
    def _(L, G, gate, thres, w_l, w_g, dout, eps):
        return (torch.empty_like(L), torch.empty_like(G), torch.empty_like(gate), torch.empty_like(w_l),
                torch.empty_like(w_g))

    @fake("logo_hip::decode_attn")
    def _(q, k_cache, v_cache, lens, gate, thres, max_len, scale):
        return torch.empty_like(q)


def generic_kernels(d: int, dtype: torch.dtype) -> bool:
    """Whether head dim ``d`` and element type ``dtype`` run on the library's
    generic attention kernels (``logo_sq_generic``: d = 256 or fp32)."""
    code = {torch.float16: _lib.DTYPE_F16, torch.float32: _lib.DTYPE_F32}.get(dtype, _lib.DTYPE_BF16)
    return bool(_lib.lib().logo_sq_generic(int(d), code))


def timed(name: str, fn, *args):
    """Call operator ``fn`` bracketed by ``_lib``'s launch hook under the C
    entry point's ``name`` (per-kernel timing in bench.py)."""
    hook = _lib._launch_hook
    if hook is not None:
        hook(name, "start")
    out = fn(*args)
    if hook is not None:
        hook(name, "end")
    return out
