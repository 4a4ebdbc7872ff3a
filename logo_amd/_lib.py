"""Loader for ``liblogo_hip.so``, the C-ABI library of the HIP kernels.

The library is built in-tree by ``logo_amd/build.py``.  There is no CPU or
PyTorch fallback: if the library is missing, or a tensor is not on a ROCm GPU,
the ops raise.
"""

import ctypes
import os
import re

import torch

# LOGO_HIP_LIB overrides the in-tree library (e.g. to time a variant build
# against the default one in the same run).
LIB_PATH = os.environ.get("LOGO_HIP_LIB") or os.path.join(os.path.dirname(os.path.abspath(__file__)),
                                                          "liblogo_hip.so")
HEADER_PATH = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include",
                           "logo_hip.h")

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# argtypes per exported symbol (must mirror include/logo_hip.h).
SIGNATURES = {
    "logo_last_error": ([], ctypes.c_char_p),
    "logo_abi_version": ([], _I),
    "logo_compact_workspace_bytes": ([_I64, _I], _SZ),
    "logo_compact": ([_P, _I64, _I, _P, _I, _P, _P, _P, _P, _P], _I),
    "logo_compact_noalloc": ([_P, _I64, _I, _P, _I, _P, _P, _P, _P], _I),
    "logo_dense_meta": ([_P, _I, _I64, _P, _P], _I),
    "logo_chunk_indices": ([_P, _I, _I, _P, _I64, _P, _P, _P], _I),
    "logo_q_start_blk": ([_P, _P, _P, _P, _I64, _I, _P, _P], _I),
    "logo_sq_fwd": ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P, _SZ, _P], _I),
    "logo_sq_workspace_bytes": ([_I64, _I, _I, _I], _SZ),
    "logo_sq_generic": ([_I, _I], _I),
    "logo_read_calibration": ([_P, _SZ, _P, _I, _I, _P], _I),
    "logo_sq_workspace_counter_bytes": ([], _SZ),
    "logo_epilogue_fwd": ([_P, _P, _P, _P, _I, _P, _P, _P, _I64, _I, _I, _F, _I, _P], _I),
    "logo_epilogue_bwd_workspace_bytes": ([_I64, _I, _I], _SZ),
    "logo_epilogue_bwd": ([_P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I, _I, _F, _P, _I, _P],
                          _I),
    "logo_decode_workspace_bytes": ([_I, _I, _I, _I], _SZ),
    "logo_decode_attn": ([_P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _I64, _I, _F, _I, _P], _I),
    "logo_head_linear": ([_P, _I64, _P, _P, _I64, _I64, _I, _I, _I, _I, _P], _I),
    "logo_head_linear_dw_workspace_bytes": ([_I64, _I, _I], _SZ),
    "logo_head_linear_dw": ([_P, _I64, _P, _I64, _P, _P, _I64, _I, _I, _I, _P], _I),
    "logo_head_linear_grad_acc": ([_P, _I64, _P, _P, _I64, _P, _I64, _I64, _I, _I, _I, _P], _I),
    "logo_decode_fused_workspace_bytes": ([_I, _I, _I, _I], _SZ),
    "logo_decode_attn_fused": ([_P, _P, _P, _P, _I64, _I, _P, _P, _P, _P, _I64, _I, _P, _P, _I, _P, _P, _F, _P, _P, _I,
                                _I, _I, _I, _F, _I, _P], _I),
    "logo_cache_append": ([_P, _P, _P, _P, _P, _I, _I, _I, _I64, _I, _I, _P], _I),
    "logo_rope_apply": ([_P, _I, _P, _I, _P, _I, _P, _I, _P, _P, _I64, _I, _I, _P], _I),
    "logo_rope": ([_P, _P, _I, _P, _P, _I, _P, _P, _I, _P, _P, _I, _P, _P, _I64, _I, _I, _I, _P], _I),
    "logo_rmsnorm": ([_P, _P, _P, _I64, _I, _F, _I, _P], _I),
    "logo_add_rmsnorm": ([_P, _P, _P, _P, _P, _I64, _I, _F, _I, _P], _I),
    "logo_silu_mul": ([_P, _I64, _P, _I64, _I, _I, _P], _I),
    "logo_head_proj": ([_P, _P, _P, _I, _P, _P, _P, _I, _P, _P, _P, _I, _I, _I, _I, _I, _P], _I),
    "logo_decode_qkv": ([_P, _I64, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _P, _I, _I, _I, _I, _I, _I64,
                         _I, _P],
                        _I),
}
_BWD = ([_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I64, _I, _I, _I, _I, _I, _I, _F, _I, _I, _P,
         _SZ, _P], _I)
for _name in ("logo_sq_bwd", "logo_sq_bwd_delta", "logo_sq_bwd_dq", "logo_sq_bwd_dkv", "logo_sq_bwd_dqkv"):
    SIGNATURES[_name] = _BWD

# Library constants (include/logo_hip.h).
BQ = 128
BKV = 128
META_HDR = 8
DTYPE_BF16 = 0
DTYPE_F32 = 1
DTYPE_F16 = 2


def thres_arg(thres: torch.Tensor):
    """(pointer, dtype code) of a one-element threshold tensor, read in place
    when it is bf16 or fp32 (no conversion launch)."""
    t = thres.detach().reshape(1)
    if t.dtype not in (torch.bfloat16, torch.float32):
        t = t.to(torch.float32)
    t = t.contiguous()
    return t, (DTYPE_BF16 if t.dtype == torch.bfloat16 else DTYPE_F32)


def meta_stride(nseq: int) -> int:
    return META_HDR + 3 * (nseq + 1)


_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m logo_amd.build`. "
                "The LoGo HIP ops have no CPU fallback.")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = res
        _lib = handle
    return _lib


def header_symbols():
    """Function names declared in include/logo_hip.h."""
    with open(HEADER_PATH) as f:
        text = f.read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(logo_[a-z0-9_]+)\s*\(", text)))


def check(rc: int, what: str) -> None:
    if rc != 0:
        msg = lib().logo_last_error().decode(errors="replace")
        raise RuntimeError(f"{what} failed (code {rc}): {msg}")


def ptr(t):
    """Device pointer of a tensor (None -> NULL)."""
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


# Optional per-launch timing hook: called as hook(name, "start"|"end") around
# every kernel launch of the ops (bench.py records HIP events through it).
_launch_hook = None


def set_launch_hook(hook):
    global _launch_hook
    _launch_hook = hook


def launch(name: str, fn, *args):
    """Call C entry point ``fn`` (named ``name``), bracketed by the hook."""
    hook = _launch_hook
    if hook is not None:
        hook(name, "start")
    check(fn(*args), name)
    if hook is not None:
        hook(name, "end")


def require_gpu(*tensors):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(
                "logo_amd ops run only on a ROCm GPU (got a tensor on "
                f"{t.device}); there is no CPU fallback")
