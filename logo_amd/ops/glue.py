"""Fused RoPE and RMSNorm launches (``csrc/glue.hip``) for the layer and model glue.

``rope_apply_`` rotates q, k and the global q, k in one launch with the eager
bf16 rounding of logo/modules/rotary.py:81-106; ``rms_norm`` computes
logo/modules/layernorm.py:17-22 in one launch.  Both run only on ROCm tensors
and raise otherwise (the modules that call them keep plain torch math for CPU
tensors).
"""

import torch

from .. import _lib

__all__ = ["rope_apply_", "rms_norm"]


def rope_apply_(tensors, cos, sin):
    """Rotate each ``[..., T, H_i, D]`` bf16 tensor of ``tensors`` (up to four,
    contiguous, all with the same leading ``[..., T]``) in place with
    ``cos/sin [..., T, D]``."""
    tensors = [t for t in tensors if t is not None]
    if not 1 <= len(tensors) <= 4:
        raise ValueError("rope_apply_ takes one to four tensors")
    _lib.require_gpu(*tensors, cos, sin)
    D = tensors[0].shape[-1]
    n = tensors[0][..., 0, 0].numel()
    for t in tensors:
        if t.dtype != torch.bfloat16 or not t.is_contiguous() or t.shape[-1] != D or t[..., 0, 0].numel() != n:
            raise ValueError("rope_apply_ needs contiguous bf16 [..., T, H, D] tensors of one shape prefix")
    cos = cos.to(torch.bfloat16).contiguous()
    sin = sin.to(torch.bfloat16).contiguous()
    if cos.numel() != n * D or sin.numel() != n * D:
        raise ValueError("cos / sin must be [..., T, D] matching the tensors")
    args = []
    for i in range(4):
        if i < len(tensors):
            args += [_lib.ptr(tensors[i]), tensors[i].shape[-2]]
        else:
            args += [None, 0]
    lib = _lib.lib()
    _lib.launch("logo_rope_apply", lib.logo_rope_apply, *args, _lib.ptr(cos), _lib.ptr(sin), n, D,
                _lib.DTYPE_BF16, _lib.stream_of(tensors[0]))
    return tensors


def rms_norm(x, weight, eps):
    """RMSNorm over the last dimension of bf16 ``x`` with bf16 ``weight``."""
    _lib.require_gpu(x, weight)
    if x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16:
        raise ValueError("rms_norm takes bf16 tensors")
    xc = x.contiguous()
    cols = xc.shape[-1]
    y = torch.empty_like(xc)
    lib = _lib.lib()
    _lib.launch("logo_rmsnorm", lib.logo_rmsnorm, _lib.ptr(xc), _lib.ptr(weight.contiguous()), _lib.ptr(y),
                xc.numel() // cols, cols, float(eps), _lib.DTYPE_BF16, _lib.stream_of(xc))
    return y
