"""Gate-threshold budget controller (counterpart of logo/update.py:17-75).

``update_gate_thres`` nudges every LoGo layer's ``gate_thres`` by
``update_rate * sign(ratio - target)``, where ``ratio`` is the fraction of
tokens the layer sent to global attention since the last call, then clears
the layer's counters.  Same signature, argument checks, return value (the
per-layer ratios ``[L, 1]``, or ``None`` for a model with no LoGo layer) and
``GATE_THRES_UPDATE_RATE`` / ``TARGET_GLOBAL_RATIO`` environment defaults as
the reference.

Differences in structure, not in results:
  * the global and total token counts of all layers travel in ONE
    ``all_reduce`` of a stacked ``[L, 2]`` fp32 tensor (the reference issues
    two, :52-54): one latency-bound collective per update instead of two;
  * everything stays on the counters' device: no host synchronisation;
  * a ``gloo`` process group gets a host copy of the counters (gloo
    collectives take CPU tensors), an RCCL (``nccl``) group the device tensor.
The counters themselves are kept in fp32 by ``LoGoAttention`` (the
reference's become bf16 after ``model.to(bf16)`` and stop counting exactly
above 256 tokens), so ``ratio`` is the exact fraction; the threshold step is
taken in the threshold's own dtype, as the reference's ``add_`` is.
"""

import os
from typing import Optional

import torch
import torch.distributed as dist

__all__ = ["update_gate_thres", "GATE_THRES_UPDATE_RATE", "TARGET_GLOBAL_RATIO"]

GATE_THRES_UPDATE_RATE = float(os.getenv("GATE_THRES_UPDATE_RATE", "0.0005"))
TARGET_GLOBAL_RATIO = float(os.getenv("TARGET_GLOBAL_RATIO", "0.5"))

_COUNTERS = ("gate_thres", "gate_avg", "global_token_count", "total_token_count")


def _all_reduce_sum(t: torch.Tensor, group) -> torch.Tensor:
    if dist.get_backend(group) == dist.Backend.GLOO and t.device.type != "cpu":
        host = t.cpu()  # synchronous copy: gloo reduces host memory
        dist.all_reduce(host, op=dist.ReduceOp.SUM, group=group)
        return host.to(t.device)
    dist.all_reduce(t, op=dist.ReduceOp.SUM, group=group)
    return t


def update_gate_thres(
    model,
    target_global_ratio: float = TARGET_GLOBAL_RATIO,
    update_rate: float = GATE_THRES_UPDATE_RATE,
    process_group=None,
) -> Optional[torch.Tensor]:
    """Update every LoGo layer's gate threshold from its accumulated
    global-token ratio (logo/update.py:17-75)."""
    if not 0.0 <= target_global_ratio <= 1.0:
        raise ValueError(f"`target_global_ratio` must be in [0, 1], got {target_global_ratio}")
    if update_rate < 0.0:
        raise ValueError(f"`update_rate` must be non-negative, got {update_rate}")

    layers = [m for m in model.modules() if all(hasattr(m, n) for n in _COUNTERS)]
    if not layers:
        return None

    with torch.no_grad():
        counts = torch.stack([torch.cat([m.global_token_count.float().reshape(1),
                                         m.total_token_count.float().reshape(1)]) for m in layers])  # [L, 2]
        if dist.is_available() and dist.is_initialized():
            counts = _all_reduce_sum(counts, process_group)
        global_count, total_count = counts[:, :1], counts[:, 1:]
        has_obs = total_count > 0
        ratio = torch.where(has_obs, global_count / total_count.clamp_min(1), torch.zeros_like(global_count))
        step = update_rate * torch.sign(ratio - target_global_ratio)
        step = torch.where(has_obs, step, torch.zeros_like(step))
        for li, m in enumerate(layers):
            m.gate_thres.add_(step[li].to(m.gate_thres.dtype))
            m.gate_avg.zero_()
            m.global_token_count.zero_()
            m.total_token_count.zero_()
    return ratio
