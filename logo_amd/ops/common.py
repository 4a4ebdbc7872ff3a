"""Selection metadata and comparison helpers.

Mirrors logo/ops/common.py (``SelInfo`` :44-68, ``build_selection`` :71-107,
``get_abs_err`` / ``get_err_ratio`` / ``assert_close`` :24-41).  The
compaction itself runs in the HIP kernels of ``csrc/compact.hip``; nothing
here computes on the CPU.
"""

from dataclasses import dataclass, field
from typing import Optional

import torch

from .. import _lib, _torch_ops

__all__ = [
    "SelInfo",
    "DeviceSelection",
    "build_selection",
    "compact_selection",
    "dense_selection",
    "prepare_chunk_indices",
    "compute_q_start_blk",
    "get_abs_err",
    "get_err_ratio",
    "assert_close",
]


def get_abs_err(x, y):
    """Max absolute difference (logo/ops/common.py:24-25)."""
    return (x.detach() - y.detach()).flatten().abs().max().item()


def get_err_ratio(x, y):
    """RMS error relative to the RMS of ``x`` (logo/ops/common.py:28-31)."""
    err = (x.detach() - y.detach()).flatten().square().mean().sqrt().item()
    base = (x.detach()).flatten().square().mean().sqrt().item()
    return err / (base + 1e-8)


def assert_close(prefix, ref, tri, ratio, err_atol=1e-6):
    """Pass if max-abs error <= err_atol, else require err ratio < ratio
    (logo/ops/common.py:34-41)."""
    abs_atol = get_abs_err(ref, tri)
    error_rate = get_err_ratio(ref, tri)
    msg = f"{prefix} diff: {abs_atol:.6e} ratio: {error_rate:.6e}"
    if abs_atol <= err_atol:
        return msg
    assert error_rate < ratio, msg
    return msg


@dataclass
class DeviceSelection:
    """Compaction result kept on the device (no host synchronisation).

    ``q_idx [lanes, N]`` int64 and ``pos [lanes, N]`` int32 hold the selected
    rows of each lane in entries ``[0, Sq_lane)``; ``meta`` is the int32 block
    described in include/logo_hip.h (Sq, tile counts, cu_q, tile prefixes).
    ``q_idx``/``pos`` are ``None`` for dense (every row) metadata.
    """

    meta: torch.Tensor
    cu: torch.Tensor
    q_idx: Optional[torch.Tensor]
    pos: Optional[torch.Tensor]
    n_tokens: int
    nseq: int
    lanes: int
    B: int = 1
    T: int = 0

    @property
    def dense(self) -> bool:
        return self.q_idx is None

    def lane_meta(self, lane: int = 0) -> torch.Tensor:
        st = _lib.meta_stride(self.nseq)
        return self.meta[lane * st:(lane + 1) * st]

    def cu_seqlens_q(self, lane: int = 0) -> torch.Tensor:
        m = self.lane_meta(lane)
        return m[_lib.META_HDR:_lib.META_HDR + self.nseq + 1]

    def sq(self, lane: int = 0) -> int:
        """Number of selected rows (synchronises with the host)."""
        return int(self.lane_meta(lane)[0].item())


@dataclass
class SelInfo:
    """Metadata for queries packed in sequence and position order
    (logo/ops/common.py:44-68).

    ``q_idx`` int64 [Sq], ``pos_ids`` int32 [Sq], ``cu_seqlens_q`` int32
    [Nseq+1], ``cu_seqlens_k`` int32 [Nseq+1]; ``B``, ``T``, ``Nseq``, ``Sq``.
    ``device`` keeps the untrimmed on-device compaction the kernels use.
    """

    q_idx: torch.Tensor
    pos_ids: torch.Tensor
    cu_seqlens_q: torch.Tensor
    cu_seqlens_k: torch.Tensor
    B: int
    T: int
    Nseq: int
    Sq: int
    device: Optional[DeviceSelection] = field(default=None, repr=False)


def _as_cu(cu_seqlens: torch.Tensor, device) -> torch.Tensor:
    return cu_seqlens.to(device=device, dtype=torch.int32).contiguous()


def compact_selection(selection: torch.Tensor, cu_seqlens: torch.Tensor) -> DeviceSelection:
    """Run the HIP compaction on ``selection`` ``[N]`` or ``[N, HQ]`` (bool).

    No host synchronisation: counts stay on the device inside ``meta``.
    """
    _lib.require_gpu(selection)
    dev = selection.device
    sel = selection.contiguous()
    if sel.dtype != torch.bool:
        raise TypeError("selection must be a bool tensor")
    n = sel.shape[0]
    lanes = 1 if sel.dim() == 1 else sel.shape[1]
    cu = _as_cu(cu_seqlens, dev)
    nseq = cu.numel() - 1
    if nseq < 1:
        raise ValueError("cu_seqlens must have at least two entries")
    q_idx, pos, meta = _torch_ops.timed("logo_compact", _torch_ops.ops().compact, sel, cu)
    return DeviceSelection(meta=meta, cu=cu, q_idx=q_idx, pos=pos, n_tokens=n, nseq=nseq, lanes=lanes)


def dense_selection(cu_seqlens: torch.Tensor, n_tokens: int, device) -> DeviceSelection:
    """Metadata for attention over every row (no compaction)."""
    cu = _as_cu(cu_seqlens, device)
    nseq = cu.numel() - 1
    _lib.require_gpu(cu)
    meta = _torch_ops.ops().dense_meta(cu, n_tokens)
    return DeviceSelection(meta=meta, cu=cu, q_idx=None, pos=None, n_tokens=n_tokens, nseq=nseq, lanes=1)


def build_selection(selection: torch.Tensor, B: int, T: int,
                    cu_seqlens: Optional[torch.Tensor] = None) -> SelInfo:
    """Selection metadata for packed variable-length input
    (logo/ops/common.py:71-107).

    Runs the HIP compaction and, like the reference's ``nonzero`` (:90), syncs
    once to size ``q_idx``/``pos_ids`` to ``Sq``.  ``selection`` is ``[1, T]``
    (or the per-head extension ``[1, T, HQ]``, in which case the returned
    tensors describe lane 0 and ``device`` holds every lane).
    """
    if cu_seqlens is None:
        raise AssertionError("build_selection requires explicit cu_seqlens")
    flat = selection.reshape(B * T, *selection.shape[2:])
    dsel = compact_selection(flat, cu_seqlens)
    dsel.B, dsel.T = B, T
    sq = dsel.sq(0)
    return SelInfo(
        q_idx=dsel.q_idx[0, :sq],
        pos_ids=dsel.pos[0, :sq],
        cu_seqlens_q=dsel.cu_seqlens_q(0).clone(),
        cu_seqlens_k=dsel.cu,
        B=B,
        T=T,
        Nseq=dsel.nseq,
        Sq=sq,
        device=dsel,
    )


def prepare_chunk_indices(cu_seqlens: torch.Tensor, chunk_size: int) -> torch.Tensor:
    """``[NT, 2]`` int32 (sequence id, block id) list on the device
    (logo/ops/common.py:110-124).  Syncs once to size the result."""
    _lib.require_gpu(cu_seqlens)
    cu = _as_cu(cu_seqlens, cu_seqlens.device)
    nseq = cu.numel() - 1
    n = int(cu[-1].item()) if nseq >= 1 else 0
    max_tiles = n // chunk_size + nseq + 1
    out = torch.empty(max_tiles, 2, dtype=torch.int32, device=cu.device)
    count = torch.empty(1, dtype=torch.int32, device=cu.device)
    ws = torch.empty(nseq + 1, dtype=torch.int32, device=cu.device)
    lib = _lib.lib()
    _lib.check(lib.logo_chunk_indices(_lib.ptr(cu), nseq, chunk_size, _lib.ptr(out), max_tiles,
                                      _lib.ptr(count), _lib.ptr(ws), _lib.stream_of(cu)),
               "logo_chunk_indices")
    return out[:int(count.item())]


def compute_q_start_blk(pos_ids: torch.Tensor, sel: SelInfo, chunk_indices_k: torch.Tensor,
                        BT: int) -> torch.Tensor:
    """First compacted-query block each key block can attend to
    (logo/ops/selected_full_attn.py:374-402)."""
    ntk = chunk_indices_k.shape[0]
    out = torch.empty(max(ntk, 1), dtype=torch.int32, device=chunk_indices_k.device)
    if ntk == 0:
        return out[:0]
    count = torch.tensor([ntk], dtype=torch.int32, device=chunk_indices_k.device)
    pos = pos_ids if pos_ids.numel() else torch.zeros(1, dtype=torch.int32, device=out.device)
    lib = _lib.lib()
    _lib.check(lib.logo_q_start_blk(_lib.ptr(pos.contiguous()), _lib.ptr(sel.cu_seqlens_q.contiguous()),
                                    _lib.ptr(chunk_indices_k.contiguous()), _lib.ptr(count), ntk, BT,
                                    _lib.ptr(out), _lib.stream_of(out)),
               "logo_q_start_blk")
    return out
