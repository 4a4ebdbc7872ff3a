"""Gate-aware decode attention and a preallocated LoGo KV cache.

``decode_attn`` replaces the decode branch of logo/layers/logo.py:228-249:
rows whose gate fails read no cache and return zeros, and no host
synchronisation decides it (the reference's ``active.any()`` at :230).

``LogoKVCache`` keeps the logical layout of logo/cache.py (per layer: local
K/V for the sliding window, global K/V ``[B, H, T, D]``) but preallocates the
global buffers to the maximum length and keeps the local branch as a ring of
``window + 1`` slots, so a decode step appends in place instead of
``torch.cat``-ing the whole cache (logo/cache.py:97-118).
"""

from typing import Optional

import torch

from .. import _lib, _torch_ops

__all__ = ["decode_attn", "decode_attn_fused", "cache_append", "decode_qkv", "LogoKVCache"]


def decode_attn(q, k_cache, v_cache, lens, gate=None, thres=None, max_len: Optional[int] = None,
                scale: Optional[float] = None):
    """``q [B, HQ, D]``; caches ``[B, H, T_cap, D]``; ``lens`` int32 ``[B]`` on the
    device; ``gate [B]`` (post-sigmoid) with ``thres`` (device tensor) or
    ``None`` for all rows.  ``max_len`` is a host-side bound on ``lens``
    (defaults to ``T_cap``).  Returns ``[B, HQ, D]``."""
    _lib.require_gpu(q, k_cache, v_cache, lens)
    B, HQ, D = q.shape
    H, t_cap = k_cache.shape[1], k_cache.shape[2]
    if scale is None:
        scale = D ** -0.5
    if max_len is None:
        max_len = t_cap
    th = None
    if gate is not None:
        gate = gate.contiguous().view(B)
        th, _ = _lib.thres_arg(thres)
    return _torch_ops.timed("logo_decode_attn", _torch_ops.ops().decode_attn, q.contiguous(), k_cache, v_cache,
                            lens, gate, th, int(max_len), float(scale))


def decode_attn_fused(q_local, k_local, v_local, lens_local, max_len_local: int, q_global, k_global, v_global,
                      lens_global, max_len_global: int, gate, thres, w_local, w_global, eps: float,
                      scale: Optional[float] = None):
    """Both decode branches and the fused epilogue in two launches:
    ``decode_attn`` of the local window (every row) and of the global cache
    (gate-aware), then the context norms, gate mask and fusion of
    ``logo_epilogue`` (logo/layers/logo.py:228-258), bit-identical to those
    three calls.  ``q_* [B, HQ, D]``; caches ``[B, H, T_cap, D]``; ``lens_*``
    int32 ``[B]``; ``max_len_local <= 256``; ``gate [B]`` post-sigmoid;
    ``w_* [D]`` the context-norm weights.  Returns ``[B, HQ, D]``."""
    _lib.require_gpu(q_local, k_local, v_local, lens_local, q_global, k_global, v_global, lens_global, gate)
    B, HQ, D = q_global.shape
    H = k_global.shape[1]
    if q_local.shape != q_global.shape or k_local.shape[:2] != (B, H) or k_global.shape[0] != B:
        raise ValueError("decode_attn_fused: q / cache shapes disagree")
    if w_local.numel() != D or w_global.numel() != D or w_local.dtype != torch.bfloat16 \
            or w_global.dtype != torch.bfloat16:
        raise ValueError("decode_attn_fused: context-norm weights must be bf16 [D]")
    if scale is None:
        scale = D ** -0.5
    ql, qg = q_local.contiguous(), q_global.contiguous()
    wl, wg = w_local.detach().contiguous(), w_global.detach().contiguous()
    out = torch.empty_like(qg)
    lib = _lib.lib()
    ws = torch.empty(lib.logo_decode_fused_workspace_bytes(B, HQ, D, int(max_len_global)), dtype=torch.uint8,
                     device=qg.device)
    gate = gate.contiguous().view(B)
    th, th_dt = _lib.thres_arg(thres)
    _lib.launch("logo_decode_attn_fused", lib.logo_decode_attn_fused,
                _lib.ptr(ql), _lib.ptr(k_local), _lib.ptr(v_local), _lib.ptr(lens_local), k_local.shape[2],
                int(max_len_local),
                _lib.ptr(qg), _lib.ptr(k_global), _lib.ptr(v_global), _lib.ptr(lens_global), k_global.shape[2],
                int(max_len_global),
                _lib.ptr(gate), _lib.ptr(th), th_dt, _lib.ptr(wl), _lib.ptr(wg), float(eps), _lib.ptr(out),
                _lib.ptr(ws), B, HQ, H, D, float(scale), _lib.DTYPE_BF16, _lib.stream_of(qg))
    return out


def cache_append(k_new, v_new, k_cache, v_cache, pos, ring: int = 0):
    """Write ``k_new/v_new [B, H, D]`` at position ``pos[b]`` (mod ``ring`` if > 0)."""
    B, H, D = k_new.shape
    lib = _lib.lib()
    _lib.launch("logo_cache_append", lib.logo_cache_append, _lib.ptr(k_new.contiguous()),
                _lib.ptr(v_new.contiguous()), _lib.ptr(k_cache), _lib.ptr(v_cache), _lib.ptr(pos), B, H, D,
                k_cache.shape[2], int(ring), _lib.DTYPE_BF16, _lib.stream_of(k_new))


def decode_qkv(qkv, wq, wk, wv, cos, sin, cache: "LogoKVCache", layer: int, heads: int, kv_heads: int,
               gate_col: Optional[int] = None):
    """One decode step's q / k / v transform for a LoGo layer in one launch.

    ``qkv [B, ldq]``: each token's stacked projection row ``[q | k | v | ...]``;
    ``wq/wk/wv``: the global ``linear_proj`` matrices; ``cos/sin [B, D]``.
    Appends the rotated k, v (local ring) and global k, v (global cache) at the
    cache's device position and returns the rotated q and global q
    ``[B, H, D]``; with ``gate_col`` (the gate logit's column in the row) also
    the gate ``sigmoid(qkv[:, gate_col])`` ``[B]`` as a third result."""
    _lib.require_gpu(qkv, wq, wk, wv, cos, sin)
    B = qkv.shape[0]
    D = wq.shape[-1]
    if qkv.stride(-1) != 1 or qkv.stride(0) % 8 != 0:
        raise ValueError("decode_qkv needs rows with unit column stride and 16-byte aligned row starts")
    if cache.seen >= cache.max_len:
        raise ValueError("cache is full")
    q = torch.empty(B, heads, D, dtype=torch.bfloat16, device=qkv.device)
    gq = torch.empty_like(q)
    gate = torch.empty(B, dtype=torch.bfloat16, device=qkv.device) if gate_col is not None else None
    cos = cos.reshape(B, D).contiguous()
    sin = sin.reshape(B, D).contiguous()
    lib = _lib.lib()
    _lib.launch("logo_decode_qkv", lib.logo_decode_qkv, _lib.ptr(qkv), qkv.stride(0), _lib.ptr(wq.contiguous()),
                _lib.ptr(wk.contiguous()), _lib.ptr(wv.contiguous()), _lib.ptr(cos), _lib.ptr(sin),
                _lib.ptr(cache._pos), _lib.ptr(q), _lib.ptr(gq), _lib.ptr(cache.local_k[layer]),
                _lib.ptr(cache.local_v[layer]), _lib.ptr(cache.global_k[layer]), _lib.ptr(cache.global_v[layer]),
                int(gate_col) if gate_col is not None else 0, _lib.ptr(gate), B, heads, kv_heads, D, cache.ring,
                cache.max_len, _lib.DTYPE_BF16, _lib.stream_of(qkv))
    return (q, gq) if gate is None else (q, gq, gate)


class LogoKVCache:
    """Preallocated per-layer cache: global ``[B, H, max_len, D]`` and a local ring
    ``[B, H, window + 1, D]`` (all rows of a batch share one length)."""

    def __init__(self, num_layers: int, batch: int, kv_heads: int, head_dim: int, max_len: int,
                 window: int = 128, dtype=torch.bfloat16, device=None):
        self.window = window
        self.ring = window + 1
        self.max_len = max_len
        shape_g = (batch, kv_heads, max_len, head_dim)
        shape_l = (batch, kv_heads, self.ring, head_dim)
        self.global_k = [torch.empty(shape_g, dtype=dtype, device=device) for _ in range(num_layers)]
        self.global_v = [torch.empty(shape_g, dtype=dtype, device=device) for _ in range(num_layers)]
        self.local_k = [torch.empty(shape_l, dtype=dtype, device=device) for _ in range(num_layers)]
        self.local_v = [torch.empty(shape_l, dtype=dtype, device=device) for _ in range(num_layers)]
        self.seen = 0
        self.batch = batch
        self._pos = torch.zeros(batch, dtype=torch.int32, device=device)
        self._len_g = torch.zeros(batch, dtype=torch.int32, device=device)
        self._len_l = torch.zeros(batch, dtype=torch.int32, device=device)
        self._step = 0        # host count of position changes
        self._lens_for = -1   # step whose lengths _len_g / _len_l hold

    def get_seq_length(self) -> int:
        return self.seen

    def prefill(self, layer: int, k_local, v_local, k_global, v_global, keep=None):
        """Store a prompt's K/V (``[B, H, T, D]``) for one layer, at positions
        [0, T).  Only an empty cache takes a prompt: the prefill attends to the
        prompt alone, so a second chunk on top of cached tokens would lose them
        (``reset()`` empties the cache for a new prompt).

        ``keep`` (bool ``[B, T]``, a padding mask): each row stores its kept
        tokens only, in order, at positions [0, n_b) -- the reference keeps the
        padded positions and masks them out of every decode step
        (logo/layers/logo.py:162-176, :230-244 with logo/layers/utils.py:44-81),
        which attends the same keys; ``set_lengths`` then records the per-row
        counts."""
        if self.seen > 0:
            raise ValueError(
                f"prefill into a cache that already holds {self.seen} tokens: a multi-token forward "
                "attends to its own tokens only; call reset() or use a new cache for a new prompt")
        T = k_global.shape[2]
        if T > self.max_len:
            raise ValueError(f"prompt of {T} tokens exceeds the cache's {self.max_len}")
        if keep is not None:
            keep = keep.to(k_global.device).bool()
            for b in range(k_global.shape[0]):
                idx = torch.nonzero(keep[b]).flatten()
                self._store_rows(layer, slice(b, b + 1), *(x[b:b + 1].index_select(2, idx)
                                                          for x in (k_local, v_local, k_global, v_global)))
            return
        self._store_rows(layer, slice(None), k_local, v_local, k_global, v_global)

    def _store_rows(self, layer, rows, k_local, v_local, k_global, v_global):
        """Positions [0, T) of batch ``rows``: the global cache, and the last
        ``ring`` positions into the local ring at slot ``p % ring``."""
        T = k_global.shape[2]
        self.global_k[layer][rows, :, :T].copy_(k_global)
        self.global_v[layer][rows, :, :T].copy_(v_global)
        lo = max(0, T - self.ring)
        for p0 in range(lo, T, self.ring):
            p1 = min(T, p0 + self.ring)
            s0 = p0 % self.ring
            n = p1 - p0
            first = min(n, self.ring - s0)
            self.local_k[layer][rows, :, s0:s0 + first].copy_(k_local[:, :, p0:p0 + first])
            self.local_v[layer][rows, :, s0:s0 + first].copy_(v_local[:, :, p0:p0 + first])
            if first < n:
                self.local_k[layer][rows, :, :n - first].copy_(k_local[:, :, p0 + first:p1])
                self.local_v[layer][rows, :, :n - first].copy_(v_local[:, :, p0 + first:p1])

    def reset(self):
        """Empty the cache (host and device positions back to 0)."""
        self.set_length(0)

    def set_length(self, seen: int):
        """Record that ``seen`` tokens are cached (host value; e.g. after a prefill)."""
        self.seen = seen
        self._pos.fill_(seen)
        self._step += 1

    def set_lengths(self, lengths):
        """Per-row cached token counts (after a prefill with a padding mask);
        the host ``seen`` becomes the largest, the bound for kernel grids."""
        lengths = torch.as_tensor(lengths).to(device=self._pos.device, dtype=torch.int32).reshape(self.batch)
        self._pos.copy_(lengths)
        self.seen = int(lengths.max())
        self._step += 1

    def advance_device(self):
        """Move the device-side position one token on (no host value involved,
        so a captured decode step can replay it); ``seen`` is the caller's
        to update."""
        self._pos.add_(1)
        self._step += 1

    def advance(self):
        """One decoded token: device position and host ``seen``."""
        self.advance_device()
        self.seen += 1

    def positions(self, T: int = 1):
        """Positions ``[B, T]`` of the next ``T`` tokens, from the device state."""
        return self._pos[:, None].to(torch.int64) + torch.arange(T, device=self._pos.device)

    def append(self, layer: int, k_local, v_local, k_global, v_global):
        """Append the new token (``[B, H, D]`` each) at position ``seen``."""
        if self.seen >= self.max_len:
            raise ValueError("cache is full")
        cache_append(k_global, v_global, self.global_k[layer], self.global_v[layer], self._pos)
        cache_append(k_local, v_local, self.local_k[layer], self.local_v[layer], self._pos, ring=self.ring)

    def lengths(self):
        """(global length, local length) device tensors for the token at the
        device position (computed on the device)."""
        torch.add(self._pos, 1, out=self._len_g)
        torch.clamp(self._len_g, max=self.ring, out=self._len_l)
        self._lens_for = self._step
        return self._len_g, self._len_l

    def step_lengths(self):
        """``lengths()`` computed once per decode step and shared by the layers."""
        if self._lens_for != self._step:
            return self.lengths()
        return self._len_g, self._len_l

    def length_bounds(self):
        """Host-side bounds on (global, local) lengths for kernel grids: tight
        in eager mode, the capacity while a decode step is being captured (the
        device lengths then grow across replays)."""
        if torch.cuda.is_current_stream_capturing():
            return self.max_len, self.ring
        n = self.seen + 1
        return n, min(n, self.ring)
