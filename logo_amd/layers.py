"""LoGo attention layer on the HIP hot path (caller side of ``sq_full_attn``).

Counterpart of ``LoGoAttention`` (logo/layers/logo.py:34-262), with the same
parameter names and config knobs, so a reference state dict loads unchanged.
The hot path (local SWA, query-sparse or dense global attention, the fused
gate / context-norm / fusion epilogue, gate-aware decode) runs on this
package's HIP kernels, and so do RoPE, the per-head global re-parameterisation
and, at decode, the transform, gate and cache appends; the dense projections
are hipBLASLt GEMMs through torch.

Differences in structure (not in results): tensors stay in ``[B, T, H, D]``
(no ``transpose(1, 2).contiguous()`` round trips, :121-158); equal-length
batches are packed into ``[1, B*T]`` for every branch, as the reference does
for its sparse branch (:199-209); decode reads a preallocated ``LogoKVCache``.

``sparse_full_attn_backend``: ``"triton"`` (the reference's name, kept so
configs load) and ``"hip"`` select the query-sparse kernel; ``"flash"``
selects dense causal global attention on the same kernels
(logo/configuration_logo.py:170-173, logo/layers/logo.py:185-224).
"""

import math
from dataclasses import dataclass, field
from typing import List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .ops.decode import LogoKVCache, decode_attn, decode_attn_fused, decode_qkv
from .ops.epilogue import logo_epilogue
from .ops.glue import attn_inputs, head_linear, head_proj, rms_norm, rope, rope_apply_
from .ops.sq_attn import dense_causal_attn, sq_full_attn, swa_attn

__all__ = ["LoGoConfig", "LoGoAttention", "Attention", "RMSNorm", "rope_cos_sin", "apply_rope", "position_ids_for"]

SPARSE_BACKENDS = ("triton", "hip")


@dataclass
class LoGoConfig:
    """The LoGo knobs of logo/configuration_logo.py:86-183 that this path uses."""

    vocab_size: int = 32000
    hidden_size: int = 2048
    intermediate_size: int = 5632
    num_hidden_layers: int = 24
    num_attention_heads: int = 16
    num_key_value_heads: Optional[int] = None
    rms_norm_eps: float = 1e-5
    rope_theta: float = 10000.0
    attention_bias: bool = False
    attention_out_bias: bool = False
    initializer_range: float = 0.02
    tie_word_embeddings: bool = True
    attn_type_list: Optional[List[int]] = None
    window_size: int = 128
    global_qk_param: str = "linear_proj"
    sparse_full_attn_backend: str = "hip"
    gate_thres_init: float = 0.5
    use_context_norm: bool = True

    def __post_init__(self):
        if self.num_key_value_heads is None:
            self.num_key_value_heads = self.num_attention_heads
        if self.attn_type_list is None:
            self.attn_type_list = [0] * self.num_hidden_layers
        if self.global_qk_param not in ("scale_offset", "linear_proj"):
            raise ValueError(f"`global_qk_param` must be 'scale_offset' or 'linear_proj', got {self.global_qk_param!r}")
        if self.sparse_full_attn_backend not in ("flash", "triton", "hip"):
            raise ValueError("`sparse_full_attn_backend` must be 'flash', 'triton' or 'hip', "
                             f"got {self.sparse_full_attn_backend!r}")
        if len(self.attn_type_list) != self.num_hidden_layers:
            raise ValueError("`attn_type_list` must have length num_hidden_layers")

    @property
    def head_dim(self) -> int:
        return self.hidden_size // self.num_attention_heads


class RMSNorm(nn.Module):
    """RMSNorm with the reference's rounding order (logo/modules/layernorm.py:9-22)."""

    def __init__(self, hidden_size: int, eps: float = 1e-6):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(hidden_size))
        self.variance_epsilon = eps

    def forward(self, x):
        if _fused_ok(x, self.weight):  # one HIP launch (inference on ROCm tensors)
            return rms_norm(x, self.weight, self.variance_epsilon)
        dt = x.dtype
        xf = x.to(torch.float32)
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.variance_epsilon)
        return self.weight * xf.to(dt)


def _fused_ok(*tensors) -> bool:
    """The fused glue kernels (no autograd) serve bf16 ROCm tensors that need
    no gradient; anything else takes the plain torch ops."""
    if any(t.requires_grad for t in tensors) and torch.is_grad_enabled():
        return False
    return all(t.is_cuda and t.dtype == torch.bfloat16 for t in tensors)


def position_ids_for(B: int, T: int, device, cu_seqlens=None, cache: Optional[LogoKVCache] = None):
    """Positions ``[B, T]`` of the tokens being processed: restarting at every
    packed segment (logo/modeling_logo.py:207-222), continuing a cache, or from
    zero.  A one-token decode step reads the cache's device position (no host
    value, so the step can be captured in a graph)."""
    if cu_seqlens is not None:
        idx = torch.arange(B * T, device=device)
        cu64 = cu_seqlens.to(device=device, dtype=torch.int64)
        seg = torch.searchsorted(cu64, idx, right=True) - 1
        return (idx - cu64[seg]).view(B, T)
    if cache is not None and T == 1:
        return cache.positions(T)
    start = cache.get_seq_length() if cache is not None else 0
    return torch.arange(start, start + T, device=device)[None].expand(B, T)


def rope_cos_sin(positions: torch.Tensor, head_dim: int, theta: float, dtype):
    """cos/sin ``[..., head_dim]`` computed in fp32, cast to ``dtype``
    (logo/modules/rotary.py:58-78, default rope type)."""
    inv_freq = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=positions.device, dtype=torch.float32) / head_dim))
    freqs = positions.to(torch.float32)[..., None] * inv_freq
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def apply_rope(x, cos, sin):
    """``x [..., T, H, D]`` with ``cos/sin [..., T, D]`` (logo/modules/rotary.py:81-106)."""
    cos = cos.unsqueeze(-2)
    sin = sin.unsqueeze(-2)
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return x * cos + rot * sin


def _rope_all(tensors, cos, sin):
    """RoPE of ``[B, T, H_i, D]`` tensors with one cos / sin: one in-place HIP
    launch when no gradient is needed, one launch each way under autograd,
    the eager ops for tensors that are not contiguous bf16 ROCm tensors."""
    tensors = list(tensors)
    on_dev = all(t.is_cuda and t.dtype == torch.bfloat16 for t in (*tensors, cos, sin)) and all(
        t.is_contiguous() for t in tensors)
    if on_dev and _fused_ok(*tensors):
        return rope_apply_(tensors, cos, sin)
    if on_dev:
        return rope(tensors, cos, sin)
    return [apply_rope(t, cos, sin) for t in tensors]


def _cos_sin(layer, B, T, device, dtype, position_ids, cu_seqlens, cache, position_embeddings):
    if position_embeddings is not None:
        return position_embeddings
    if position_ids is None:
        position_ids = position_ids_for(B, T, device, cu_seqlens, cache)
    return rope_cos_sin(position_ids, layer.head_dim, layer.config.rope_theta, dtype)


def _pack_cu(B, T, cu_seqlens, device):
    """Packed ``[1, B*T]`` segments: the given ``cu_seqlens`` (for ``B == 1``)
    or one segment per batch row (logo/layers/logo.py:199-209)."""
    if cu_seqlens is None:
        return torch.arange(0, (B + 1) * T, T, dtype=torch.int32, device=device)
    assert B == 1, "cu_seqlens requires packed [1, N] input"
    return cu_seqlens.to(torch.int32)


class VarlenPlan:
    """How the flash-attention branches see a ``[B, T]`` batch
    (logo/layers/utils.py:136-226): packed segments ``cu`` over the kept
    tokens, and ``keep`` -- the flat indices of the kept tokens when a padding
    mask drops some (None: every token, in order)."""

    def __init__(self, cu: torch.Tensor, keep: Optional[torch.Tensor] = None):
        self.cu, self.keep = cu, keep

    def pack(self, x):
        """``[B, T, H, D]`` -> ``[1, N_kept, H, D]``."""
        flat = x.reshape(-1, x.shape[-2], x.shape[-1])
        return (flat if self.keep is None else flat.index_select(0, self.keep))[None]

    def unpack(self, y, B: int, T: int):
        """``[1, N_kept, H, D]`` -> ``[B, T, H, D]``, dropped tokens zero (pad_input).
        A reshape, not ``y[0]``: the backward of an index allocates a zero
        ``[1, N, H, D]`` gradient and copies into it."""
        y = y.reshape(y.shape[1:])
        if self.keep is None:
            return y.view(B, T, y.shape[-2], y.shape[-1])
        out = y.new_zeros(B * T, y.shape[-2], y.shape[-1])
        return out.index_copy(0, self.keep, y).view(B, T, y.shape[-2], y.shape[-1])


def padding_mask(attention_mask: Optional[torch.Tensor]) -> Optional[torch.Tensor]:
    """A 2-D padding mask only when it masks something (logo/layers/utils.py:144,
    logo/modeling_logo.py:293-305), as bool."""
    if attention_mask is None:
        return None
    mask = attention_mask.bool()
    return mask if not bool(mask.all()) else None


def varlen_plan(B: int, T: int, device, cu_seqlens=None, attention_mask=None, position_ids=None) -> VarlenPlan:
    """The segments the local (and "flash" global) branch attends within, in
    the reference's order of precedence (logo/layers/utils.py:155-226):
    explicit ``cu_seqlens``; else a 2-D padding mask (its kept tokens, one
    segment per batch row, :180-201); else ``position_ids`` that restart
    (a new segment at every position 0, :84-104, :203-224); else one segment per
    batch row.  Host syncs on the mask / position values, as the reference's."""
    if cu_seqlens is not None:
        assert B == 1, "cu_seqlens requires packed [1, N] input"
        return VarlenPlan(cu_seqlens.to(device=device, dtype=torch.int32))
    mask = padding_mask(attention_mask)
    if mask is not None:
        mask = mask.to(device).reshape(B, -1)[:, -T:]
        keep = torch.nonzero(mask.flatten()).flatten()
        cu = F.pad(torch.cumsum(mask.sum(-1, dtype=torch.int32), 0, dtype=torch.int32), (1, 0))
        return VarlenPlan(cu, keep)
    if position_ids is not None and T != 1:
        pid = position_ids.to(device).reshape(-1, T).expand(B, T)
        if not bool((torch.diff(pid, dim=-1) >= 0).all()):
            flat = pid.flatten()
            starts = torch.nonzero(flat == 0).flatten().to(torch.int32)
            n = torch.tensor([B * T], dtype=torch.int32, device=device)
            if starts.numel() == 0 or int(starts[0]) != 0:
                starts = torch.cat([torch.zeros(1, dtype=torch.int32, device=device), starts])
            return VarlenPlan(torch.cat([starts, n]))
    return VarlenPlan(_pack_cu(B, T, None, device))


def _per_head_linear(x, w):
    """``x [..., H, D] @ w [H, D, E]`` per head.  bf16 ROCm tensors with square
    per-head maps take the HIP kernels, which read and write the ``[..., H,
    D]`` layout in place (forward, input and weight gradients); anything else
    one batched GEMM over heads (both operands contiguous: bf16 batched
    products are only used with contiguous right operands here)."""
    lead = x.shape[:-2]
    H, D = x.shape[-2], x.shape[-1]
    wgrad = w.requires_grad and torch.is_grad_enabled()
    if (x.is_cuda and x.dtype == torch.bfloat16 and w.dtype == torch.bfloat16 and tuple(w.shape) == (H, D, D)
            and (D == 128 or (D == 64 and not wgrad))):
        return head_linear(x, w)
    xh = x.reshape(-1, H, D).transpose(0, 1).contiguous()  # [H, N, D]
    y = torch.bmm(xh, w.to(x.dtype).contiguous())  # [H, N, E]
    return y.transpose(0, 1).reshape(*lead, H, w.shape[-1]).contiguous()


class LoGoAttention(nn.Module):
    """Token-level dynamic local-global attention (logo/layers/logo.py:34-262)."""

    def __init__(self, config: LoGoConfig, layer_idx: int = 0):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.hidden_size = config.hidden_size
        self.num_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        self.q_proj = nn.Linear(self.hidden_size, self.num_heads * self.head_dim, bias=config.attention_bias)
        self.k_proj = nn.Linear(self.hidden_size, self.num_key_value_heads * self.head_dim, bias=config.attention_bias)
        self.v_proj = nn.Linear(self.hidden_size, self.num_key_value_heads * self.head_dim, bias=config.attention_bias)
        self.o_proj = nn.Linear(self.hidden_size, self.hidden_size, bias=config.attention_out_bias)
        self.local_window_size = config.window_size
        self.global_qk_param = config.global_qk_param
        H, HK, D = self.num_heads, self.num_key_value_heads, self.head_dim
        if self.global_qk_param == "scale_offset":
            self.q_global_scale = nn.Parameter(torch.ones(H * D))
            self.q_global_offset = nn.Parameter(torch.zeros(H * D))
            self.k_global_scale = nn.Parameter(torch.ones(HK * D))
            self.k_global_offset = nn.Parameter(torch.zeros(HK * D))
            self.v_global_scale = nn.Parameter(torch.ones(HK * D))
            self.v_global_offset = nn.Parameter(torch.zeros(HK * D))
        else:
            eye = torch.eye(D)
            self.q_global_proj = nn.Parameter(eye.repeat(H, 1, 1))
            self.k_global_proj = nn.Parameter(eye.repeat(HK, 1, 1))
            self.v_global_proj = nn.Parameter(eye.repeat(HK, 1, 1))
        self.gate_proj = nn.Linear(self.hidden_size, 1, bias=False)
        self.use_context_norm = config.use_context_norm
        if self.use_context_norm:
            self.context_norm_local = RMSNorm(D, eps=config.rms_norm_eps)
            self.context_norm_global = RMSNorm(D, eps=config.rms_norm_eps)
        self.sparse_full_attn_backend = config.sparse_full_attn_backend
        self.register_buffer("gate_thres", torch.full((1,), config.gate_thres_init))
        # counters kept in fp32 even in a bf16 model (the reference's become bf16
        # and lose integer precision above 256, logo/layers/logo.py:74-76)
        self.register_buffer("gate_avg", torch.zeros(1, dtype=torch.float32), persistent=False)
        self.register_buffer("global_token_count", torch.zeros(1, dtype=torch.float32), persistent=False)
        self.register_buffer("total_token_count", torch.zeros(1, dtype=torch.float32), persistent=False)

    def _apply(self, fn, recurse=True):
        out = super()._apply(fn, recurse)
        for name in ("gate_avg", "global_token_count", "total_token_count"):
            buf = getattr(self, name)
            if buf.dtype != torch.float32:
                setattr(self, name, buf.float())
        return out

    def _global_qkv(self, q, k, v):
        """Global re-parameterisation on ``[B, T, H, D]`` (logo/layers/logo.py:80-94)."""
        if self.global_qk_param == "scale_offset":
            sh = lambda x, s, o: x * s.view(x.shape[-2], x.shape[-1]) + o.view(x.shape[-2], x.shape[-1])
            return (sh(q, self.q_global_scale, self.q_global_offset),
                    sh(k, self.k_global_scale, self.k_global_offset),
                    sh(v, self.v_global_scale, self.v_global_offset))
        ws = (self.q_global_proj, self.k_global_proj, self.v_global_proj)
        n_tok = q.shape[0] * q.shape[1]
        if n_tok <= 64 and _fused_ok(q, k, v, *ws) and q.shape[-1] <= 128:
            # decode sizes: one launch for the three projections
            return tuple(head_proj((q, k, v), ws))
        return (_per_head_linear(q, self.q_global_proj), _per_head_linear(k, self.k_global_proj),
                _per_head_linear(v, self.v_global_proj))

    def _fused_inputs_ok(self, hidden_states) -> bool:
        """Training-size bf16 calls of the linear_proj form take the one-node
        projections (q, k, v, gate) + global maps + RoPE (``attn_inputs``; cos
        / sin must be ``[B, T, D]`` bf16 too): its backward sums the gradient
        pairs of q, k, v and the four of h inside its own launches."""
        if self.global_qk_param == "scale_offset" or not torch.is_grad_enabled():
            return False
        B, T, _ = hidden_states.shape
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, self.gate_proj.weight, self.q_global_proj,
              self.k_global_proj, self.v_global_proj)
        return (self.head_dim == 128 and B * T > 64
                and all(t.is_cuda and t.dtype == torch.bfloat16 for t in (hidden_states, *ws)))

    def _fuse(self, local, glob, gate):
        """Context norms + gate mask + fusion; ``local/glob [B, T, H, D]``."""
        if self.use_context_norm:
            return logo_epilogue(local, glob, gate, self.gate_thres, self.context_norm_local.weight,
                                 self.context_norm_global.weight, self.context_norm_local.variance_epsilon)
        g = gate.masked_fill(gate < self.gate_thres, 0.0)
        B, T = local.shape[:2]
        return ((1 - g) * local.reshape(B, T, -1) + g * glob.reshape(B, T, -1))

    def _decode_weight(self):
        """The q, k, v and gate projection weights stacked for one decode GEMM
        (gate row then zero rows up to a multiple of 8, so every stacked row
        starts 16-byte aligned), rebuilt when a weight changes."""
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, self.gate_proj.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype) for w in ws)
        cached = getattr(self, "_decode_w", None)
        if cached is None or cached[0] != key:
            pad = (-sum(w.shape[0] for w in ws)) % 8
            stacked = torch.cat([w.detach() for w in ws]
                                + [ws[0].new_zeros(pad, ws[0].shape[1])]).contiguous()
            self._decode_w = (key, stacked)
        return self._decode_w[1]

    def _fused_decode_ok(self, hidden_states, past_key_value):
        if past_key_value is None or hidden_states.shape[1] != 1 or self.global_qk_param != "linear_proj":
            return False
        if self.q_proj.bias is not None or self.k_proj.bias is not None or self.v_proj.bias is not None:
            return False
        ws = (self.q_proj.weight, self.k_proj.weight, self.v_proj.weight, self.gate_proj.weight,
              self.q_global_proj, self.k_global_proj, self.v_global_proj)
        return self.head_dim in (64, 128) and _fused_ok(hidden_states, *ws)

    def _decode_fused(self, hidden_states, cache: LogoKVCache, position_embeddings, position_ids):
        """Decode step with the stacked q / k / v / gate GEMM and one launch for
        the global projections, RoPE and cache appends (same arithmetic as the
        step-by-step path: the same roundings, in the same order)."""
        B = hidden_states.shape[0]
        H, HK, D = self.num_heads, self.num_key_value_heads, self.head_dim
        qkv = F.linear(hidden_states, self._decode_weight()).view(B, -1)
        n_qkv = (H + 2 * HK) * D
        cos, sin = _cos_sin(self, B, 1, hidden_states.device, qkv.dtype, position_ids, None, cache,
                            position_embeddings)
        q, gq, gate = decode_qkv(qkv, self.q_global_proj, self.k_global_proj, self.v_global_proj, cos, sin, cache,
                                 self.layer_idx, H, HK, gate_col=n_qkv)
        gate = gate.view(B, 1, 1)
        len_g, len_l = cache.step_lengths()
        bound_g, bound_l = cache.length_bounds()
        li = self.layer_idx
        if self.use_context_norm and bound_l <= 256 and _fused_ok(self.context_norm_local.weight,
                                                                 self.context_norm_global.weight):
            # both branches and the epilogue in two launches
            out = decode_attn_fused(q, cache.local_k[li], cache.local_v[li], len_l, bound_l, gq, cache.global_k[li],
                                    cache.global_v[li], len_g, bound_g, gate.view(B), self.gate_thres,
                                    self.context_norm_local.weight, self.context_norm_global.weight,
                                    self.context_norm_local.variance_epsilon)
            return out.view(B, 1, H * D), gate
        local = decode_attn(q, cache.local_k[li], cache.local_v[li], len_l, max_len=bound_l)
        glob = decode_attn(gq, cache.global_k[li], cache.global_v[li], len_g, gate.view(B), self.gate_thres,
                           max_len=bound_g)
        return self._fuse(local.view(B, 1, H, D), glob.view(B, 1, H, D), gate.view(B, 1)), gate

    def forward(self, hidden_states, attention_mask=None, position_ids=None, cu_seqlens=None,
                past_key_value: Optional[LogoKVCache] = None, output_attentions: bool = False,
                use_cache: bool = False, cache_position=None, position_embeddings=None, max_seqlen=None, **kwargs):
        """Same arguments as logo/layers/logo.py:96-110.  ``attention_mask`` is a
        2-D padding mask ``[B, T]``; a decode step ignores it (the cache holds
        each row's kept tokens only, see ``LogoKVCache.prefill``)."""
        B, T, _ = hidden_states.shape
        H, HK, D = self.num_heads, self.num_key_value_heads, self.head_dim
        if self._fused_decode_ok(hidden_states, past_key_value):
            out, gate = self._decode_fused(hidden_states, past_key_value, position_embeddings, position_ids)
            if self.training:
                with torch.no_grad():
                    self.gate_avg.add_(gate.sum().float())
                    self.global_token_count.add_((gate >= self.gate_thres).sum().float())
                    self.total_token_count.add_(gate.numel())
            return self.o_proj(out), None, past_key_value
        cs = lambda dtype: _cos_sin(self, B, T, hidden_states.device, dtype, position_ids,  # noqa: E731
                                    cu_seqlens, past_key_value, position_embeddings)
        cos = sin = None
        if self._fused_inputs_ok(hidden_states):
            cos, sin = cs(hidden_states.dtype)
        if cos is not None and all(t.is_cuda and t.dtype == torch.bfloat16 and tuple(t.shape) == (B, T, D)
                                   for t in (cos, sin)):
            q, k, v, gq, gk, gv, logit = attn_inputs(
                hidden_states, self.q_proj, self.k_proj, self.v_proj, self.gate_proj,
                (self.q_global_proj, self.k_global_proj, self.v_global_proj), cos, sin, H, HK)
            gate = torch.sigmoid(logit)  # [B, T, 1]
        else:
            q = self.q_proj(hidden_states).view(B, T, H, D)
            k = self.k_proj(hidden_states).view(B, T, HK, D)
            v = self.v_proj(hidden_states).view(B, T, HK, D)
            gq, gk, gv = self._global_qkv(q, k, v)
            gate = torch.sigmoid(self.gate_proj(hidden_states))  # [B, T, 1]
            if cos is None:
                cos, sin = cs(q.dtype)
            q, k, gq, gk = _rope_all((q, k, gq, gk), cos, sin)

        if past_key_value is not None and T == 1:
            out = self._decode(q, k, v, gq, gk, gv, gate, past_key_value)
        else:
            plan = varlen_plan(B, T, q.device, cu_seqlens, attention_mask, position_ids)
            if past_key_value is not None:
                keep = padding_mask(attention_mask)
                past_key_value.prefill(self.layer_idx, k.transpose(1, 2), v.transpose(1, 2),
                                       gk.transpose(1, 2), gv.transpose(1, 2),
                                       keep=None if keep is None else keep.reshape(B, -1)[:, -T:])
            out = self._prefill(q, k, v, gq, gk, gv, gate, cu_seqlens, plan)

        if self.training:
            with torch.no_grad():
                self.gate_avg.add_(gate.sum().float())
                self.global_token_count.add_((gate >= self.gate_thres).sum().float())
                self.total_token_count.add_(gate.numel())
        return self.o_proj(out), None, past_key_value

    def _prefill(self, q, k, v, gq, gk, gv, gate, cu_seqlens, plan: VarlenPlan):
        """Local SWA within ``plan``'s segments (logo/layers/logo.py:162-182).
        The sparse global branch packs each batch row as one sequence unless
        ``cu_seqlens`` is given, ignoring a padding mask and position resets
        exactly as the reference's does (:188-209); the "flash" global branch
        attends within ``plan``'s segments like the local one (:210-224)."""
        B, T, H, D = q.shape
        N = B * T
        local = plan.unpack(swa_attn(plan.pack(q), plan.pack(k), plan.pack(v), plan.cu,
                                     window=self.local_window_size), B, T)
        if self.sparse_full_attn_backend in SPARSE_BACKENDS:
            cu = _pack_cu(B, T, cu_seqlens, q.device)
            pk = lambda x: x.reshape(1, N, x.shape[2], x.shape[3])  # noqa: E731
            selection = (gate.reshape(1, N) >= self.gate_thres)
            glob = sq_full_attn(pk(gq), pk(gk), pk(gv), selection, cu_seqlens=cu).view(B, T, H, D)
        else:
            glob = plan.unpack(dense_causal_attn(plan.pack(gq), plan.pack(gk), plan.pack(gv), plan.cu), B, T)
        return self._fuse(local, glob, gate.view(B, T))

    def _decode(self, q, k, v, gq, gk, gv, gate, cache: LogoKVCache):
        B, _, H, D = q.shape
        cache.append(self.layer_idx, k[:, 0], v[:, 0], gk[:, 0], gv[:, 0])
        len_g, len_l = cache.step_lengths()
        bound_g, bound_l = cache.length_bounds()
        local = decode_attn(q[:, 0], cache.local_k[self.layer_idx], cache.local_v[self.layer_idx], len_l,
                            max_len=bound_l)
        glob = decode_attn(gq[:, 0], cache.global_k[self.layer_idx], cache.global_v[self.layer_idx], len_g,
                           gate.view(B), self.gate_thres, max_len=bound_g)
        return self._fuse(local.view(B, 1, H, D), glob.view(B, 1, H, D), gate.view(B, 1))


class Attention(nn.Module):
    """Plain causal attention layer, used where ``attn_type_list[i] != 0``
    (logo/layers/attn.py:22-127, selected at logo/modeling_logo.py:47-51):
    q / k / v projections, RoPE, dense causal attention over each packed
    segment, o_proj.  The reference runs flash-attn; here the attention is this
    package's HIP kernel in dense mode (every row, no compaction), prefill and
    training alike, and a decode step reads the layer's full K/V from the
    preallocated cache with the decode kernel (every row active).  Same
    parameter names as the reference, so its state dict loads."""

    def __init__(self, config: LoGoConfig, layer_idx: int = 0):
        super().__init__()
        self.config = config
        self.layer_idx = layer_idx
        self.hidden_size = config.hidden_size
        self.num_heads = config.num_attention_heads
        self.num_key_value_heads = config.num_key_value_heads
        self.head_dim = config.head_dim
        if self.head_dim * self.num_heads != self.hidden_size:
            raise ValueError(f"hidden_size must be divisible by num_heads (got `hidden_size`: {self.hidden_size}"
                             f" and `num_heads`: {self.num_heads}).")
        H, HK, D = self.num_heads, self.num_key_value_heads, self.head_dim
        self.q_proj = nn.Linear(self.hidden_size, H * D, bias=config.attention_bias)
        self.k_proj = nn.Linear(self.hidden_size, HK * D, bias=config.attention_bias)
        self.v_proj = nn.Linear(self.hidden_size, HK * D, bias=config.attention_bias)
        self.o_proj = nn.Linear(self.hidden_size, self.hidden_size, bias=config.attention_out_bias)

    def forward(self, hidden_states, attention_mask=None, position_ids=None, cu_seqlens=None,
                past_key_value: Optional[LogoKVCache] = None, output_attentions: bool = False,
                use_cache: bool = False, cache_position=None, position_embeddings=None, max_seqlen=None, **kwargs):
        """Same arguments as logo/layers/attn.py:62-76; a padding mask or
        restarting ``position_ids`` select the segments as in the LoGo layer's
        local branch (``varlen_plan``)."""
        B, T, _ = hidden_states.shape
        H, HK, D = self.num_heads, self.num_key_value_heads, self.head_dim
        q = self.q_proj(hidden_states).view(B, T, H, D)
        k = self.k_proj(hidden_states).view(B, T, HK, D)
        v = self.v_proj(hidden_states).view(B, T, HK, D)
        cos, sin = _cos_sin(self, B, T, hidden_states.device, q.dtype, position_ids, cu_seqlens, past_key_value,
                            position_embeddings)
        q, k = _rope_all((q, k), cos, sin)
        if past_key_value is not None and T == 1:
            cache = past_key_value
            # the local ring of a plain layer is never read; it takes the same rows
            cache.append(self.layer_idx, k[:, 0], v[:, 0], k[:, 0], v[:, 0])
            len_g, _ = cache.step_lengths()
            bound_g, _ = cache.length_bounds()
            out = decode_attn(q[:, 0], cache.global_k[self.layer_idx], cache.global_v[self.layer_idx], len_g,
                              max_len=bound_g).view(B, 1, H * D)
        else:
            plan = varlen_plan(B, T, q.device, cu_seqlens, attention_mask, position_ids)
            if past_key_value is not None:
                kt, vt = k.transpose(1, 2), v.transpose(1, 2)
                keep = padding_mask(attention_mask)
                past_key_value.prefill(self.layer_idx, kt, vt, kt, vt,
                                       keep=None if keep is None else keep.reshape(B, -1)[:, -T:])
            out = plan.unpack(dense_causal_attn(plan.pack(q), plan.pack(k), plan.pack(v), plan.cu), B, T)
            out = out.reshape(B, T, H * D)
        return self.o_proj(out), None, past_key_value
