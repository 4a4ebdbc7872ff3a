"""Float64 torch restatement of LoGoAttention.forward for layer-level parity.

Follows logo/layers/logo.py:96-262 (projections, linear_proj / scale_offset
re-parameterisation :80-94, sigmoid gate :130, RoPE on both branches :132-139
with logo/modules/rotary.py:58-106, local SWA window 128 :162-182 via
logo/layers/utils.py:144-147, sparse global branch :188-209 with the semantics
of logo/ops/selected_full_attn.py:495-527, context norms :180-181 / :225-226,
masked fusion :256-258, o_proj :259) with dense masked softmax, so autograd
gives the backward.  The comparison is made "given the same gate decisions":
the caller supplies the selection (gate >= thres) the device computed, while
the gate values used in the fusion are this reference's own (differentiable)
sigmoid(gate_proj(h)).  Its attention core is checked against oracle.attn in
tests/test_layer_ref.py.

``store_dtype=torch.bfloat16`` restates the reference *as it runs in bf16*
(its attention kernels also round P and dS, ``_AttnRounded``):
the arithmetic of each op stays in float64, but every tensor the eager bf16
module chain stores is rounded to bf16 where that chain stores it -- the
projection outputs, the global projections, the gate logit and sigmoid,
RoPE's cos / sin (computed in fp32, logo/modules/rotary.py:58-78) and each of
its products and sums (:101-105), the attention outputs, RMSNorm's normalised
rows and weighted output (logo/modules/layernorm.py:17-22), the fusion's
(1 - g), both products and their sum (logo/layers/logo.py:257), and o_proj's
output -- and, in the backward, every gradient flowing back through those
tensors is rounded too, as bf16 autograd stores it.
"""

import torch


class _Store(torch.autograd.Function):
    """Round to the storage dtype and back, forward and backward."""

    @staticmethod
    def forward(ctx, x, dtype):
        ctx.dtype = dtype
        return x.to(dtype).to(x.dtype)

    @staticmethod
    def backward(ctx, g):
        return g.to(ctx.dtype).to(g.dtype), None


def _storer(dtype):
    if dtype is None:
        return lambda x: x
    return lambda x: _Store.apply(x, dtype)


def _rmsnorm(x, w, eps, R=lambda t: t):
    return R(w * R(x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)))


def _rope(x, pos, theta, R=lambda t: t, fp32_angles=False):
    D = x.shape[-1]
    adt = torch.float32 if fp32_angles else torch.float64
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=adt, device=x.device) / D))
    fr = pos.to(x.device).to(adt)[..., None] * inv
    emb = torch.cat((fr, fr), -1)
    cos, sin = emb.cos().unsqueeze(-2).to(x.dtype), emb.sin().unsqueeze(-2).to(x.dtype)
    cos, sin = R(cos).detach(), R(sin).detach()
    half = D // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), -1)
    return R(R(x * cos) + R(rot * sin))


class _AttnRounded(torch.autograd.Function):
    """Masked softmax attention in the input's dtype (float64 here) that rounds
    P to ``dtype`` before P V, and P and dS before the three backward products,
    as the reference's Triton kernels do (P, :99; dS and P, :209-210,
    :305-311 of logo/ops/selected_full_attn.py) and flash-attn does; delta
    uses the stored (rounded) output (:135-137).  One head at a time, so the
    [N, N] score blocks of a full-size layer stay small."""

    @staticmethod
    def forward(ctx, q, k, v, mask, scale, dtype):
        # q, k, v [N, H, D] (k, v already repeated over the GQA group)
        rnd = lambda t: t.to(dtype).to(t.dtype)  # noqa: E731
        o = torch.empty_like(v[:, :, :1].expand(-1, -1, v.shape[2])).contiguous()
        lse = q.new_empty(q.shape[1], q.shape[0])
        for h in range(q.shape[1]):
            S = (q[:, h] @ k[:, h].T) * scale
            S = S.masked_fill(~mask, float("-inf"))
            m = S.max(-1, keepdim=True).values
            P = torch.exp(S - m)
            l = P.sum(-1, keepdim=True)
            o[:, h] = (rnd(P) @ v[:, h]) / l
            lse[h] = (m + torch.log(l))[:, 0]
        ctx.save_for_backward(q, k, v, mask, lse, o)
        ctx.scale, ctx.dtype = scale, dtype
        return o

    @staticmethod
    def backward(ctx, do):
        q, k, v, mask, lse, o = ctx.saved_tensors
        rnd = lambda t: t.to(ctx.dtype).to(t.dtype)  # noqa: E731
        dq, dk, dv = torch.zeros_like(q), torch.zeros_like(k), torch.zeros_like(v)
        o_stored = rnd(o)
        for h in range(q.shape[1]):
            S = (q[:, h] @ k[:, h].T) * ctx.scale
            P = torch.exp(S.masked_fill(~mask, float("-inf")) - lse[h][:, None])
            dP = do[:, h] @ v[:, h].T
            delta = (o_stored[:, h] * do[:, h]).sum(-1, keepdim=True)
            dS = rnd(P * (dP - delta))
            dq[:, h] = ctx.scale * (dS @ k[:, h])
            dk[:, h] = ctx.scale * (dS.T @ q[:, h])
            dv[:, h] = rnd(P).T @ do[:, h]
        return dq, dk, dv, None, None, None


def _attn(q, k, v, seg, pos, sel, window, round_dtype=None):
    """q [N, H, D], k/v [N, HK, D]; seg/pos [N]; sel bool [N] or None;
    round_dtype: None (exact softmax attention) or the dtype the reference's
    kernels round P and dS to (``_AttnRounded``)."""
    N, H, D = q.shape
    G = H // k.shape[1]
    kk = k.repeat_interleave(G, 1)
    vv = v.repeat_interleave(G, 1)
    same = seg[:, None] == seg[None, :]
    causal = pos[None, :] <= pos[:, None]
    mask = same & causal
    if window is not None:
        mask &= pos[None, :] >= pos[:, None] - window
    if round_dtype is not None:
        o = _AttnRounded.apply(q, kk, vv, mask, D ** -0.5, round_dtype)
    else:
        S = torch.einsum("qhd,khd->hqk", q, kk) * D ** -0.5
        P = torch.softmax(S.masked_fill(~mask[None], float("-inf")), -1)
        o = torch.einsum("hqk,khd->qhd", P, vv)
    if sel is not None:
        o = o * sel[:, None, None].to(o.dtype)
    return o


def logo_layer_ref(h, p, cfg, sel_bt, cu=None, backend="hip", store_dtype=None, attention_mask=None):
    """``h [B, T, C]`` float64; ``p`` dict of float64 params (reference names);
    ``sel_bt [B, T]`` bool: which tokens pass the gate threshold;
    ``store_dtype``: None (float64 throughout) or the dtype the reference's
    module chain stores its tensors in (see the module docstring);
    ``attention_mask [B, T]``: a padding mask, with the reference's semantics
    (logo/layers/utils.py:180-201, logo/modeling_logo.py:421-432): RoPE at
    generate's positions (kept tokens counted, pads at 1), the local branch
    and the "flash" global branch over each row's kept tokens (pads give 0),
    the sparse global branch over the whole padded row."""
    R = _storer(store_dtype)
    h = R(h)  # the layer input is stored too: its gradient is rounded once summed
    B, T, C = h.shape
    H, HK, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    # nn.Linear, with the bias when the config has one (attention_bias /
    # attention_out_bias, logo/layers/logo.py:50-58)
    lin = lambda x, name: x @ p[name + ".weight"].T + (p[name + ".bias"] if name + ".bias" in p else 0)  # noqa: E731
    q = R(lin(h, "q_proj")).view(B, T, H, D)
    k = R(lin(h, "k_proj")).view(B, T, HK, D)
    v = R(lin(h, "v_proj")).view(B, T, HK, D)
    if cfg.global_qk_param == "linear_proj":
        gq = R(torch.einsum("bthd,hde->bthe", q, p["q_global_proj"]))
        gk = R(torch.einsum("bthd,hde->bthe", k, p["k_global_proj"]))
        gv = R(torch.einsum("bthd,hde->bthe", v, p["v_global_proj"]))
    else:
        gq = R(R(q * p["q_global_scale"].view(H, D)) + p["q_global_offset"].view(H, D))
        gk = R(R(k * p["k_global_scale"].view(HK, D)) + p["k_global_offset"].view(HK, D))
        gv = R(R(v * p["v_global_scale"].view(HK, D)) + p["v_global_offset"].view(HK, D))
    N = B * T
    if cu is None:
        seg = torch.arange(N) // T
        pos = torch.arange(N) % T
    else:
        cul = cu.tolist()
        seg = torch.zeros(N, dtype=torch.long)
        pos = torch.zeros(N, dtype=torch.long)
        for s in range(len(cul) - 1):
            seg[cul[s]:cul[s + 1]] = s
            pos[cul[s]:cul[s + 1]] = torch.arange(cul[s + 1] - cul[s])
    seg, pos = seg.to(h.device), pos.to(h.device)
    posbt = pos.view(B, T)
    keep = None
    if attention_mask is not None:
        keep = attention_mask.to(h.device).bool().reshape(N)
        kept_pos = attention_mask.to(h.device).long().cumsum(-1) - 1
        posbt = kept_pos.masked_fill(~attention_mask.to(h.device).bool(), 1)
        # kept tokens: row segments with positions among the kept; every pad its
        # own segment (its output is zeroed below)
        lseg = torch.where(keep, seg, -1 - torch.arange(N, device=h.device))
        lpos = kept_pos.reshape(N).clamp_min(0)
    f32 = store_dtype in (torch.bfloat16, torch.float16)  # the reference computes angles in fp32
    q, k = _rope(q, posbt, cfg.rope_theta, R, f32), _rope(k, posbt, cfg.rope_theta, R, f32)
    gq, gk = _rope(gq, posbt, cfg.rope_theta, R, f32), _rope(gk, posbt, cfg.rope_theta, R, f32)
    gate = R(torch.sigmoid(R(h @ p["gate_proj.weight"].T)))  # [B, T, 1]
    sel_bt = sel_bt.to(h.device)
    sel = sel_bt.reshape(N) if backend != "flash" else None
    lseg, lpos = (seg, pos) if keep is None else (lseg, lpos)
    local = R(_attn(q.reshape(N, H, D), k.reshape(N, HK, D), v.reshape(N, HK, D), lseg, lpos, keep,
                    cfg.window_size, store_dtype))
    gseg, gpos = (lseg, lpos) if backend == "flash" else (seg, pos)
    gsel = sel if keep is None or backend != "flash" else keep
    glob = R(_attn(gq.reshape(N, H, D), gk.reshape(N, HK, D), gv.reshape(N, HK, D), gseg, gpos, gsel, None,
                   store_dtype))
    local = _rmsnorm(local, p["context_norm_local.weight"], cfg.rms_norm_eps, R).reshape(B, T, C)
    glob = _rmsnorm(glob, p["context_norm_global.weight"], cfg.rms_norm_eps, R).reshape(B, T, C)
    g = gate.masked_fill(~sel_bt.reshape(B, T, 1), 0.0)
    out = R(R(R(1 - g) * local) + R(g * glob))
    return R(lin(out, "o_proj"))


def plain_attn_layer_ref(h, p, cfg, cu=None):
    """Float64 restatement of the plain attention layer
    (logo/layers/attn.py:62-127): projections, RoPE, dense causal attention per
    packed segment, o_proj."""
    B, T, C = h.shape
    H, HK, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    q = (h @ p["q_proj.weight"].T).view(B, T, H, D)
    k = (h @ p["k_proj.weight"].T).view(B, T, HK, D)
    v = (h @ p["v_proj.weight"].T).view(B, T, HK, D)
    N = B * T
    if cu is None:
        seg = torch.arange(N) // T
        pos = torch.arange(N) % T
    else:
        cul = cu.tolist()
        seg = torch.zeros(N, dtype=torch.long)
        pos = torch.zeros(N, dtype=torch.long)
        for s in range(len(cul) - 1):
            seg[cul[s]:cul[s + 1]] = s
            pos[cul[s]:cul[s + 1]] = torch.arange(cul[s + 1] - cul[s])
    posbt = pos.view(B, T)
    q, k = _rope(q, posbt, cfg.rope_theta), _rope(k, posbt, cfg.rope_theta)
    o = _attn(q.reshape(N, H, D), k.reshape(N, HK, D), v.reshape(N, HK, D), seg, pos, None, None)
    return o.reshape(B, T, C) @ p["o_proj.weight"].T
