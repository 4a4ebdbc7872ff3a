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
"""

import torch


def _rmsnorm(x, w, eps):
    return w * (x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps))


def _rope(x, pos, theta):
    D = x.shape[-1]
    inv = 1.0 / (theta ** (torch.arange(0, D, 2, dtype=torch.float64) / D))
    fr = pos.double()[..., None] * inv
    emb = torch.cat((fr, fr), -1)
    cos, sin = emb.cos().unsqueeze(-2), emb.sin().unsqueeze(-2)
    half = D // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), -1)
    return x * cos + rot * sin


def _attn(q, k, v, seg, pos, sel, window):
    """q [N, H, D], k/v [N, HK, D]; seg/pos [N]; sel bool [N] or None."""
    N, H, D = q.shape
    G = H // k.shape[1]
    kk = k.repeat_interleave(G, 1)
    vv = v.repeat_interleave(G, 1)
    same = seg[:, None] == seg[None, :]
    causal = pos[None, :] <= pos[:, None]
    mask = same & causal
    if window is not None:
        mask &= pos[None, :] >= pos[:, None] - window
    S = torch.einsum("qhd,khd->hqk", q, kk) * D ** -0.5
    P = torch.softmax(S.masked_fill(~mask[None], float("-inf")), -1)
    o = torch.einsum("hqk,khd->qhd", P, vv)
    if sel is not None:
        o = o * sel[:, None, None].to(o.dtype)
    return o


def logo_layer_ref(h, p, cfg, sel_bt, cu=None, backend="hip"):
    """``h [B, T, C]`` float64; ``p`` dict of float64 params (reference names);
    ``sel_bt [B, T]`` bool: which tokens pass the gate threshold."""
    B, T, C = h.shape
    H, HK, D = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
    q = (h @ p["q_proj.weight"].T).view(B, T, H, D)
    k = (h @ p["k_proj.weight"].T).view(B, T, HK, D)
    v = (h @ p["v_proj.weight"].T).view(B, T, HK, D)
    if cfg.global_qk_param == "linear_proj":
        gq = torch.einsum("bthd,hde->bthe", q, p["q_global_proj"])
        gk = torch.einsum("bthd,hde->bthe", k, p["k_global_proj"])
        gv = torch.einsum("bthd,hde->bthe", v, p["v_global_proj"])
    else:
        gq = q * p["q_global_scale"].view(H, D) + p["q_global_offset"].view(H, D)
        gk = k * p["k_global_scale"].view(HK, D) + p["k_global_offset"].view(HK, D)
        gv = v * p["v_global_scale"].view(HK, D) + p["v_global_offset"].view(HK, D)
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
    gq, gk = _rope(gq, posbt, cfg.rope_theta), _rope(gk, posbt, cfg.rope_theta)
    gate = torch.sigmoid(h @ p["gate_proj.weight"].T)  # [B, T, 1]
    sel = sel_bt.reshape(N) if backend != "flash" else None
    local = _attn(q.reshape(N, H, D), k.reshape(N, HK, D), v.reshape(N, HK, D), seg, pos, None, cfg.window_size)
    glob = _attn(gq.reshape(N, H, D), gk.reshape(N, HK, D), gv.reshape(N, HK, D), seg, pos, sel, None)
    local = _rmsnorm(local, p["context_norm_local.weight"], cfg.rms_norm_eps).reshape(B, T, C)
    glob = _rmsnorm(glob, p["context_norm_global.weight"], cfg.rms_norm_eps).reshape(B, T, C)
    g = gate.masked_fill(~sel_bt.reshape(B, T, 1), 0.0)
    out = (1 - g) * local + g * glob
    return out @ p["o_proj.weight"].T


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
