"""Minimal LoGo causal LM around the HIP attention path, for decode with a KV cache.

Counterpart of ``LoGoForCausalLM`` (logo/modeling_logo.py:308-380) with the
decoder stack of :42-106 and :136-275 (pre-norm RMSNorm layers, SwiGLU MLP
logo/modules/mlp.py:10-27, final RMSNorm, tied or separate LM head).  Parameter
names follow the reference so its state dict loads.  It exists to drive the
prefill + greedy decode workload through ``LoGoAttention``
and ``LogoKVCache``: the preallocated cache replaces the reference's
``torch.cat`` growth (logo/cache.py:115-118) and the gate-aware decode kernel
its dense ``active.any()`` branch (logo/layers/logo.py:228-249).

Out of scope here, as for the rest of this package: training losses, the HF
``generate`` machinery, sampling strategies other than greedy, and the budget
controller (logo/update.py).
"""

import math
from typing import Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from .layers import (Attention, LoGoAttention, LoGoConfig, RMSNorm, _fused_ok, padding_mask, position_ids_for,
                     rope_cos_sin)
from .ops.decode import LogoKVCache
from .ops.glue import add_rms_norm, silu_mul

__all__ = ["LoGoMLP", "LoGoDecoderLayer", "LoGoModel", "LoGoForCausalLM"]


class LoGoMLP(nn.Module):
    """SwiGLU feed-forward (logo/modules/mlp.py:10-27, ``hidden_act = silu``)."""

    def __init__(self, config: LoGoConfig):
        super().__init__()
        self.gate_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.up_proj = nn.Linear(config.hidden_size, config.intermediate_size, bias=False)
        self.down_proj = nn.Linear(config.intermediate_size, config.hidden_size, bias=False)

    def _gate_up_weight(self):
        """gate_proj and up_proj weights stacked for one GEMM, rebuilt when
        either changes."""
        ws = (self.gate_proj.weight, self.up_proj.weight)
        key = tuple((w.data_ptr(), w._version, w.dtype) for w in ws)
        cached = getattr(self, "_gu_w", None)
        if cached is None or cached[0] != key:
            self._gu_w = (key, torch.cat([w.detach() for w in ws]).contiguous())
        return self._gu_w[1]

    def forward(self, x):
        if _fused_ok(x, self.gate_proj.weight, self.up_proj.weight) and self.gate_proj.weight.shape[0] % 8 == 0:
            # inference: one GEMM for gate and up, one launch for silu * mul
            return self.down_proj(silu_mul(F.linear(x, self._gate_up_weight())))
        return self.down_proj(F.silu(self.gate_proj(x)) * self.up_proj(x))


class LoGoDecoderLayer(nn.Module):
    """Pre-norm attention + MLP block (logo/modeling_logo.py:42-106); the
    attention is LoGo's or plain per ``config.attn_type_list``."""

    def __init__(self, config: LoGoConfig, layer_idx: int):
        super().__init__()
        # attn_type_list[i] == 0: LoGo attention, else plain causal attention
        # (logo/modeling_logo.py:47-51)
        if config.attn_type_list[layer_idx] == 0:
            self.self_attn = LoGoAttention(config, layer_idx)
        else:
            self.self_attn = Attention(config, layer_idx)
        self.mlp = LoGoMLP(config)
        self.input_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)
        self.post_attention_layernorm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, hidden_states, attention_mask=None, position_ids=None, cu_seqlens=None,
                past_key_value: Optional[LogoKVCache] = None, position_embeddings=None):
        residual = hidden_states
        h = self.input_layernorm(hidden_states)
        h, _, _ = self.self_attn(h, attention_mask=attention_mask, position_ids=position_ids, cu_seqlens=cu_seqlens,
                                 past_key_value=past_key_value, position_embeddings=position_embeddings)
        hidden_states = residual + h
        residual = hidden_states
        h = self.mlp(self.post_attention_layernorm(hidden_states))
        return residual + h


class LoGoModel(nn.Module):
    """Embedding, decoder layers and the final norm (logo/modeling_logo.py:136-275)."""

    def __init__(self, config: LoGoConfig):
        super().__init__()
        self.config = config
        self.embed_tokens = nn.Embedding(config.vocab_size, config.hidden_size)
        self.layers = nn.ModuleList([LoGoDecoderLayer(config, i) for i in range(config.num_hidden_layers)])
        self.norm = RMSNorm(config.hidden_size, eps=config.rms_norm_eps)

    def forward(self, input_ids, attention_mask=None, position_ids=None, cu_seqlens=None,
                past_key_value: Optional[LogoKVCache] = None):
        """``attention_mask``: a 2-D padding mask ``[B, T]`` (passed on only when
        it masks something, logo/modeling_logo.py:293-305); without explicit
        ``position_ids`` a padded batch takes generate's positions, the count
        of kept tokens before each one (pads at 1,
        logo/modeling_logo.py:421-432).  A decode step reads its positions
        from the cache."""
        h = self.embed_tokens(input_ids)
        B, T = input_ids.shape
        mask = padding_mask(attention_mask) if T > 1 else None
        if position_ids is None and mask is not None:
            position_ids = mask.long().cumsum(-1) - 1
            position_ids.masked_fill_(~mask, 1)
            position_ids = position_ids[:, -T:]
        pos = position_ids if position_ids is not None else position_ids_for(B, T, input_ids.device, cu_seqlens,
                                                                             past_key_value)
        # rotary cos / sin once for all layers (logo/modeling_logo.py:233-234)
        pe = rope_cos_sin(pos.expand(B, T), self.config.head_dim, self.config.rope_theta, h.dtype)
        if _fused_ok(h) and h.shape[-1] <= 4096:
            # inference: each residual add fused with the norm that follows it
            # (post-attention norm, the next layer's input norm, the final norm)
            resid, normed = h, self.layers[0].input_layernorm(h)
            for i, layer in enumerate(self.layers):
                a, _, _ = layer.self_attn(normed, attention_mask=mask, position_ids=position_ids,
                                          cu_seqlens=cu_seqlens, past_key_value=past_key_value,
                                          position_embeddings=pe)
                pn = layer.post_attention_layernorm
                resid, normed = add_rms_norm(resid, a, pn.weight, pn.variance_epsilon)
                m = layer.mlp(normed)
                nn_ = self.layers[i + 1].input_layernorm if i + 1 < len(self.layers) else self.norm
                resid, normed = add_rms_norm(resid, m, nn_.weight, nn_.variance_epsilon)
            return normed
        for layer in self.layers:
            h = layer(h, attention_mask=mask, position_ids=position_ids, cu_seqlens=cu_seqlens,
                      past_key_value=past_key_value, position_embeddings=pe)
        return self.norm(h)


class LoGoForCausalLM(nn.Module):
    """Causal LM head over ``LoGoModel`` (logo/modeling_logo.py:308-380)."""

    def __init__(self, config: LoGoConfig):
        super().__init__()
        self.config = config
        self.model = LoGoModel(config)
        self.lm_head = nn.Linear(config.hidden_size, config.vocab_size, bias=False)
        if config.tie_word_embeddings:
            self.lm_head.weight = self.model.embed_tokens.weight

    @torch.no_grad()
    def init_weights(self, generator: Optional[torch.Generator] = None):
        """Random init as ``post_init`` / ``_init_weights`` do
        (logo/modeling_logo.py:117-133): Linear ~ N(0, initializer_range), with
        std / sqrt(2 L) for o_proj and down_proj; Embedding ~ N(0, 1 / (2 hidden));
        norms at one and the global ``linear_proj`` matrices at identity (they
        are not Linear modules).  A tied LM head keeps the embedding's values."""
        c = self.config
        std = c.initializer_range
        out_std = std / math.sqrt(2 * c.num_hidden_layers)
        tied = self.lm_head.weight is self.model.embed_tokens.weight
        for name, mod in self.named_modules():
            if isinstance(mod, nn.Embedding):
                mod.weight.normal_(0.0, math.sqrt(1.0 / (2 * c.hidden_size)), generator=generator)
            elif isinstance(mod, nn.Linear):
                if tied and mod is self.lm_head:
                    continue
                s = out_std if name.endswith(("o_proj", "down_proj")) else std
                mod.weight.normal_(0.0, s, generator=generator)
                if mod.bias is not None:
                    mod.bias.zero_()

    def new_cache(self, batch: int, max_len: int, device=None) -> LogoKVCache:
        c = self.config
        return LogoKVCache(c.num_hidden_layers, batch, c.num_key_value_heads, c.head_dim, max_len,
                           window=c.window_size, device=device)

    def forward(self, input_ids, attention_mask=None, position_ids=None, cu_seqlens=None,
                past_key_value: Optional[LogoKVCache] = None, last_only: bool = False):
        """Logits ``[B, T, V]`` (or ``[B, V]`` of the last position with
        ``last_only``: a 16K-token prompt batch would otherwise materialise
        tens of GB of logits)."""
        h = self.model(input_ids, attention_mask=attention_mask, position_ids=position_ids, cu_seqlens=cu_seqlens,
                       past_key_value=past_key_value)
        if last_only:
            h = h[:, -1]
        return self.lm_head(h)

    @torch.no_grad()
    def prefill(self, input_ids, cache: LogoKVCache, attention_mask=None):
        """Run the prompt ``[B, T]`` through the model, filling ``cache``; returns
        the last position's logits ``[B, V]``.  A left-padded batch
        (``attention_mask [B, T]``, zeros before each row's tokens, as
        generate pads) caches each row's own tokens and continues at its own
        position."""
        mask = padding_mask(attention_mask)
        if mask is not None and not bool(mask[:, -1].all()):
            raise ValueError("prefill with a padding mask expects left padding (every row's last token kept)")
        logits = self.forward(input_ids, attention_mask=mask, past_key_value=cache, last_only=True)
        if mask is None:
            cache.set_length(input_ids.shape[1])
        else:
            cache.set_lengths(mask.sum(-1))
        return logits

    @torch.no_grad()
    def decode_step(self, tokens, cache: LogoKVCache):
        """One decode step for ``tokens [B]`` at position ``cache.seen``;
        returns logits ``[B, V]``."""
        logits = self.forward(tokens[:, None], past_key_value=cache, last_only=True)
        cache.advance()
        return logits

    @torch.no_grad()
    def capture_greedy_decode(self, tokens, cache: LogoKVCache):
        """Capture one decode step into a HIP graph, for greedy decoding.

        ``tokens [B]`` (int64, on the device) seeds a static input buffer.  The
        returned ``step()`` replays the graph, which runs the whole model on
        the buffered tokens at the cache's device position, writes the logits
        to a static buffer, appends the K/V and advances the device position;
        then, outside the graph (a multi-block reduction may record memset
        nodes), it writes the argmax tokens back into the input buffer and
        advances the host ``cache.seen``.  ``step`` returns (logits, next
        tokens), both static buffers overwritten by the next call.  The cache
        needs room for every step (``cache.max_len``).  Capturing runs
        nothing: the cache is unchanged until the first replay.  The eager
        path should have run once with these shapes (library handles and
        workspaces initialise on first use)."""
        tok_buf = tokens.detach().clone()
        stream = torch.cuda.Stream(device=tokens.device)
        stream.wait_stream(torch.cuda.current_stream())
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.stream(stream):
            with torch.cuda.graph(graph, stream=stream):
                logits = self.forward(tok_buf[:, None], past_key_value=cache, last_only=True)
                cache.advance_device()
        torch.cuda.current_stream().wait_stream(stream)

        def step():
            if cache.seen >= cache.max_len:
                raise ValueError("cache is full")
            graph.replay()
            cache.seen += 1
            torch.argmax(logits, dim=-1, out=tok_buf)
            return logits, tok_buf

        step.graph = graph
        return step

    @torch.no_grad()
    def greedy_generate(self, input_ids, max_new_tokens: int, cache: Optional[LogoKVCache] = None,
                        attention_mask=None):
        """Greedy decoding: returns the generated tokens ``[B, max_new_tokens]``;
        ``attention_mask`` for a left-padded prompt batch."""
        B, T = input_ids.shape
        if cache is None:
            cache = self.new_cache(B, T + max_new_tokens, device=input_ids.device)
        tok = self.prefill(input_ids, cache, attention_mask=attention_mask).argmax(-1)
        out = [tok]
        for _ in range(max_new_tokens - 1):
            tok = self.decode_step(tok, cache).argmax(-1)
            out.append(tok)
        return torch.stack(out, dim=1)
