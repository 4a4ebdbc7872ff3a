"""GPU check of the causal LM's decode path against its prefill path.

Decoding token by token through the preallocated cache (cache append, local
ring and gate-aware decode kernels) must give, at every step, the logits that
a full prefill over the same token sequence gives at its last position (query-
sparse / sliding-window kernels).  The two paths share no attention kernel.
Gate thresholds of -1 (every token global) and 2 (every token local) make the
routing identical on both paths, so only arithmetic differs; mixed routing is
covered by the layer test against the float64 restatement.
"""

import pytest
import torch

from logo_amd.layers import LoGoConfig
from logo_amd.model import LoGoForCausalLM

pytestmark = pytest.mark.gpu


def _model(gpu, thres, seed=0, attn_types=None):
    cfg = LoGoConfig(vocab_size=512, hidden_size=256, intermediate_size=512,
                     num_hidden_layers=2 if attn_types is None else len(attn_types),
                     num_attention_heads=4, window_size=128, gate_thres_init=thres, attn_type_list=attn_types)
    m = LoGoForCausalLM(cfg)
    g = torch.Generator()
    g.manual_seed(seed)
    m.init_weights(g)
    with torch.no_grad():
        for layer in m.model.layers:  # global branch differs from the local one
            if not hasattr(layer.self_attn, "q_global_proj"):
                continue
            for p in (layer.self_attn.q_global_proj, layer.self_attn.k_global_proj,
                      layer.self_attn.v_global_proj):
                p.add_(torch.randn(p.shape, generator=g) * 0.05)
    return m.to(device=gpu, dtype=torch.bfloat16).eval()


@pytest.mark.parametrize("thres,attn_types", [(-1.0, None), (2.0, None), (0.5, [1, 1]), (-1.0, [0, 1, 0])])
def test_decode_matches_prefill(gpu, thres, attn_types):
    """Also with plain attention layers (attn_type_list != 0), alone and mixed
    with LoGo layers."""
    m = _model(gpu, thres, attn_types=attn_types)
    B, T, steps = 2, 190, 12
    g = torch.Generator()
    g.manual_seed(1)
    ids = torch.randint(0, 512, (B, T), generator=g).to(gpu)
    cache = m.new_cache(B, T + steps, device=gpu)
    logits = m.prefill(ids, cache)
    seq = ids
    for s in range(steps):
        ref = m(seq, last_only=True)  # fresh prefill over the whole sequence
        err = (logits.float() - ref.float()).abs().max().item()
        scale = ref.float().abs().max().item()
        assert err <= 0.03 * scale + 1e-3, f"step {s}: max |decode - prefill| {err:.4f} (logit scale {scale:.3f})"
        tok = ref.argmax(-1)
        seq = torch.cat([seq, tok[:, None]], dim=1)
        logits = m.decode_step(tok, cache)
    assert cache.seen == T + steps


def test_greedy_generate_shapes(gpu):
    m = _model(gpu, 0.5)
    ids = torch.randint(0, 512, (3, 40), generator=torch.Generator().manual_seed(2)).to(gpu)
    out = m.greedy_generate(ids, 5)
    assert out.shape == (3, 5) and out.dtype == torch.int64
    assert int(out.min()) >= 0 and int(out.max()) < 512


def test_graph_decode_matches_eager(gpu):
    """Replays of the captured decode step, with eager decoding and
    synchronisations in between, match eager decode steps on a twin cache."""
    m = _model(gpu, 0.5)
    B, T, steps = 2, 150, 6
    g = torch.Generator()
    g.manual_seed(3)
    ids = torch.randint(0, 512, (B, T), generator=g).to(gpu)
    ca = m.new_cache(B, T + steps + 2, device=gpu)
    cb = m.new_cache(B, T + steps + 2, device=gpu)
    tok_a = m.prefill(ids, ca).argmax(-1)
    tok_b = m.prefill(ids, cb).argmax(-1)
    tok_a = m.decode_step(tok_a, ca).argmax(-1)  # one eager step on each initialises the libraries
    tok_b = m.decode_step(tok_b, cb).argmax(-1)
    step = m.capture_greedy_decode(tok_b, cb)
    assert cb.seen == T + 1
    for s in range(steps):
        la = m.decode_step(tok_a, ca)
        tok_a = la.argmax(-1)
        torch.cuda.synchronize()
        lb, tok_b = step()
        torch.cuda.synchronize()
        err = (la.float() - lb.float()).abs().max().item()
        scale = la.float().abs().max().item()
        assert err <= 1e-2 * scale + 1e-3, f"replay {s}: max |eager - graph| {err:.4f} (scale {scale:.3f})"
        assert torch.equal(tok_a, tok_b), f"replay {s}: greedy tokens differ"
    assert cb.seen == ca.seen == T + 1 + steps
    assert torch.equal(ca._pos, cb._pos)


def test_fused_decode_step_matches_unfused(gpu):
    """The decode step with the stacked q/k/v/gate GEMM and the fused
    transform launch gives the step-by-step path's logits (up to the
    stacked GEMM's own rounding) and the same greedy tokens."""
    from logo_amd.layers import LoGoAttention

    m = _model(gpu, 0.5)
    g = torch.Generator()
    g.manual_seed(3)
    ids = torch.randint(0, 512, (4, 150), generator=g).to(gpu)
    ca, cb = m.new_cache(4, 170, device=gpu), m.new_cache(4, 170, device=gpu)
    tok = m.prefill(ids, ca).argmax(-1)
    m.prefill(ids, cb)
    for _ in range(6):
        la = m.decode_step(tok, ca)
        orig = LoGoAttention._fused_decode_ok
        LoGoAttention._fused_decode_ok = lambda self, h, c: False
        try:
            lb = m.decode_step(tok, cb)
        finally:
            LoGoAttention._fused_decode_ok = orig
        err = (la.float() - lb.float()).abs().max().item()
        assert err <= 0.02 * lb.float().abs().max().item() + 1e-3
        tok = lb.argmax(-1)


def test_second_prefill_rejected_and_reset_repeats_first(gpu):
    """A prompt on top of cached tokens is refused (it would attend to its own
    chunk only); after reset() the same prompt gives the same logits."""
    m = _model(gpu, 0.5)
    g = torch.Generator()
    g.manual_seed(2)
    ids = torch.randint(0, 512, (2, 150), generator=g).to(gpu)
    cache = m.new_cache(2, 300, device=gpu)
    first = m.prefill(ids, cache)
    with pytest.raises(ValueError, match="already holds"):
        m.prefill(ids, cache)
    cache.reset()
    again = m.prefill(ids, cache)
    assert torch.equal(first, again)


@pytest.mark.parametrize("backend,thres", [("flash", -1.0), ("hip", 2.0)])
def test_left_padded_generate_matches_each_row_alone(gpu, backend, thres):
    """Greedy decoding of a left-padded prompt batch (generate's padding,
    logo/modeling_logo.py:421-432): the cache keeps each row's own tokens and
    each row continues at its own position, so every row's logits match those
    of the same prompt decoded alone without padding.  (Routes where the
    reference attends padded keys -- its sparse global prefill -- are left
    out: threshold 2 sends every token to the local branch.)"""
    from logo_amd.layers import LoGoConfig as Cfg

    cfg = Cfg(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=2, num_attention_heads=4,
              window_size=128, gate_thres_init=thres, sparse_full_attn_backend=backend)
    m = LoGoForCausalLM(cfg)
    g = torch.Generator()
    g.manual_seed(9)
    m.init_weights(g)
    with torch.no_grad():
        for layer in m.model.layers:
            for p in (layer.self_attn.q_global_proj, layer.self_attn.k_global_proj, layer.self_attn.v_global_proj):
                p.add_(torch.randn(p.shape, generator=g) * 0.05)
    m = m.to(device=gpu, dtype=torch.bfloat16).eval()
    lens, T, steps = [190, 60, 141], 190, 8
    ids = torch.randint(1, 512, (3, T), generator=g)
    mask = torch.zeros(3, T, dtype=torch.long)
    for b, n in enumerate(lens):
        mask[b, T - n:] = 1
        ids[b, :T - n] = 0
    cache = m.new_cache(3, T + steps, device=gpu)
    logits = m.prefill(ids.to(gpu), cache, attention_mask=mask.to(gpu))
    assert cache._pos.tolist() == lens
    toks, outs = [], []
    for s in range(steps):
        outs.append(logits.float())
        tok = logits.argmax(-1)
        toks.append(tok)
        logits = m.decode_step(tok, cache)
    for b, n in enumerate(lens):
        alone = m.new_cache(1, n + steps, device=gpu)
        lg = m.prefill(ids[b:b + 1, T - n:].to(gpu), alone)
        for s in range(steps):
            err = (lg.float()[0] - outs[s][b]).abs().max().item()
            scale = outs[s][b].abs().max().item()
            assert err <= 0.03 * scale + 1e-3, f"row {b} step {s}: max diff {err:.4f} (scale {scale:.3f})"
            lg = m.decode_step(toks[s][b:b + 1], alone)
