"""LogoKVCache refuses a prompt on top of cached tokens (CPU, no kernels run).

A multi-token forward attends to its own tokens only, so writing a second
prompt chunk at [0, T) of a non-empty cache would silently drop the cached
context; the reference's cache appends instead (logo/cache.py:90-115).
"""

import pytest
import torch

from logo_amd.ops.decode import LogoKVCache


def _kv(B=2, H=2, T=5, D=8):
    return [torch.randn(B, H, T, D) for _ in range(4)]


def test_second_prefill_is_rejected_until_reset():
    cache = LogoKVCache(num_layers=2, batch=2, kv_heads=2, head_dim=8, max_len=32, window=4, device="cpu")
    cache.prefill(0, *_kv())
    cache.prefill(1, *_kv())  # every layer of one prompt fills while seen == 0
    cache.set_length(5)
    with pytest.raises(ValueError, match="already holds 5 tokens"):
        cache.prefill(0, *_kv())
    cache.reset()
    assert cache.get_seq_length() == 0 and int(cache._pos.max()) == 0
    k = _kv(T=7)
    cache.prefill(0, *k)
    assert torch.equal(cache.global_k[0][:, :, :7], k[2].to(cache.global_k[0].dtype))


def test_prompt_longer_than_cache_is_rejected():
    cache = LogoKVCache(num_layers=1, batch=1, kv_heads=1, head_dim=8, max_len=4, window=2, device="cpu")
    with pytest.raises(ValueError, match="exceeds"):
        cache.prefill(0, *_kv(B=1, H=1, T=5))
