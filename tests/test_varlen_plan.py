"""The segment plan of the local / "flash" branches for padded and
position-packed batches (logo/layers/utils.py:36-104, :155-226), on the CPU."""

import torch

from logo_amd.layers import VarlenPlan, padding_mask, varlen_plan
from logo_amd.ops.decode import LogoKVCache


def test_explicit_cu_seqlens_wins():
    cu = torch.tensor([0, 3, 10], dtype=torch.int64)
    plan = varlen_plan(1, 10, "cpu", cu_seqlens=cu, attention_mask=torch.zeros(1, 10),
                       position_ids=torch.zeros(1, 10))
    assert plan.keep is None and plan.cu.dtype == torch.int32 and plan.cu.tolist() == [0, 3, 10]


def test_padding_mask_unpads_rows_in_order():
    mask = torch.tensor([[0, 0, 1, 1, 1], [1, 1, 1, 1, 1], [0, 1, 1, 0, 1]])
    plan = varlen_plan(3, 5, "cpu", attention_mask=mask)
    assert plan.cu.tolist() == [0, 3, 8, 11]
    assert plan.keep.tolist() == [2, 3, 4, 5, 6, 7, 8, 9, 11, 12, 14]
    x = torch.arange(3 * 5 * 2 * 1, dtype=torch.float32).view(3, 5, 2, 1)
    packed = plan.pack(x)
    assert packed.shape == (1, 11, 2, 1)
    back = plan.unpack(packed, 3, 5)
    assert torch.equal(back[mask.bool()], x[mask.bool()]) and not back[~mask.bool()].any()


def test_mask_without_padding_is_ignored():
    assert padding_mask(torch.ones(2, 4)) is None
    plan = varlen_plan(2, 4, "cpu", attention_mask=torch.ones(2, 4))
    assert plan.keep is None and plan.cu.tolist() == [0, 4, 8]


def test_position_ids_with_resets_pack_segments():
    pid = torch.tensor([[0, 1, 2, 0, 1, 0, 1, 2]])
    plan = varlen_plan(1, 8, "cpu", position_ids=pid)
    assert plan.keep is None and plan.cu.tolist() == [0, 3, 5, 8]
    # monotone positions (no reset): one segment per row, as the reference's
    # plain (non-varlen) call
    plan = varlen_plan(2, 4, "cpu", position_ids=torch.arange(4)[None].expand(2, 4))
    assert plan.cu.tolist() == [0, 4, 8]
    # a decode-sized call never packs by positions
    plan = varlen_plan(2, 1, "cpu", position_ids=torch.tensor([[5], [0]]))
    assert plan.cu.tolist() == [0, 1, 2]


def test_plan_pack_unpack_identity_without_keep():
    plan = VarlenPlan(torch.tensor([0, 6], dtype=torch.int32))
    x = torch.randn(2, 3, 4, 8)
    assert torch.equal(plan.unpack(plan.pack(x), 2, 3), x)


def test_cache_prefill_keeps_each_rows_tokens():
    B, H, T, D, W = 3, 2, 6, 4, 3
    cache = LogoKVCache(num_layers=1, batch=B, kv_heads=H, head_dim=D, max_len=16, window=W, device="cpu",
                        dtype=torch.float32)
    k = torch.arange(B * H * T * D, dtype=torch.float32).view(B, H, T, D)
    keep = torch.tensor([[0, 0, 1, 1, 1, 1], [1] * 6, [0, 0, 0, 0, 0, 1]], dtype=torch.bool)
    cache.prefill(0, k, -k, 2 * k, -2 * k, keep=keep)
    cache.set_lengths(keep.sum(-1))
    assert cache.seen == 6 and cache._pos.tolist() == [4, 6, 1]
    for b in range(B):
        kept = k[b][:, keep[b]]
        n = kept.shape[1]
        assert torch.equal(cache.global_k[0][b, :, :n], 2 * kept)
        assert torch.equal(cache.global_v[0][b, :, :n], -2 * kept)
        # the last `ring` kept positions sit at slot p % ring
        for p in range(max(0, n - cache.ring), n):
            assert torch.equal(cache.local_k[0][b, :, p % cache.ring], kept[:, p])
            assert torch.equal(cache.local_v[0][b, :, p % cache.ring], -kept[:, p])
