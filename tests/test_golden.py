"""Committed golden vectors (tests/golden/logo_golden.npz, written by
tests/golden/make_golden.py from the CPU oracle).

CPU half: the oracle, run on the stored inputs, still reproduces the stored
outputs (integer outputs exactly, float outputs to float32 storage precision),
so a change to the oracle cannot silently move the parity target.

GPU half: the HIP path, called through the public ops on the stored inputs,
matches the stored outputs -- compaction bit-exact; attention outputs and
gradients within the north-star tolerance (max-abs 2e-2, mean-abs 2e-3);
the epilogue against its bf16 rounding chain and float64 gradients; decode
within the attention tolerance.
"""

import os

import numpy as np
import pytest
import torch

from oracle import attn, compact, decode, epilogue
from tests.helpers import assert_within

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "logo_golden.npz")


@pytest.fixture(scope="module")
def fx():
    with np.load(GOLDEN, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


def f32(bits):
    return (np.asarray(bits).astype(np.uint32) << 16).view(np.float32)


def bf16_tensor(bits, dev):
    return torch.from_numpy(np.asarray(bits).astype(np.int16)).view(torch.bfloat16).to(dev)


def close(got, ref, name):
    np.testing.assert_allclose(got.astype(np.float32), ref, rtol=2e-6, atol=1e-7, equal_nan=True, err_msg=name)


ATTN_CASES = ("sqa", "sqb", "swa")


# ---------------------------------------------------------------- CPU half


def test_oracle_reproduces_compaction(fx):
    cu = fx["cmp_cu"]
    for name in ("tok", "heads"):
        sel = fx["cmp_sel"] if name == "tok" else fx["cmp_sel_heads"]
        for li, lane in enumerate(compact.build_selection(sel, cu)):
            assert np.array_equal(lane["q_idx"], fx[f"cmp_{name}{li}_q_idx"])
            assert np.array_equal(lane["pos_ids"], fx[f"cmp_{name}{li}_pos"])
            assert np.array_equal(lane["cu_seqlens_q"], fx[f"cmp_{name}{li}_cu_q"])
    lane = compact.build_selection(fx["cmp_sel"], cu)[0]
    for bt in (16, 64):
        assert np.array_equal(compact.prepare_chunk_indices(cu, bt), fx[f"cmp_chunks_{bt}"])
        qs = compact.compute_q_start_blk(lane["pos_ids"], lane["cu_seqlens_q"], cu, bt, int(cu[-1]))
        assert np.array_equal(qs, fx[f"cmp_q_start_{bt}"])


@pytest.mark.parametrize("case", ATTN_CASES)
def test_oracle_reproduces_attention(fx, case):
    q, k, v, do = (f32(fx[f"{case}_{n}"]) for n in ("q", "k", "v", "do"))
    sel = fx.get(f"{case}_sel")
    window = int(fx[f"{case}_window"]) if f"{case}_window" in fx else None
    cu = fx[f"{case}_cu"]
    o, lse = attn.sq_attn_fwd(q, k, v, sel, cu, window=window)
    dq, dk, dv = attn.sq_attn_bwd(q, k, v, o, do, sel, cu, window=window)
    for name, got in (("o", o), ("lse", lse), ("dq", dq), ("dk", dk), ("dv", dv)):
        close(got, fx[f"{case}_{name}"], f"{case}_{name}")


def test_oracle_reproduces_epilogue(fx):
    L, G, gate, w_l, w_g, dout = (f32(fx[f"epi_{n}"]) for n in ("L", "G", "gate", "w_l", "w_g", "dout"))
    eps, thres = float(fx["epi_eps"]), float(fx["epi_thres"])
    out_bf = epilogue.epilogue_fwd(L, G, gate, thres, w_l, w_g, eps, bf16=True)
    assert np.array_equal(out_bf, f32(fx["epi_out_bf16"]))
    close(epilogue.epilogue_fwd(L, G, gate, thres, w_l, w_g, eps, bf16=False), fx["epi_out"], "epi_out")
    for name, got in zip(("dL", "dG", "dgate", "dw_l", "dw_g"),
                         epilogue.epilogue_bwd(L, G, gate, thres, w_l, w_g, eps, dout)):
        close(got, fx[f"epi_{name}"], f"epi_{name}")


def test_oracle_reproduces_decode(fx):
    q, k, v = (f32(fx[f"dec_{n}"]) for n in ("q", "k", "v"))
    lens = fx["dec_lens"]
    active = f32(fx["dec_gate"]) >= float(fx["dec_thres"])
    close(decode.decode_attn(q, k, v, lens, active), fx["dec_out"], "dec_out")
    close(decode.decode_attn(q, k, v, lens, None), fx["dec_out_all"], "dec_out_all")


def test_golden_fixes_known_facts(fx):
    """Facts the fixtures must show whatever the oracle: unselected rows are
    zero with nan lse; row 0 of a segment returns v_0; an inactive decode row
    is zero; the windowed case reduces to v_0 at each segment start."""
    for case in ("sqa", "sqb"):
        sel = fx[f"{case}_sel"]
        o = fx[f"{case}_o"]
        hq = o.shape[1]
        sel2 = np.broadcast_to(sel[:, None], (sel.shape[0], hq)) if sel.ndim == 1 else sel
        assert np.all(o[~sel2] == 0) and np.all(np.isnan(fx[f"{case}_lse"][~sel2]))
        assert np.all(fx[f"{case}_dq"][~sel2] == 0)
    v = f32(fx["sqa_v"])
    np.testing.assert_allclose(fx["sqa_o"][0, 0], v[0, 0], rtol=1e-6)
    for s in fx["swa_cu"][:-1]:
        np.testing.assert_allclose(fx["swa_o"][s, 1], f32(fx["swa_v"])[s, 1], rtol=1e-6)
    assert np.all(fx["dec_out"][2] == 0)


# ---------------------------------------------------------------- GPU half


@pytest.mark.gpu
def test_gpu_compaction_matches_golden(gpu, fx):
    from logo_amd.ops import build_selection, compute_q_start_blk, prepare_chunk_indices
    from logo_amd.ops.common import compact_selection

    cu = torch.from_numpy(fx["cmp_cu"]).to(gpu)
    n = int(fx["cmp_cu"][-1])
    info = build_selection(torch.from_numpy(fx["cmp_sel"]).to(gpu)[None], 1, n, cu_seqlens=cu)
    assert np.array_equal(info.q_idx.cpu().numpy(), fx["cmp_tok0_q_idx"])
    assert np.array_equal(info.pos_ids.cpu().numpy(), fx["cmp_tok0_pos"])
    assert np.array_equal(info.cu_seqlens_q.cpu().numpy(), fx["cmp_tok0_cu_q"])
    for bt in (16, 64):
        ck = prepare_chunk_indices(cu, bt)
        assert np.array_equal(ck.cpu().numpy(), fx[f"cmp_chunks_{bt}"])
        qs = compute_q_start_blk(info.pos_ids, info, ck, bt)
        assert np.array_equal(qs.cpu().numpy(), fx[f"cmp_q_start_{bt}"])
    dsel = compact_selection(torch.from_numpy(fx["cmp_sel_heads"]).to(gpu), cu)
    for li in range(fx["cmp_sel_heads"].shape[1]):
        sq = dsel.sq(li)
        assert np.array_equal(dsel.q_idx[li, :sq].cpu().numpy(), fx[f"cmp_heads{li}_q_idx"])
        assert np.array_equal(dsel.pos[li, :sq].cpu().numpy(), fx[f"cmp_heads{li}_pos"])
        assert np.array_equal(dsel.cu_seqlens_q(li).cpu().numpy(), fx[f"cmp_heads{li}_cu_q"])


@pytest.mark.gpu
@pytest.mark.parametrize("case", ATTN_CASES)
def test_gpu_attention_matches_golden(gpu, fx, case):
    from logo_amd.ops import sq_full_attn, swa_attn

    q, k, v, do = (bf16_tensor(fx[f"{case}_{n}"], gpu)[None] for n in ("q", "k", "v", "do"))
    q, k, v = (x.requires_grad_() for x in (q, k, v))
    cu = torch.from_numpy(fx[f"{case}_cu"]).to(gpu)
    if f"{case}_window" in fx:
        o = swa_attn(q, k, v, cu, window=int(fx[f"{case}_window"]))
    else:
        o = sq_full_attn(q, k, v, torch.from_numpy(fx[f"{case}_sel"]).to(gpu)[None], cu_seqlens=cu)
    o.backward(do)
    torch.cuda.synchronize()
    for name, got in (("o", o), ("dq", q.grad), ("dk", k.grad), ("dv", v.grad)):
        assert_within(f"{case}_{name}", got[0], fx[f"{case}_{name}"])


@pytest.mark.gpu
def test_gpu_epilogue_matches_golden(gpu, fx):
    from logo_amd.ops.epilogue import logo_epilogue

    L, G, gate, w_l, w_g, dout = (bf16_tensor(fx[f"epi_{n}"], gpu) for n in ("L", "G", "gate", "w_l", "w_g", "dout"))
    L, G, gate, w_l, w_g = (x.requires_grad_() for x in (L, G, gate, w_l, w_g))
    thres = torch.tensor([float(fx["epi_thres"])], dtype=torch.bfloat16, device=gpu)
    out = logo_epilogue(L, G, gate, thres, w_l, w_g, float(fx["epi_eps"]))
    out.backward(dout)
    got = out.detach().float().cpu().numpy()
    ref_bf = f32(fx["epi_out_bf16"])
    assert (got == ref_bf).mean() >= 0.98
    ref = fx["epi_out"].astype(np.float64)
    err = np.abs(got - ref)
    assert (err / np.maximum(1.0, np.abs(ref))).max() <= 2e-2 and err.mean() <= 2e-3
    for name, t in (("dL", L.grad), ("dG", G.grad)):
        r = fx[f"epi_{name}"].astype(np.float64)
        e = np.abs(t.float().cpu().numpy() - r)
        assert (e / np.maximum(1.0, np.abs(r))).max() <= 2e-2 and e.mean() <= 2e-3, name
    for name, t in (("dgate", gate.grad), ("dw_l", w_l.grad), ("dw_g", w_g.grad)):
        r = fx[f"epi_{name}"].astype(np.float64)
        e = np.abs(t.float().cpu().numpy() - r)
        assert e.max() <= 1e-2 * max(1.0, np.abs(r).max()), name


@pytest.mark.gpu
def test_gpu_decode_matches_golden(gpu, fx):
    from logo_amd.ops.decode import decode_attn

    q, k, v, gate = (bf16_tensor(fx[f"dec_{n}"], gpu) for n in ("q", "k", "v", "gate"))
    lens = torch.from_numpy(fx["dec_lens"]).to(gpu)
    thres = torch.tensor([float(fx["dec_thres"])], dtype=torch.bfloat16, device=gpu)
    out = decode_attn(q, k, v, lens, gate, thres, max_len=int(fx["dec_lens"].max()))
    assert_within("dec_out", out, fx["dec_out"])
    assert_within("dec_out_all", decode_attn(q, k, v, lens, max_len=int(fx["dec_lens"].max())), fx["dec_out_all"])
