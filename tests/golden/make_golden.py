"""Writes tests/golden/logo_golden.npz: small input/output vectors for every
function on the LoGo attention hot path, produced by the CPU oracle
(``oracle/``) in float64.

The reference ships no golden vectors or known-answer tests for this path (its
one test, tests/test_model.py, only prints), so the fixtures come from the
oracle, which tests/test_oracle_*.py pin by closed forms, brute force and
torch autograd.  Committing them freezes the oracle's answers: a later change
to the oracle that moves any of them fails tests/test_golden.py on the CPU,
and the GPU half of that file checks the HIP kernels against the same vectors.

Inputs are generated with numpy's PCG64 from the seeds below, rounded to bf16
and stored as raw bf16 bit patterns (uint16); outputs are float32 (integer
outputs in their own dtypes).  Regenerate with
``python tests/golden/make_golden.py`` from the repository root.

Cases (reference file:line of the behaviour each one fixes):
  cmp_*   compaction, per token and per head, with an empty and a one-token
          segment (logo/ops/common.py:71-107), tile lists
          (logo/ops/common.py:110-124) and dK/dV start blocks
          (logo/ops/selected_full_attn.py:374-402);
  sqa_*   query-sparse attention fwd+bwd, per-token selection, GQA (HQ=4,
          H=2), D=64, varlen with an empty segment
          (logo/ops/selected_full_attn.py:449-527);
  sqb_*   the same with the per-(token, head) selection extension, D=128;
  swa_*   sliding-window attention, window 16, D=64, two segments
          (logo/layers/utils.py:144-147);
  epi_*   gate-threshold / RMSNorm / fusion epilogue fwd (bf16 rounding
          chain) and bwd (logo/layers/logo.py:180-181, :225-226, :256-258;
          logo/modules/layernorm.py:17-22);
  dec_*   gate-aware decode over a ragged cache (logo/layers/logo.py:228-249).
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

from oracle import attn, compact, decode, epilogue  # noqa: E402

OUT = os.path.join(HERE, "logo_golden.npz")


def bf16_bits(x):
    """Round float32 to bf16 (nearest even) and return the uint16 bit patterns."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def from_bits(b):
    return (b.astype(np.uint32) << 16).view(np.float32)


def bf16_randn(rng, shape, scale=1.0):
    return bf16_bits(rng.standard_normal(shape).astype(np.float32) * np.float32(scale))


def attn_case(prefix, rng, n, hq, h, d, cu, selection, window=None):
    q = bf16_randn(rng, (n, hq, d), 0.5)
    k = bf16_randn(rng, (n, h, d), 0.5)
    v = bf16_randn(rng, (n, h, d))
    do = bf16_randn(rng, (n, hq, d))
    qf, kf, vf, dof = (from_bits(x) for x in (q, k, v, do))
    o, lse = attn.sq_attn_fwd(qf, kf, vf, selection, cu, window=window)
    dq, dk, dv = attn.sq_attn_bwd(qf, kf, vf, o, dof, selection, cu, window=window)
    out = {f"{prefix}_q": q, f"{prefix}_k": k, f"{prefix}_v": v, f"{prefix}_do": do,
           f"{prefix}_cu": np.asarray(cu, dtype=np.int32),
           f"{prefix}_o": o.astype(np.float32), f"{prefix}_lse": lse.astype(np.float32),
           f"{prefix}_dq": dq.astype(np.float32), f"{prefix}_dk": dk.astype(np.float32),
           f"{prefix}_dv": dv.astype(np.float32)}
    if selection is not None:
        out[f"{prefix}_sel"] = np.asarray(selection, dtype=bool)
    if window is not None:
        out[f"{prefix}_window"] = np.int32(window)
    return out


def make():
    rng = np.random.Generator(np.random.PCG64(20260101))
    fx = {}

    # compaction: segments of 120, 0, 1 and 179 tokens
    cu = np.array([0, 120, 120, 121, 300], dtype=np.int32)
    sel = rng.random(300) < 0.4
    sel[0] = True
    sel_h = rng.random((300, 3)) < 0.3
    fx["cmp_cu"], fx["cmp_sel"], fx["cmp_sel_heads"] = cu, sel, sel_h
    for name, s in (("tok", sel), ("heads", sel_h)):
        lanes = compact.build_selection(s, cu)
        for li, lane in enumerate(lanes):
            fx[f"cmp_{name}{li}_q_idx"] = lane["q_idx"]
            fx[f"cmp_{name}{li}_pos"] = lane["pos_ids"]
            fx[f"cmp_{name}{li}_cu_q"] = lane["cu_seqlens_q"]
    lane = compact.build_selection(sel, cu)[0]
    for bt in (16, 64):
        ck = compact.prepare_chunk_indices(cu, bt)
        fx[f"cmp_chunks_{bt}"] = ck
        fx[f"cmp_q_start_{bt}"] = compact.compute_q_start_blk(lane["pos_ids"], lane["cu_seqlens_q"], cu, bt, 300)

    # query-sparse attention, per token, GQA, D=64, segments 40 / 0 / 56
    n = 96
    sel_a = rng.random(n) < 0.5
    sel_a[0] = True
    fx.update(attn_case("sqa", rng, n, 4, 2, 64, [0, 40, 40, 96], sel_a))

    # per-(token, head) selection, D=128, one segment
    n = 64
    sel_b = rng.random((n, 2)) < 0.5
    sel_b[0, :] = True
    fx.update(attn_case("sqb", rng, n, 2, 1, 128, [0, n], sel_b))

    # sliding window 16, D=64, segments 30 / 34
    fx.update(attn_case("swa", rng, 64, 2, 2, 64, [0, 30, 64], None, window=16))

    # epilogue: 16 tokens x 2 heads x 128
    n, H, D = 16, 2, 128
    L = bf16_randn(rng, (n, H, D))
    G = bf16_randn(rng, (n, H, D))
    gate = from_bits(bf16_bits(1.0 / (1.0 + np.exp(-rng.standard_normal(n).astype(np.float32)))))
    G_f = from_bits(G)
    G_f[gate < 0.5] = 0.0  # unselected global rows are zero (sq_full_attn output)
    G = bf16_bits(G_f)
    w_l = bf16_bits(1 + 0.1 * rng.standard_normal(D).astype(np.float32))
    w_g = bf16_bits(1 + 0.1 * rng.standard_normal(D).astype(np.float32))
    dout = bf16_randn(rng, (n, H * D))
    eps, thres = 1e-5, 0.5
    Lf, Gf, wl, wg, dof = (from_bits(x) for x in (L, G, w_l, w_g, dout))
    out_bf = epilogue.epilogue_fwd(Lf, Gf, gate, thres, wl, wg, eps, bf16=True)
    out64 = epilogue.epilogue_fwd(Lf, Gf, gate, thres, wl, wg, eps, bf16=False)
    dL, dG, dgate, dwl, dwg = epilogue.epilogue_bwd(Lf, Gf, gate, thres, wl, wg, eps, dof)
    fx.update({"epi_L": L, "epi_G": G, "epi_gate": bf16_bits(gate), "epi_w_l": w_l, "epi_w_g": w_g,
               "epi_dout": dout, "epi_eps": np.float32(eps), "epi_thres": np.float32(thres),
               "epi_out_bf16": bf16_bits(out_bf), "epi_out": out64.astype(np.float32),
               "epi_dL": dL.astype(np.float32), "epi_dG": dG.astype(np.float32),
               "epi_dgate": dgate.astype(np.float32), "epi_dw_l": dwl.astype(np.float32),
               "epi_dw_g": dwg.astype(np.float32)})

    # decode: batch 3, HQ=4, H=2, D=128, ragged lengths, one inactive row
    B, HQ, H, D, T = 3, 4, 2, 128, 48
    lens = np.array([48, 1, 37], dtype=np.int32)
    q = bf16_randn(rng, (B, HQ, D))
    k = bf16_randn(rng, (B, H, T, D), 0.5)
    v = bf16_randn(rng, (B, H, T, D))
    gate_d = bf16_bits(np.array([0.75, 0.625, 0.25], dtype=np.float32))
    active = from_bits(gate_d) >= 0.5
    qf, kf, vf = (from_bits(x) for x in (q, k, v))
    fx.update({"dec_q": q, "dec_k": k, "dec_v": v, "dec_lens": lens, "dec_gate": gate_d,
               "dec_thres": np.float32(0.5),
               "dec_out": decode.decode_attn(qf, kf, vf, lens, active).astype(np.float32),
               "dec_out_all": decode.decode_attn(qf, kf, vf, lens, None).astype(np.float32)})
    return fx


if __name__ == "__main__":
    fixtures = make()
    np.savez_compressed(OUT, **fixtures)
    print(f"wrote {OUT}: {len(fixtures)} arrays, {os.path.getsize(OUT)} bytes")
