// Query-sparse causal attention backward, dk / dv with the GQA sum
// (logo/ops/selected_full_attn.py:231-337, :433-445), for gfx950: K and V of
// a 128-key block held in registers, the compacted query rows streamed
// through LDS, dK / dV of the whole group stored once in bf16.
#include "sq_attn.hpp"

namespace logo {

// ---------------------------------------------------------------------------
// Backward dk / dv
// ---------------------------------------------------------------------------
// Query rows staged per LDS buffer: two 64-row sub-tiles per step, half the
// barriers, copy issues and step bookkeeping per row of 64-row steps.  Two
// stages take 131 KB (one workgroup per CU, as its registers already allow);
// the second stage's LDS addresses lie past the 64 KB reach of the
// instruction offset, so the compiler keeps them in spare AGPRs.
constexpr int kDkvRows = 128;
constexpr int kDkvStages = 2;
template <int D>
constexpr int dkv_stage_bytes() { return 2 * kDkvRows * D * 2 + 3 * kDkvRows * 4; }

template <typename EL, int D, bool SPARSE, bool WINDOW>
__global__ __launch_bounds__(256) LOGO_OCC_DKV void sq_dkv_kernel(const AttnArgs a) {
  using E8 = typename Elem<EL>::x8;
  using E4 = typename Elem<EL>::x4;
  constexpr int DS = D / 16, DT = D / 32;
  using GQ = TileGeom<D, kSwz>;  // Q and dO read along rows (S, dP) and transposed (dK, dV)
  char* const smem_b = logo_smem;
  constexpr int RS = kDkvRows, NSUB = RS / 64;
  static_assert(GQ::ELEMS == 64 * D, "64-row swizzled tiles");
  // stage b: [Q rows][dO rows][lse][delta][pos], RS rows each; Q and dO as
  // NSUB consecutive 64-row swizzled tiles
  auto sQ = [&](int b) { return reinterpret_cast<bf16*>(smem_b + b * dkv_stage_bytes<D>()); };
  auto sO = [&](int b) { return sQ(b) + RS * D; };
  auto sLse = [&](int b) { return reinterpret_cast<float*>(sQ(b) + 2 * RS * D); };
  auto sDelta = [&](int b) { return sLse(b) + RS; };
  auto sPos = [&](int b) { return reinterpret_cast<int*>(sLse(b) + 2 * RS); };

  int rank, h;
  xcd_remap(blockIdx.x, a.h, rank, h);
  const int32_t* meta0 = a.meta;
  const int ntk = meta0[2];
  if (rank >= ntk) return;
  const int tile = rank;  // early key blocks (most queries) first
  const int32_t* cu_tk = meta0 + kMetaHdr + 2 * (a.nseq + 1);
  const int s = seg_of(cu_tk, a.nseq, tile);
  const int k0 = (tile - cu_tk[s]) * kBKV;
  const int bos = a.cu[s];
  const int seqlen = a.cu[s + 1] - bos;
  const int k_last = min(k0 + kBKV, seqlen) - 1;

  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, i = l & 31, g = l >> 5;
  const int kw0 = k0 + 32 * wave;
  const bool wave_active = kw0 < seqlen;
  const int kw_last = min(kw0 + 31, seqlen - 1);
  const int key = kw0 + i;
  const bool valid_k = key < seqlen;
  const int W = a.window;
  const float c = a.scale_log2;
  // Sparse mode streams the delta phase's copies q_sel = bf16(-c q) and
  // do_sel = -dO: the S and dP accumulators then start from lse and delta
  // (loaded as the MFMAs' C operands), P = exp2(-S') and the negated
  // dS = P dP', which leaves dK scaled by c and dV negated.
  constexpr bool NEG = SPARSE;
  const float dk_mul = NEG ? a.scale / a.scale_log2 : a.scale;
  const float dv_mul = NEG ? -1.f : 1.f;

  E8 kreg[DS], vreg[DS];
  {
    const int64_t off = ((int64_t)(bos + key) * a.h + h) * D + 8 * g;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      kreg[ds] = valid_k ? *reinterpret_cast<const E8*>(a.k + off + 16 * ds) : E8{};
      vreg[ds] = valid_k ? *reinterpret_cast<const E8*>(a.v + off + 16 * ds) : E8{};
    }
  }
  f32x16 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dkacc[dt] = f32x16{};
    dvacc[dt] = f32x16{};
  }

  TileReader<D, kSwz> rd;
  rd.init();
  // q / dO rows: stride D (compacted copies) or HQ * D (dense inputs).  The
  // copies are buffer loads: a FLAT-encoded copy in flight would make every
  // LDS operand wait of the compute phases a full lgkmcnt(0) drain.
  TileBufDma<D> dma;
  dma.init(SPARSE ? D : a.hq * D);
  float lse_n = 0.f, delta_n = 0.f;
  int pos_n = -1;
  for (int gg = 0; gg < a.g; ++gg) {
    const int hq = h * a.g + gg;
    const int lane_sel = a.lanes > 1 ? hq : 0;
    const int32_t* cu_q = a.meta + (int64_t)lane_sel * a.meta_stride + kMetaHdr;
    const RowView<SPARSE> rv = row_view<SPARSE>(a, lane_sel, bos);
    const QSide<D, SPARSE> qs(a, a.q_sel, a.q, hq), os(a, a.do_sel, a.dout, hq);
    const int q_lo = cu_q[s], q_hi = cu_q[s + 1];
    // first row in [lo, hi) whose position is >= x (rows ascend by position;
    // dense rows are the positions themselves)
    auto lb_pos = [&](int lo, int hi, int x) {
      return SPARSE ? wave_lower_bound(rv.ps, lo, hi, x) : min(max(q_lo + x, lo), hi);
    };
    const int rq0 = lb_pos(q_lo, q_hi, k0);
    const int rq_end = WINDOW ? lb_pos(rq0, q_hi, k_last + W + 1) : q_hi;
    // This wave's keys kw0 .. kw_last: rows before lb0 see none of them,
    // rows from lb1 on see all of them (causally), rows from lb2 on are past
    // the window of the last one.
    int lb0 = rq_end, lb1 = rq_end, lb2 = rq_end;
    if (wave_active && rq0 < rq_end) {
      lb0 = lb_pos(rq0, rq_end, kw0);
      lb1 = lb_pos(lb0, rq_end, kw_last);
      if (WINDOW) lb2 = lb_pos(lb1, rq_end, kw_last + W + 1);
    }
    const float* lse_h = a.lse + (int64_t)hq * a.n;
    const float* delta_h = a.delta + (int64_t)hq * a.n;
    auto load_tile = [&](int rt, int b) {
      if (tid < RS) {
        const int rr = rt + tid;
        const bool ok = rr < rq_end;
        const int rc = min(rr, rq_end - 1);
        lse_n = lse_h[rc];
        delta_n = delta_h[rc];
        pos_n = ok ? rv.posn(rr) : -1;
      }
      // rows past rq_end are clamped to a real row and masked (pos = -1)
      // (last_row may be negative for the second sub-tile: every row then
      // reads row rq_end - 1)
#pragma unroll
      for (int u = 0; u < NSUB; ++u) {
        if (rt + 64 * (u + 1) <= rq_end) {
          dma.issue(sQ(b) + 64 * D * u, qs.row(rt + 64 * u));
          dma.issue(sO(b) + 64 * D * u, os.row(rt + 64 * u));
        } else {
          dma.issue_clamped(sQ(b) + 64 * D * u, qs.row(rt + 64 * u), rq_end - 1 - rt - 64 * u);
          dma.issue_clamped(sO(b) + 64 * D * u, os.row(rt + 64 * u), rq_end - 1 - rt - 64 * u);
        }
      }
    };
    auto store_stats = [&](int b) {
      if (tid < RS) {
        sLse(b)[tid] = lse_n;
        sDelta(b)[tid] = delta_n;
        sPos(b)[tid] = pos_n;
      }
    };

    // Two LDS stages: step t computes from stage t % 2 while the copy for
    // step t + 1 lands in the other.
    auto step = [&](auto buf_tag, int rt) {
      constexpr int B = decltype(buf_tag)::value;
      const bool has_next = rt + RS < rq_end;
      if (has_next) load_tile(rt + RS, B ^ 1);
      const bf16* qb = sQ(B);
      const bf16* ob = sO(B);
      const float* lb = sLse(B);
      const float* dlb = sDelta(B);
      const int* pob = sPos(B);
      const int last = min(rt + RS - 1, rq_end - 1);
      // Each 64-row sub-tile as two 32-row halves h0, h1, its MFMAs in eight
      // blocks of DS slots (one wave per SIMD):
      //   S(h0) | dP(h0) | S(h1) | dP(h1) | dV(h0) | dK(h0) | dV(h1) | dK(h1)
      // The softmax arithmetic of a half is split into P = exp2(S*c - lse)
      // (needs S) and dS = P * (dP - delta) (needs dP and P), placed under
      // blocks 1-2 (P of h0), 3 (dS of h0), 4-5 (P of h1) and 6 (dS of h1),
      // so six of the eight blocks carry VALU work.  A slot is one MFMA, its
      // share of the arithmetic and the LDS read of the operand used PF slots
      // later (across sub-tiles too).  Scheduling fences between slots keep
      // this order, so the VALU work issues under the MFMAs.
      auto compute = [&](auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        constexpr int NS = 2 * DS;  // MFMAs per half and pass: S and dP over D / 16 k-steps
        constexpr int SPT = 4 * NS; // slots per sub-tile
        constexpr int PF = 4;       // operand prefetch distance, in slots
        constexpr int IPP = 16 / (2 * DS);  // P items per slot (over two blocks)
        constexpr int IPD = 16 / DS;        // dS items per slot (over one block)
        static_assert(IPP * 2 * DS == 16 && IPD * DS == 16, "a half has 16 row items per lane");
        f32x16 sacc[2], pacc[2];
        E8 pbf[2][2], dbf[2][2];  // [half][hh]
        E8 opA[NSUB * 2 * NS];    // S/dP operands: Q rows / dO rows
        E8 opC[NSUB * 2 * NS];    // dV/dK operands: dO^T / Q^T
        f32x4 l4[NSUB][2][4], d4[NSUB][2][4];
        int4 p4[NSUB][2][4];
        // A operand a of sub-tile u: half a / NS; S (first DS) or dP (next DS), k-step a % DS
        auto load_a = [&](auto u_c, auto a_c) {
          constexpr int U = decltype(u_c)::value, A = decltype(a_c)::value;
          constexpr int QQ = A / NS, KK = A % NS;
          opA[U * 2 * NS + A] = rd.template row<EL>(KK >= DS ? ob : qb, 64 * U + 32 * QQ, KK % DS);
        };
        // C operand c of sub-tile u: half c / NS; dV (first DS) or dK (next DS); hh, dt
        auto load_c = [&](auto u_c, auto c_c) {
          constexpr int U = decltype(u_c)::value, C = decltype(c_c)::value;
          constexpr int QQ = C / NS, KK = C % NS, HH = (KK % DS) / DT, DTI = KK % DT;
          opC[U * 2 * NS + C] = rd.template tr<EL>(KK >= DS ? qb : ob, 64 * U + 16 * (2 * QQ + HH), DTI);
        };
        // the operand first used at slot T
        auto load_for_slot = [&](auto t_c) {
          constexpr int T = decltype(t_c)::value, U = T / SPT, L = T % SPT;
          if constexpr (L < 2 * NS) load_a(std::integral_constant<int, U>{}, std::integral_constant<int, L>{});
          else load_c(std::integral_constant<int, U>{}, std::integral_constant<int, L - 2 * NS>{});
        };
        // lse / positions (P) and delta (dS) of query rows 64u + 32qq + 8m + 4g + (0..3)
        auto load_pstats = [&](int u, int qq, int m) {
          const int qr = 64 * u + 32 * qq + 8 * m + 4 * g;
          if constexpr (!NEG) l4[u][qq][m] = lds_load(reinterpret_cast<const f32x4*>(lb + qr));
          if constexpr (MASK) p4[u][qq][m] = lds_load(reinterpret_cast<const int4*>(pob + qr));
        };
        auto load_dstats = [&](int u, int qq, int m) {
          const int qr = 64 * u + 32 * qq + 8 * m + 4 * g;
          d4[u][qq][m] = lds_load(reinterpret_cast<const f32x4*>(dlb + qr));
        };
        // NEG: the 16 lse (delta) values of a half, the initial accumulator of
        // its S (dP) MFMAs; item j of the accumulator is query row rowmap(g, j)
        auto load_lse_half = [&](int u, int qq) {
#pragma unroll
          for (int m = 0; m < 4; ++m)
            l4[u][qq][m] = lds_load(reinterpret_cast<const f32x4*>(lb + 64 * u + 32 * qq + 8 * m + 4 * g));
        };
        auto load_delta_half = [&](int u, int qq) {
#pragma unroll
          for (int m = 0; m < 4; ++m) load_dstats(u, qq, m);
        };
        auto cat16 = [](const f32x4 (&v)[4]) -> f32x16 {
          const auto lo = __builtin_shufflevector(v[0], v[1], 0, 1, 2, 3, 4, 5, 6, 7);
          const auto hi = __builtin_shufflevector(v[2], v[3], 0, 1, 2, 3, 4, 5, 6, 7);
          return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
        };
        auto mfma_a = [&](auto u_c, auto a_c) {
          constexpr int U = decltype(u_c)::value, A = decltype(a_c)::value;
          constexpr int QQ = A / NS, KK = A % NS;
          const E8 op = opA[U * 2 * NS + A];
          if constexpr (KK < DS) {
            const f32x16 c0 = NEG ? cat16(l4[U][QQ]) : f32x16{};
            sacc[QQ] = mfma32(op, kreg[KK], KK == 0 ? c0 : sacc[QQ]);
          } else {
            const f32x16 c0 = NEG ? cat16(d4[U][QQ]) : f32x16{};
            pacc[QQ] = mfma32(op, vreg[KK - DS], KK == DS ? c0 : pacc[QQ]);
          }
        };
        auto mfma_c = [&](auto u_c, auto c_c) {
          constexpr int U = decltype(u_c)::value, C = decltype(c_c)::value;
          constexpr int QQ = C / NS, KK = C % NS, HH = (KK % DS) / DT, DTI = KK % DT;
          const E8 op = opC[U * 2 * NS + C];
          // D = 128: P and dS are packed at least four slots before their MFMAs
          // read them; D = 64 (four-slot blocks) keeps the leading wait states
          if constexpr (DS >= 8) {
            if constexpr (KK < DS) mfma32_agpr_ready(dvacc[DTI], op, pbf[QQ][HH]);
            else mfma32_agpr_ready(dkacc[DTI], op, dbf[QQ][HH]);
          } else {
            if constexpr (KK < DS) mfma32_agpr(dvacc[DTI], op, pbf[QQ][HH]);
            else mfma32_agpr(dkacc[DTI], op, dbf[QQ][HH]);
          }
        };
        // row item jj of half qq: items 4m..4m+3 are query rows 32qq + 8m + 4g + e.
        // An item's inputs are anchored ahead of its slot's MFMA (which then
        // separates the anchor from the VALU op that reads them), its
        // arithmetic follows the MFMA, and pairs of items are packed to bf16
        // one slot later: a VALU op right behind an anchor or an exp2 that
        // wrote its input would cost an s_nop.  P items leave P in sacc
        // (fp32), dS items leave dS in pacc.
        auto p_pre = [&](int qq, auto jj_c) {
          constexpr int JJ = decltype(jj_c)::value;
          float sv = sacc[qq][JJ];
          pin(sv);
          return sv;
        };
        auto p_item = [&](auto u_c, int qq, auto jj_c, float sv) {
          constexpr int U = decltype(u_c)::value, JJ = decltype(jj_c)::value;
          constexpr int M = JJ / 4, E = JJ % 4;
          // NEG: sv = lse - c s, so P = exp2(-sv) (the negation is a source modifier)
          float pv = NEG ? fast_exp2(-sv) : fast_exp2(fmaf(sv, c, -l4[U][qq][M][E]));
          if constexpr (MASK) {
            const int pq = p4[U][qq][M][E];
            bool vis = key <= pq;
            if (WINDOW) vis = vis && key >= pq - W;
            if (!vis) pv = 0.f;
          }
          pin(pv);
          sacc[qq][JJ] = pv;
        };
        auto p_pack = [&](int qq, auto jj_c) {
          constexpr int JJ = decltype(jj_c)::value;
          if constexpr (JJ % 2 == 1) {
            pbf[qq][JJ / 8][JJ % 8 - 1] = (EL)sacc[qq][JJ - 1];
            pbf[qq][JJ / 8][JJ % 8] = (EL)sacc[qq][JJ];
          }
          // a finished group stays here: sunk to its MFMA, the packing would
          // write the operand too close before it
          if constexpr (JJ % 8 == 7) pin(pbf[qq][JJ / 8]);
        };
        auto ds_pre = [&](int qq, auto jj_c, float& pv, float& dpv) {
          constexpr int JJ = decltype(jj_c)::value;
          pv = sacc[qq][JJ];
          dpv = pacc[qq][JJ];
          pin(pv);
          pin(dpv);
        };
        auto ds_item = [&](auto u_c, int qq, auto jj_c, float pv, float dpv) {
          constexpr int U = decltype(u_c)::value, JJ = decltype(jj_c)::value;
          constexpr int M = JJ / 4, E = JJ % 4;
          // NEG: dpv = delta - dP, and dS is kept negated (dO was negated too)
          float dsv = NEG ? pv * dpv : pv * (dpv - d4[U][qq][M][E]);
          pin(dsv);
          pacc[qq][JJ] = dsv;
        };
        auto ds_pack = [&](int qq, auto jj_c) {
          constexpr int JJ = decltype(jj_c)::value;
          if constexpr (JJ % 2 == 1) {
            dbf[qq][JJ / 8][JJ % 8 - 1] = (EL)pacc[qq][JJ - 1];
            dbf[qq][JJ / 8][JJ % 8] = (EL)pacc[qq][JJ];
          }
          if constexpr (JJ % 8 == 7) pin(dbf[qq][JJ / 8]);
        };
        // stats of (sub-tile u, half qq, group m) are read DS/2 slots before
        // the first item of group m needs them; the P items of half qq start at
        // block 1 + 3qq, its dS items at block 3 + 3qq
        auto pstats_slot = [](int u, int qq, int m) { return SPT * u + DS * (1 + 3 * qq) + 4 * m / IPP - DS / 2; };
        auto dstats_slot = [](int u, int qq, int m) { return SPT * u + DS * (3 + 3 * qq) + 4 * m / IPD - DS / 2; };
        // NEG: lse (delta) of half qq are read LD slots before its first S (dP)
        // MFMA, blocks 0 / 2 (1 / 3) of the sub-tile; negative slots go in the
        // prologue
        constexpr int LD = DS / 2;
        auto lse_slot = [](int u, int qq) { return SPT * u + 2 * DS * qq - LD; };
        auto delta_slot = [](int u, int qq) { return SPT * u + DS * (2 * qq + 1) - LD; };

        if constexpr (NEG) {
#pragma unroll
          for (int u = 0; u < NSUB; ++u)
#pragma unroll
            for (int qq = 0; qq < 2; ++qq) {
              if (lse_slot(u, qq) < 0) load_lse_half(u, qq);
              if (delta_slot(u, qq) < 0) load_delta_half(u, qq);
            }
        }
        static_for<PF>([&](auto t_c) { load_for_slot(t_c); });
        static_for<NSUB * SPT>([&](auto s_c) {
          constexpr int S = decltype(s_c)::value, U = S / SPT, L = S % SPT;
          constexpr int BLK = L / DS, K = L % DS;
          using UC = std::integral_constant<int, U>;
          __builtin_amdgcn_sched_barrier(0);
          // the slot's P items (blocks 1, 2, 4, 5) and dS items (blocks 3, 6)
          constexpr bool HASP = BLK == 1 || BLK == 2 || BLK == 4 || BLK == 5, HASD = BLK == 3 || BLK == 6;
          constexpr int QP = BLK >= 4, JP = ((BLK - 1) % 3) * DS + K, QD = BLK == 6;
          float sv[IPP], pv[IPD], dpv[IPD];
          if constexpr (HASP)
            static_for<IPP>([&](auto i_c) {
              constexpr int I = decltype(i_c)::value;
              sv[I] = p_pre(QP, std::integral_constant<int, JP * IPP + I>{});
            });
          if constexpr (HASD)
            static_for<IPD>([&](auto i_c) {
              constexpr int I = decltype(i_c)::value;
              ds_pre(QD, std::integral_constant<int, K * IPD + I>{}, pv[I], dpv[I]);
            });
          if constexpr (L < 2 * NS) mfma_a(UC{}, std::integral_constant<int, L>{});
          else mfma_c(UC{}, std::integral_constant<int, L - 2 * NS>{});
          if constexpr (S + PF < NSUB * SPT) load_for_slot(std::integral_constant<int, S + PF>{});
#pragma unroll
          for (int u = 0; u < NSUB; ++u)
#pragma unroll
            for (int qq = 0; qq < 2; ++qq) {
              if (NEG) {
                if (lse_slot(u, qq) == S) load_lse_half(u, qq);
                if (delta_slot(u, qq) == S) load_delta_half(u, qq);
              }
#pragma unroll
              for (int m = 0; m < 4; ++m) {
                if ((MASK || !NEG) && pstats_slot(u, qq, m) == S) load_pstats(u, qq, m);
                if (!NEG && dstats_slot(u, qq, m) == S) load_dstats(u, qq, m);
              }
            }
          if constexpr (HASP)
            static_for<IPP>([&](auto i_c) {
              constexpr int I = decltype(i_c)::value;
              p_item(UC{}, QP, std::integral_constant<int, JP * IPP + I>{}, sv[I]);
            });
          if constexpr (HASD)
            static_for<IPD>([&](auto i_c) {
              constexpr int I = decltype(i_c)::value;
              ds_item(UC{}, QD, std::integral_constant<int, K * IPD + I>{}, pv[I], dpv[I]);
            });
          // the previous slot's items, packed (no item is formed in block 0 or
          // 7, so a sub-tile's packs stay inside it; a group of eight is first
          // read DT slots after its last pack at the earliest)
          if constexpr (L >= 1) {
            constexpr int LB = (L - 1) / DS, LK = (L - 1) % DS;
            if constexpr (LB == 1 || LB == 2 || LB == 4 || LB == 5)
              static_for<IPP>([&](auto i_c) {
                p_pack(LB >= 4, std::integral_constant<int, (((LB - 1) % 3) * DS + LK) * IPP + decltype(i_c)::value>{});
              });
            if constexpr (LB == 3 || LB == 6)
              static_for<IPD>([&](auto i_c) {
                ds_pack(LB == 6, std::integral_constant<int, LK * IPD + decltype(i_c)::value>{});
              });
          }
        });
        __builtin_amdgcn_sched_barrier(0);
      };
      // the step's last row is before lb0 (sees none of the wave's keys) or
      // its first row is past lb2 (past the window); rows before lb1, the
      // window and clamped rows past rq_end need the mask
      const bool skip = !wave_active || last < lb0 || (WINDOW && rt >= lb2);
      if (!skip) {
        const bool need_mask = WINDOW || rt < lb1 || (rt + RS > rq_end);
        if (need_mask) compute(std::true_type{});
        else compute(std::false_type{});
      }
      if (has_next) store_stats(B ^ 1);
      else agpr_acc_drain();  // the head's last step: dK / dV may be read next
      wait_vmem();
      __syncthreads();
    };

    if (rq0 < rq_end) {
      load_tile(rq0, 0);
      store_stats(0);
    }
    wait_vmem();
    __syncthreads();
    for (int rt = rq0; rt < rq_end; rt += 2 * RS) {
      step(BufTag<0>{}, rt);
      if (rt + RS < rq_end) step(BufTag<1>{}, rt + RS);
    }
  }

  agpr_acc_drain();
  // dK and dV leave through LDS (free after the last step's barrier) as whole
  // rows: each wave writes its 32 keys' rows (8-byte pieces into swizzled
  // chunks), then 16 lanes store one row's D * 2 bytes together.  Stored from
  // the accumulators directly, every 8-byte piece would touch its own row.
  {
    using GT = TileGeom<D, kSwz>;
    bf16* const blk_k = reinterpret_cast<bf16*>(smem_b);  // 128 rows: two 64-row tiles
    bf16* const blk_v = blk_k + 2 * GT::ELEMS;
    const int row = 32 * wave + i, rr = row & 63;
    bf16* const rk = blk_k + (row >> 6) * GT::ELEMS;
    bf16* const rv_ = blk_v + (row >> 6) * GT::ELEMS;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        E4 kv, vv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kv[e] = (EL)(dkacc[dt][4 * q4 + e] * dk_mul);
          vv[e] = (EL)(dvacc[dt][4 * q4 + e] * dv_mul);
        }
        // d = 32 dt + 8 q4 + 4 g: half g of chunk 4 dt + q4
        *reinterpret_cast<E4*>(rk + GT::off(rr, 4 * dt + q4) + 4 * g) = kv;
        *reinterpret_cast<E4*>(rv_ + GT::off(rr, 4 * dt + q4) + 4 * g) = vv;
      }
    __syncthreads();
    constexpr int CHR = D / 8;      // 16-byte chunks per row
    constexpr int RPP = 256 / CHR;  // rows per pass
    const int ch = tid % CHR;
    const int nkey = min(kBKV, seqlen - k0);
    for (int r = tid / CHR; r < nkey; r += RPP) {
      const int64_t off = ((int64_t)(bos + k0 + r) * a.h + h) * D + 8 * ch;
      const int lo = (r >> 6) * GT::ELEMS + GT::off(r & 63, ch);
      // non-temporal: the step reads dK / dV no more (four packed sequences
      // of 32K tokens in all: dk/dv -2%)
      st_nt(reinterpret_cast<u32x4*>(a.dk + off), *reinterpret_cast<const u32x4*>(blk_k + lo));
      st_nt(reinterpret_cast<u32x4*>(a.dv + off), *reinterpret_cast<const u32x4*>(blk_v + lo));
    }
  }
}

template <int D>
constexpr size_t dkv_smem() { return (size_t)kDkvStages * dkv_stage_bytes<D>(); }

template <typename EL, int D, bool SPARSE, bool WINDOW>
static int launch_dkv(const AttnArgs& a, hipStream_t st) {
  const int64_t ntmax = (a.n + kBKV - 1) / kBKV + a.nseq;
  auto kern = sq_dkv_kernel<EL, D, SPARSE, WINDOW>;
  LOGO_HIP_CHECK(allow_smem(kern, dkv_smem<D>()));
  hipLaunchKernelGGL(kern, dim3((unsigned)(ntmax * a.h)), dim3(256), dkv_smem<D>(), st, a);
  LOGO_LAUNCH_CHECK("sq_dkv_kernel");
  return LOGO_OK;
}

template <int D, bool SPARSE, bool WINDOW>
static int launch_dkv_bf16(const AttnArgs& a, hipStream_t st) { return launch_dkv<bf16, D, SPARSE, WINDOW>(a, st); }

int sq_launch_dkv(const AttnArgs& a, hipStream_t st, int d, bool sparse, bool window, bool half) {
  if (half) return d == 128 ? launch_dkv<f16, 128, true, false>(a, st) : launch_dkv<f16, 64, true, false>(a, st);
  return LOGO_DISPATCH(launch_dkv_bf16, a, st, d, sparse, window);
}

}  // namespace logo
