// Query-sparse causal attention backward, dq (logo/ops/selected_full_attn.py:141-228,
// :424-432), for gfx950: P and dS recomputed from the stored log2-domain LSE
// and delta, dq rows scattered in bf16.
#include "sq_attn.hpp"

namespace logo {

// ---------------------------------------------------------------------------
// Backward dq, 64 rows per wave
// ---------------------------------------------------------------------------
// Two waves x 64 compacted rows (two 32-row blocks) per workgroup (kBQ = 128),
// one wave per SIMD and two workgroups per CU, so every K / V operand read from
// LDS feeds the MFMAs of both row blocks (half the LDS traffic per MFMA of 32
// rows per wave).  Q, dO (MFMA B
// operands) and the dQ accumulators live in AGPRs; S and dP in VGPRs.
// Keys are processed in 32-key halves; step (t, h) of key tile t runs
//   X: the S^T / dP^T MFMAs of the next half ((t, 1) or (t + 1, 0)) while the
//      VALU forms P = exp2(S c - lse) and dS = P (dP - delta) of half (t, h)
//      (delta, and in sparse mode lse, enter as the accumulators' start
//      values);
//   Y: the dQ^T += K^T dS^T MFMAs of half (t, h).
// K and V tiles (64 keys) sit in two LDS slots each (slot = tile & 1).
// K(t + 1) is copied during step (t, 0), after K(t - 1)'s last read (step
// (t - 1, 1)); V(t + 2) during step (t, 1), after V(t)'s last read (step
// (t, 0)).  Every step ends with the copy wait and a barrier.
template <typename EL, int D, bool SPARSE, bool WINDOW>
__global__ __launch_bounds__(128) LOGO_OCC_DQ64 void sq_dq64_kernel(const AttnArgs a) {
  using E8 = typename Elem<EL>::x8;
  using E4 = typename Elem<EL>::x4;
  constexpr int DS = D / 16, DT = D / 32;
  constexpr int NX = 2 * DS;    // X slots: K row operand (even), V row operand (odd)
  constexpr int NY = 2 * DT;    // Y slots: K^T operands (16-key step hh, column block dt)
  constexpr int IX = 16 / NX;   // VALU items per X slot and row block (16 per half)
  constexpr int PF = 2;         // operand prefetch distance, in slots
  using GT = TileGeom<D, kSwz>;
  bf16* const smem = dyn_smem();
  auto tileK = [&](int b) { return smem + b * GT::ELEMS; };
  auto tileV = [&](int b) { return smem + 2 * GT::ELEMS + b * GT::ELEMS; };

  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, i = l & 31, g = l >> 5;
  QTile<SPARSE> qt;
  if (!qt.init(a, wave, i, WINDOW, 64, false, !WINDOW)) {
    if constexpr (SPARSE) zero_empty_lane<D>(a, a.dq, nullptr, qt, 128);
    return;
  }
  const int hq = qt.hq, W = a.window;
  int rr[2], pr[2];
  bool vr[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    rr[b] = qt.r0 + 64 * wave + 32 * b + i;
    vr[b] = rr[b] < qt.r_end;
    pr[b] = vr[b] ? qt.rv.posn(rr[b]) : -1;
  }

  E8 qreg[2][DS], doreg[2][DS];
  float lse_q[2], delta_q[2];
  {
    const QSide<D, SPARSE> qs(a, a.q_sel, a.q, hq), os(a, a.do_sel, a.dout, hq);
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int rc = vr[b] ? rr[b] : qt.r0;
      const bf16* qrow = qs.row(rc) + 8 * g;
      const bf16* orow = os.row(rc) + 8 * g;
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) {
        qreg[b][ds] = vr[b] ? *reinterpret_cast<const E8*>(qrow + 16 * ds) : E8{};
        doreg[b][ds] = vr[b] ? *reinterpret_cast<const E8*>(orow + 16 * ds) : E8{};
      }
      lse_q[b] = vr[b] ? a.lse[(int64_t)hq * a.n + rr[b]] : 0.f;
      delta_q[b] = vr[b] ? a.delta[(int64_t)hq * a.n + rr[b]] : 0.f;
    }
  }
  const float c = a.scale_log2;
  // Sparse mode reads the delta phase's copies q_sel = bf16(-c q) and
  // do_sel = -dO, so the S accumulators start from lse (a splat C operand,
  // fixed for the workgroup's rows): P = exp2(-S'); dP' = -dP gives the
  // negated dS = P (dP' + delta), which leaves dQ negated.  The dP
  // accumulators start from a delta splat in the same way (+delta in sparse
  // mode, -delta in dense mode), so dS is one multiply per score.
  constexpr bool NEG = SPARSE;
  f32x16 c_lse[2], c_del[2];
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      c_lse[b][j] = NEG ? lse_q[b] : 0.f;
      c_del[b][j] = NEG ? delta_q[b] : -delta_q[b];
    }
  const float dq_mul = NEG ? -a.scale : a.scale;

  f32x16 dqacc[2][DT];  // AGPRs
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) dqacc[b][dt] = f32x16{};
  f32x16 sp[2][2][2];  // [half parity][row block][S, dP]
  E8 dsb[2][2];    // dS of the current half as B operands [row block][16-key step]

  TileReader<D, kSwz> rd;
  rd.init();
  const int64_t rstride = (int64_t)a.h * D;
  const bf16* kbase = a.k + ((int64_t)qt.bos * a.h + qt.h) * D;
  const bf16* vbase = a.v + ((int64_t)qt.bos * a.h + qt.h) * D;
  const int seqlen = qt.seqlen;
  TileBufDma<D, 2> dma;
  dma.init((int)rstride);
  auto load_one = [&](bf16* tile, const bf16* src, int j0) {
    if (j0 + 64 <= seqlen) dma.issue(tile, src + j0 * rstride);
    else dma.issue_clamped(tile, src + j0 * rstride, seqlen - 1 - j0);
  };

  const int kv_lo = qt.kv_lo;
  const int nt = (qt.kv_hi - kv_lo + 63) >> 6;
  // step t of the walk takes key tile ph(t): ascending, or from the last
  // tile down (qt.desc); the two 32-key halves of a tile go in key order
  const bool desc = qt.desc;
  auto ph = [&](int t) { return desc ? nt - 1 - t : t; };
  int hw_lo = 0, hw_hi = 0;  // 32-key halves (in key order) this wave's rows can see
  if (qt.wave_active) {
    hw_hi = min(2 * nt, ((qt.pmax - kv_lo) >> 5) + 1);
    hw_lo = WINDOW ? (max(0, qt.pmin - W - kv_lo) >> 5) : 0;
  }

  // step (t, H): PAR = t & 1 (K / V slot of tile t)
  auto step = [&](auto par_tag, auto h_tag, int t) {
    constexpr int PAR = decltype(par_tag)::value, H = decltype(h_tag)::value;
    if (H == 0) {
      if (t + 1 < nt) load_one(tileK(PAR ^ 1), kbase, kv_lo + 64 * ph(t + 1));
    } else {
      if (t + 2 < nt) load_one(tileV(PAR), vbase, kv_lo + 64 * ph(t + 2));
    }
    // X reads the next half: rows 32 of tile t (H = 0) or rows 0 of tile t + 1
    const bf16* kx = tileK(H == 0 ? PAR : PAR ^ 1);
    const bf16* vx = tileV(H == 0 ? PAR : PAR ^ 1);
    constexpr int XR = H == 0 ? 32 : 0;
    const bf16* ky = tileK(PAR);  // K^T of the current half, rows 32 H
    // the current half and the next one, as halves in key order (t = -1:
    // only the next half, the first of the walk)
    const int hx = t >= 0 ? 2 * ph(t) + H : -1;
    const int hn = H == 0 ? (t >= 0 ? 2 * ph(t) + 1 : -1) : (t + 1 < nt ? 2 * ph(t + 1) : -1);
    const int j0h = kv_lo + 32 * hx;

    auto body = [&](auto dox_tag, auto dov_tag, auto mask_tag) {
      constexpr bool DOX = decltype(dox_tag)::value;    // S / dP of the next half
      constexpr bool DOV = decltype(dov_tag)::value;    // dS and dQ of the current half
      constexpr bool MASK = decltype(mask_tag)::value;  // the current half crosses a mask edge
      E8 op[NX + NY];
      auto load_op = [&](auto s_c) {
        constexpr int S = decltype(s_c)::value;
        if constexpr (S < NX) {
          if constexpr (DOX) op[S] = rd.template row<EL>(S % 2 ? vx : kx, XR, S / 2);
        } else {
          constexpr int Y = S - NX;
          if constexpr (DOV) op[S] = rd.template tr<EL>(ky, 32 * H + 16 * (Y / DT), Y % DT);
        }
      };
      static_for<PF>([&](auto s_c) { load_op(s_c); });
      int hi[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) hi[b] = pr[b] - j0h - 4 * g;
      static_for<NX + NY>([&](auto s_c) {
        constexpr int S = decltype(s_c)::value;
        __builtin_amdgcn_sched_barrier(0);
        // dS = P dP' of the items whose P was formed in slot s - 1: one slot
        // after their exp2, so that no VALU op reads an exp2 result right
        // behind it (a one-wait-state hazard, which would cost an s_nop)
        auto ds_items = [&](auto b_c, auto s_c) {
          constexpr int B = decltype(b_c)::value, SP = decltype(s_c)::value;
          static_for<IX>([&](auto e_c) {
            constexpr int JJ = SP * IX + decltype(e_c)::value;
            float dsv = sp[H][B][0][JJ] * sp[H][B][1][JJ];
            pin(dsv);
            sp[H][B][1][JJ] = dsv;
          });
        };
        // bf16 packing of a group of eight dS items, one slot after the dS of
        // its last item (its P formed in slot s - 2)
        auto pack = [&](auto b_c, auto s_c) {
          constexpr int B = decltype(b_c)::value, SP = decltype(s_c)::value;
          constexpr int LAST = SP * IX + IX - 1;
          if constexpr (SP >= 0 && LAST % 8 == 7) dsb[B][LAST / 8] = acc_to<EL>(sp[H][B][1], LAST / 8);
        };
        if constexpr (S < NX) {
          // one wave per SIMD issues in order: each MFMA is followed by the
          // VALU items of its row block, which run under it
          constexpr int DSI = S / 2, KIND = S % 2;
          E8 o;
          if constexpr (DOX) o = op[S];
          static_for<2>([&](auto b_c) {
            constexpr int B = decltype(b_c)::value;
            if constexpr (B == 1) __builtin_amdgcn_sched_barrier(0);
            // the slot's scores, anchored ahead of the MFMA (which then
            // separates the anchor from the exp2 that reads them)
            float sv[IX];
            if constexpr (DOV)
              static_for<IX>([&](auto e_c) {
                constexpr int E = decltype(e_c)::value;
                sv[E] = sp[H][B][0][S * IX + E];
                pin(sv[E]);
              });
            if constexpr (DOX) {
              const E8 bop = KIND ? doreg[B][DSI] : qreg[B][DSI];
              const f32x16 c0 = KIND ? c_del[B] : (NEG ? c_lse[B] : f32x16{});
              sp[H ^ 1][B][KIND] = mfma32(o, bop, DSI == 0 ? c0 : sp[H ^ 1][B][KIND]);
            }
            if constexpr (DOV) {
              static_for<IX>([&](auto e_c) {
                constexpr int E = decltype(e_c)::value, JJ = S * IX + E;
                float pv = NEG ? fast_exp2(-sv[E]) : fast_exp2(fmaf(sv[E], c, -lse_q[B]));
                if constexpr (MASK) {
                  constexpr int off = 8 * (JJ / 4) + (JJ % 4);
                  bool vis = off <= hi[B];
                  if (WINDOW) vis = vis && off >= hi[B] - W;
                  if (!vis) pv = 0.f;
                }
                sp[H][B][0][JJ] = pv;
              });
              if constexpr (S >= 1) ds_items(b_c, std::integral_constant<int, S - 1>{});
              pack(b_c, std::integral_constant<int, S - 2>{});
            }
          });
        } else {
          constexpr int Y = S - NX;
          if constexpr (DOV) {
            E8 o = op[S];
            // the last slot's dS items under the first MFMA, their group's
            // packing under the second (first read DT slots later)
            mfma32_agpr_ready(dqacc[0][Y % DT], o, dsb[0][Y / DT]);
            if constexpr (Y == 0) {
              ds_items(std::integral_constant<int, 0>{}, std::integral_constant<int, NX - 1>{});
              ds_items(std::integral_constant<int, 1>{}, std::integral_constant<int, NX - 1>{});
            }
            mfma32_agpr_ready(dqacc[1][Y % DT], o, dsb[1][Y / DT]);
            if constexpr (Y == 0) {
              pack(std::integral_constant<int, 0>{}, std::integral_constant<int, NX - 1>{});
              pack(std::integral_constant<int, 1>{}, std::integral_constant<int, NX - 1>{});
            }
          }
        }
        if constexpr (S + PF < NX + NY) load_op(std::integral_constant<int, S + PF>{});
      });
      __builtin_amdgcn_sched_barrier(0);
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    const bool dox = hn >= 0 && hn >= hw_lo && hn < hw_hi;
    const bool dov = hx >= 0 && hx >= hw_lo && hx < hw_hi;
    const bool mask = (j0h + 31 > qt.pmin) || (WINDOW && j0h < qt.pmax - W);
    if (dox && dov) {
      if (mask) body(T_{}, T_{}, T_{});
      else body(T_{}, T_{}, F_{});
    } else if (dox) {
      body(T_{}, F_{}, F_{});
    } else if (dov) {
      body(F_{}, T_{}, T_{});
    }
    wait_vmem();
    __syncthreads();
  };

  load_one(tileK(0), kbase, kv_lo + 64 * ph(0));
  load_one(tileV(0), vbase, kv_lo + 64 * ph(0));
  wait_vmem();
  __syncthreads();
  step(BufTag<1>{}, BufTag<1>{}, -1);  // S / dP of half (0, 0); copies V(1)
  for (int t = 0; t < nt; t += 2) {
    step(BufTag<0>{}, BufTag<0>{}, t);
    step(BufTag<0>{}, BufTag<1>{}, t);
    if (t + 1 < nt) {
      step(BufTag<1>{}, BufTag<0>{}, t + 1);
      step(BufTag<1>{}, BufTag<1>{}, t + 1);
    }
    if (t + 2 >= nt) agpr_acc_drain();  // the epilogue reads dQ next
  }

  agpr_acc_drain();
  if constexpr (SPARSE)
    if (qt.piece == 0) zero_unselected<D>(a, a.dq, nullptr, qt, 128);
  if (qt.nsplit > 1) {
    // Key-range split: partial dQ of this piece as [wave][row block][dt][item]
    // [lane]; the last piece of the tile to arrive adds the others' to its own.
    constexpr int PQF = 2 * 2 * DT * 16 * 64;  // floats per piece
    float* const part0 = a.part + (int64_t)(hq * 2 * a.split_cap + qt.trank * qt.nper) * PQF;
    {
      float* pq = part0 + (int64_t)qt.piece * PQF + wave * (2 * DT * 16 * 64);
#pragma unroll
      for (int b = 0; b < 2; ++b)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) st_agent(pq + ((b * DT + dt) * 16 + e) * 64 + l, dqacc[b][dt][e]);
    }
    if (!split_arrive(a.cnt + hq * 2 * a.split_cap + qt.trank, qt.nsplit, reinterpret_cast<int*>(smem))) return;
    // sum the pieces in piece order from zero, whichever arrived last, so the
    // result does not depend on the arrival order
    // (one 16-float block at a time, to keep the registers of the main loop)
#pragma unroll
    for (int b = 0; b < 2; ++b)
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
        f32x16 sum = f32x16{};
        for (int pc = 0; pc < qt.nsplit; ++pc) {
          if (pc == qt.piece) {
            sum += dqacc[b][dt];
          } else {
            const float* pq = part0 + (int64_t)pc * PQF + wave * (2 * DT * 16 * 64) + (b * DT + dt) * 16 * 64;
#pragma unroll
            for (int e = 0; e < 16; ++e) sum[e] += ld_agent(pq + e * 64 + l);
          }
        }
        dqacc[b][dt] = sum;
      }
  }
  // dQ leaves through LDS as whole rows: each wave writes its 64 rows (8-byte
  // pieces into swizzled chunks) over the K / V tiles, then 16 lanes store
  // one row's D * 2 bytes together (rows are scattered tokens, each row
  // contiguous).  Stored from the accumulators directly, every 8-byte piece
  // would touch its own row.
  {
    using GT = TileGeom<D, kSwz>;
    __syncthreads();  // every wave is done with the K / V tiles
#pragma unroll
    for (int b = 0; b < 2; ++b) {
      const int rr_ = 32 * b + i;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          E4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (EL)(dqacc[b][dt][4 * q4 + e] * dq_mul);
          // d = 32 dt + 8 q4 + 4 g: half g of chunk 4 dt + q4
          *reinterpret_cast<E4*>(smem + wave * GT::ELEMS + GT::off(rr_, 4 * dt + q4) + 4 * g) = v;
        }
    }
    __syncthreads();
    constexpr int CHR = D / 8;        // 16-byte chunks per row
    constexpr int RPP = 128 / CHR;    // rows per pass (128 threads)
    const int ch = threadIdx.x % CHR;
    const int nrow = qt.r_end - qt.r0;
    for (int r = threadIdx.x / CHR; r < nrow; r += RPP) {
      const int64_t tok = qt.rv.token(qt.r0 + r);
      const u32x4 v = *reinterpret_cast<const u32x4*>(smem + (r >> 6) * GT::ELEMS + GT::off(r & 63, ch));
      st_nt(reinterpret_cast<u32x4*>(a.dq + (tok * a.hq + hq) * D + 8 * ch), v);  // not read back in the step
    }
  }
}

template <int D>
constexpr size_t dq_smem() { return (size_t)4 * TileGeom<D, kSwz>::ELEMS * sizeof(bf16); }

template <typename EL, int D, bool SPARSE, bool WINDOW>
static int launch_dq(const AttnArgs& a_in, hipStream_t st) {
  AttnArgs a = a_in;
  const int64_t ntmax = (a.n + kBQ - 1) / kBQ + a.nseq;
  if (WINDOW) a.split_cap = 0;
  else split_setup(a, 2, dq_part_floats(D));
  const int64_t nblk = std::max<int64_t>(ntmax, 2 * a.split_cap) * a.hq;
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "grid too large");
  auto kern = sq_dq64_kernel<EL, D, SPARSE, WINDOW>;
  LOGO_HIP_CHECK(allow_smem(kern, dq_smem<D>()));
  hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(128), dq_smem<D>(), st, a);
  LOGO_LAUNCH_CHECK("sq_dq64_kernel");
  return LOGO_OK;
}

template <int D, bool SPARSE, bool WINDOW>
static int launch_dq_bf16(const AttnArgs& a, hipStream_t st) { return launch_dq<bf16, D, SPARSE, WINDOW>(a, st); }

int sq_launch_dq(const AttnArgs& a, hipStream_t st, int d, bool sparse, bool window, bool half) {
  if (half) return d == 128 ? launch_dq<f16, 128, true, false>(a, st) : launch_dq<f16, 64, true, false>(a, st);
  return LOGO_DISPATCH(launch_dq_bf16, a, st, d, sparse, window);
}

}  // namespace logo
