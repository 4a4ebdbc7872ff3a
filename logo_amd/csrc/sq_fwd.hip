// Query-sparse causal attention forward for gfx950 (logo/ops/selected_full_attn.py:33-121,
// :340-362): compacted query rows gathered in the kernel, K / V streamed
// through LDS, online softmax in the exp2 domain, o rows scattered in place.
#include "sq_attn.hpp"

namespace logo {

// ---------------------------------------------------------------------------
// Forward, software-pipelined inside each wave
// ---------------------------------------------------------------------------
// Iteration t of the workgroup loop (t = -1 .. nt - 1; key tile t starts at
// kv_lo + 64 t) runs two phases of MFMA slots on every wave:
//   X: the S^T MFMAs of tile t + 1 (K(t+1) rows from LDS), while the VALU turns
//      the first part of S(t) into P(t) = exp2(S c - base), sums it and packs
//      it to bf16;
//   Y: the O += V(t)^T P(t) MFMAs, key step by key step, while the VALU
//      finishes P(t) ahead of the key steps that read it, masks S(t+1) and
//      takes its row max.
// The row statistics of tile t + 1 (new reference max, rescale of O and l)
// follow Y.  K therefore runs one tile ahead of V: iteration t reads K(t+1)
// from K slot (t+1)&1 and V(t) from V slot t&1, and loads K(t+2) into K slot
// t&1 and V(t+1) into V slot (t+1)&1, both last read in iteration t - 1.
// Each wave only works on the tiles its own rows can see ([tw_lo, tw_hi));
// outside them it still copies its share of the tiles and meets the barriers.
// NW waves x 32 rows per workgroup (kBQ = 128 rows, or two tiles with 8
// waves), two waves per SIMD.
//
// Online softmax with a lazy rescale: the reference max of a row moves only
// when the row's max grew by more than 2^8 in the exp2 domain (or on its first
// visible key), so O and l are rarely rescaled and P <= 2^8 stays exact.
// Masks compare a compile-time offset per accumulator item with one per-lane
// bound: key j0 + 32 kk + rowmap(g, jj) is visible iff its offset from
// j0 + 4 g lies in [hi - W, hi], hi = p - j0 - 4 g.
template <typename EL, int D, bool SPARSE, bool WINDOW, int NW>
__global__ __launch_bounds__(64 * NW) LOGO_OCC_FWD void sq_fwd_pipe_kernel(const AttnArgs a) {
  using E8 = typename Elem<EL>::x8;
  using E4 = typename Elem<EL>::x4;
  constexpr int DS = D / 16, DT = D / 32;
  constexpr int NX = 2 * DS;   // S MFMAs per tile (two 32-key halves x DS k-steps)
  constexpr int NY = 4 * DT;   // PV MFMAs per tile (DT column blocks x 4 key steps)
  constexpr int IY = 32 / NY;  // mask / max items per Y slot
  // The 32 P items of a tile (per lane) are spread evenly over the X slots and
  // the first three quarters of Y less one slot (the 8-wave form: the first
  // half less one, measured 0.8% faster there; its 4-wave form would spill):
  // PV runs key-step major (Y slot y: key step y / DT, column block y % DT),
  // so pb[k] is first read at Y slot DT k, and the softmax work is split
  // between both phases instead of crowding X.  An item's exp2 runs in its
  // slot, its row-sum add and its bf16 packing one slot later.
  constexpr int NPS = NX + (NW == 8 ? 2 : 3) * DT - 1;  // slots that carry P items
  constexpr auto pslot = [](int it) constexpr { return it * NPS / 32; };
  // first item of slot s (items of slot s: [pfirst(s), pfirst(s + 1)))
  constexpr auto pfirst = [](int s) constexpr { return (32 * s + NPS - 1) / NPS < 32 ? (32 * s + NPS - 1) / NPS : 32; };
  constexpr int kMaxPerSlot = (32 + NPS - 1) / NPS;
  static_assert(pfirst(NPS) == 32 && pslot(pfirst(1)) == 1 && pslot(pfirst(1) - 1) == 0, "slot ranges");
  // a group is packed one slot after its last item
  static_assert(pslot(7) + 1 < NX && pslot(15) + 1 < NX + DT && pslot(23) + 1 < NX + 2 * DT &&
                    pslot(31) + 1 < NX + 3 * DT,
                "each group of eight P items is packed before its PV MFMAs");
  constexpr int PF = 4;        // operand prefetch distance, in slots
  using GT = TileGeom<D, kSwz>;
  bf16* const smem = dyn_smem();
  auto tileK = [&](int b) { return smem + b * GT::ELEMS; };
  auto tileV = [&](int b) { return smem + 2 * GT::ELEMS + b * GT::ELEMS; };

  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, i = l & 31, g = l >> 5;
  QTile<SPARSE> qt;
  if (!qt.init(a, wave, i, WINDOW, 32, NW == 8, !WINDOW)) {
    if constexpr (SPARSE) zero_empty_lane<D>(a, a.o, a.lse, qt, 64 * NW);
    return;
  }
  const int hq = qt.hq, p = qt.p, W = a.window;

  // Sparse mode holds q pre-scaled and negated, bf16(-c q) with
  // c = scale * log2(e), the same rounding as the backward's compacted copies:
  // S' = -c q.k, so the forward's LSE and the backward's recomputed P come
  // from identical products.  Scores are then in the exp2 domain already,
  // masked scores are +inf and the row statistic is a minimum.
  constexpr bool NEG = SPARSE;
  E8 qreg[DS];
  {
    const bf16* qrow = a.q + (qt.t * a.hq + hq) * D + 8 * g;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      const E8 qv = qt.valid ? *reinterpret_cast<const E8*>(qrow + 16 * ds) : E8{};
      qreg[ds] = NEG ? scale8(qv, -a.scale_log2) : qv;
    }
  }

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  f32x16 sbuf[2][2];  // [t & 1][32-key half]: S of the current and the next tile
  E8 pb[4];       // P(t) as the B operand of PV, one per 16-key step
  float m_run = -INFINITY, l_run = 0.f, base = 0.f;  // m_run: running row max of c s
  // NEG: the S' accumulators start from the row's current base (a splat C
  // operand), so they hold S' + base and P = exp2(-acc) needs no add; when a
  // tile moves the base, its accumulators are shifted once by the difference.
  f32x16 cbase = f32x16{};
  const float c = a.scale_log2;

  TileReader<D, kSwz> rd;  // K read along rows, V transposed
  rd.init();
  const int64_t rstride = (int64_t)a.h * D;
  const bf16* kbase = a.k + ((int64_t)qt.bos * a.h + qt.h) * D;
  const bf16* vbase = a.v + ((int64_t)qt.bos * a.h + qt.h) * D;
  const int seqlen = qt.seqlen;
  TileBufDma<D, NW> dma;
  dma.init((int)rstride);
  // rows past the sequence end are clamped to its last key (masked: p < seqlen)
  auto load_one = [&](bf16* tile, const bf16* src, int j0) {
    if (j0 + 64 <= seqlen) dma.issue(tile, src + j0 * rstride);
    else dma.issue_clamped(tile, src + j0 * rstride, seqlen - 1 - j0);
  };

  const int kv_lo = qt.kv_lo;
  const int nt = (qt.kv_hi - kv_lo + 63) >> 6;
  // step t of the walk takes key tile ph(t): ascending, or from the last
  // tile down (qt.desc)
  const bool desc = qt.desc;
  auto ph = [&](int t) { return desc ? nt - 1 - t : t; };
  int tw_lo = 0, tw_hi = 0;  // steps whose tiles this wave's rows can see
  if (qt.wave_active) {
    tw_hi = min(nt, ((qt.pmax - kv_lo) >> 6) + 1);
    tw_lo = WINDOW ? (max(0, qt.pmin - W - kv_lo) >> 6) : 0;
    if (desc) {
      const int lo = nt - tw_hi;
      tw_hi = nt - tw_lo;
      tw_lo = lo;
    }
  }

  auto step = [&](auto par_tag, int t) {
    constexpr int PAR = decltype(par_tag)::value;  // t & 1
    if (t + 2 < nt) load_one(tileK(PAR), kbase, kv_lo + 64 * ph(t + 2));
    if (t + 1 < nt) load_one(tileV(PAR ^ 1), vbase, kv_lo + 64 * ph(t + 1));
    const bf16* kb = tileK(PAR ^ 1);
    const bf16* vb = tileV(PAR);
    const int j0n = kv_lo + 64 * ph(t + 1);

    auto body = [&](auto dos_tag, auto dopv_tag, auto mask_tag) {
      constexpr bool DOS = decltype(dos_tag)::value;    // S(t+1) and its statistics
      constexpr bool DOPV = decltype(dopv_tag)::value;  // P(t) and O += V^T P
      constexpr bool MASK = decltype(mask_tag)::value;  // S(t+1) crosses a mask edge
      // slot s < NX: K row operand (half s / DS, k-step s % DS);
      // slot s >= NX: V^T operand (key step (s - NX) / DT, column block (s - NX) % DT)
      E8 op[NX + NY];
      auto load_op = [&](auto s_c) {
        constexpr int S = decltype(s_c)::value;
        if constexpr (S < NX) {
          if constexpr (DOS) op[S] = rd.template row<EL>(kb, 32 * (S / DS), S % DS);
        } else {
          if constexpr (DOPV) op[S] = rd.template tr<EL>(vb, 16 * ((S - NX) / DT), (S - NX) % DT);
        }
      };
      static_for<PF>([&](auto s_c) { load_op(s_c); });
      const int hi = p - j0n - 4 * g;  // mask bound of S(t+1) items
      float mx = NEG ? INFINITY : -INFINITY, psum = 0.f;
      static_for<NX + NY>([&](auto s_c) {
        constexpr int S = decltype(s_c)::value;
        __builtin_amdgcn_sched_barrier(0);
        // the slot's P(t) scores (items [pfirst(S), pfirst(S + 1))), anchored
        // ahead of its MFMA (which then separates the anchor from the exp2
        // that reads them)
        constexpr int I0 = pfirst(S), NI = pfirst(S + 1) - I0;
        float spv[kMaxPerSlot];
        if constexpr (DOPV)
          static_for<NI>([&](auto i_c) {
            constexpr int I = decltype(i_c)::value, IT = I0 + I;
            spv[I] = sbuf[PAR][IT / 16][IT % 16];
            pin(spv[I]);
          });
        if constexpr (S < NX) {
          if constexpr (DOS) {
            constexpr int KK = S / DS, DSI = S % DS;
            const E8 o = op[S];
            sbuf[PAR ^ 1][KK] = mfma32(o, qreg[DSI], DSI == 0 ? (NEG ? cbase : f32x16{}) : sbuf[PAR ^ 1][KK]);
          }
        } else {
          constexpr int Y = S - NX;
          if constexpr (DOPV) {
            const E8 o = op[S];
            oacc[Y % DT] = mfma32(o, pb[Y / DT], oacc[Y % DT]);
          }
          if constexpr (DOS) {
            float sv[IY];
            static_for<IY>([&](auto e_c) {
              constexpr int E = decltype(e_c)::value, IT = Y * IY + E;
              constexpr int KK = IT / 16, JJ = IT % 16;
              sv[E] = sbuf[PAR ^ 1][KK][JJ];
              // the masked path rewrites S, so it anchors its value here; the
              // unmasked path only reads it (the max3 asm keeps the order),
              // and an anchor would force a copy of every score
              if constexpr (MASK) pin(sv[E]);
              if constexpr (MASK) {
                constexpr int off = 32 * KK + 8 * (JJ / 4) + (JJ % 4);
                bool vis = off <= hi;
                if (WINDOW) vis = vis && off >= hi - W;
                if (!vis) sv[E] = NEG ? INFINITY : -INFINITY;
                sbuf[PAR ^ 1][KK][JJ] = sv[E];
              }
            });
#pragma unroll
            for (int e = 0; e < IY; e += 2)
              mx = NEG ? min3_f32(mx, sv[e], sv[e + 1]) : max3_f32(mx, sv[e], sv[e + 1]);
          }
        }
        // P(t) items assigned to this slot (X or Y); the row sum and the bf16
        // packing of the previous slot's items, one slot after their exp2
        // (a VALU op right behind an exp2 that wrote its input would cost an
        // s_nop)
        if constexpr (DOPV) {
          static_for<NI>([&](auto i_c) {
            constexpr int I = decltype(i_c)::value, IT = I0 + I;
            float pv = NEG ? fast_exp2(-spv[I]) : fast_exp2(fmaf(spv[I], c, -base));
            pin(pv);
            sbuf[PAR][IT / 16][IT % 16] = pv;
          });
          if constexpr (S >= 1) {
            constexpr int J0 = pfirst(S - 1), NJ = I0 - J0;
            static_for<NJ>([&](auto i_c) {
              constexpr int IT = J0 + decltype(i_c)::value;
              psum += sbuf[PAR][IT / 16][IT % 16];
              if constexpr (IT % 8 == 7) pb[IT / 8] = acc_to<EL>(sbuf[PAR][IT / 16], (IT / 8) & 1);
            });
            if constexpr (NJ > 0) pin(psum);
          }
        }
        if constexpr (S + PF < NX + NY) load_op(std::integral_constant<int, S + PF>{});
      });
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (DOPV) l_run += psum;
      if constexpr (DOS) {
        // tile max of c s (NEG: the accumulators hold base - c s)
        const float mxs = NEG ? base - pair_min(mx) : pair_max(mx) * c;
        const bool grow = mxs - m_run > 8.f;
        const bool any_grow = __ballot(grow);
        const float m_new = any_grow ? fmaxf(m_run, mxs) : m_run;
        const float nbase = (m_new == -INFINITY) ? 0.f : m_new;
        const float alpha = fast_exp2(m_run - nbase);
        l_run *= alpha;
        m_run = m_new;
        if (NEG && any_grow) {
          // rebase the next tile's scores (S' + base -> S' + nbase) and the splat
          const float shift = nbase - base;
#pragma unroll
          for (int kk = 0; kk < 2; ++kk) sbuf[PAR ^ 1][kk] += shift;
#pragma unroll
          for (int j = 0; j < 16; ++j) cbase[j] = nbase;
        }
        base = nbase;
        if (__ballot(alpha != 1.f)) {
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
        }
      }
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    const bool doS = t + 1 >= tw_lo && t + 1 < tw_hi;
    const bool doPV = t >= tw_lo && t < tw_hi;
    const bool maskn = (j0n + 63 > qt.pmin) || (WINDOW && j0n < qt.pmax - W);
    if (doS && doPV) {
      if (maskn) body(T_{}, T_{}, T_{});
      else body(T_{}, T_{}, F_{});
    } else if (doS) {
      body(T_{}, F_{}, T_{});
    } else if (doPV) {
      body(F_{}, T_{}, F_{});
    }
    wait_vmem();
    __syncthreads();
  };

  load_one(tileK(0), kbase, kv_lo + 64 * ph(0));
  wait_vmem();
  __syncthreads();
  for (int t = -1; t < nt; t += 2) {
    step(BufTag<1>{}, t);
    if (t + 1 < nt) step(BufTag<0>{}, t + 1);
  }

  float l_tot = pair_sum(l_run);
  if constexpr (SPARSE)
    if (qt.piece == 0) zero_unselected<D>(a, a.o, a.lse, qt, 64 * NW);
  if (qt.nsplit > 1) {
    // Key-range split: store this piece's partial (O unnormalised, relative to
    // its base m_run; per row m_run and l) as [wave][dt][item][lane]; the last
    // piece of the tile to arrive rescales all of them to the largest base.
    constexpr int OF = DT * 16 * 64;  // O floats per wave
    float* const part0 = a.part + (int64_t)(hq * 2 * a.split_cap + qt.trank * qt.nper) * NW * (OF + 64);
    {
      float* po = part0 + (int64_t)qt.piece * NW * (OF + 64) + wave * (OF + 64);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int e = 0; e < 16; ++e) st_agent(po + (dt * 16 + e) * 64 + l, oacc[dt][e]);
      st_agent(po + OF + l, g == 0 ? m_run : l_tot);
    }
    if (!split_arrive(a.cnt + hq * 2 * a.split_cap + qt.trank, qt.nsplit, reinterpret_cast<int*>(smem))) return;
    // combine in piece order from zero, whichever arrived last, so the
    // result does not depend on the arrival order
    float mc[kMaxSplit], lc[kMaxSplit];
    float mx = -INFINITY;
    for (int pc = 0; pc < qt.nsplit; ++pc) {
      const float* po = part0 + (int64_t)pc * NW * (OF + 64) + wave * (OF + 64);
      mc[pc] = pc == qt.piece ? m_run : ld_agent(po + OF + i);
      lc[pc] = pc == qt.piece ? l_tot : ld_agent(po + OF + 32 + i);
      if (lc[pc] > 0.f) mx = fmaxf(mx, mc[pc]);
    }
    f32x16 osum[DT];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) osum[dt] = f32x16{};
    float lsum = 0.f;
    for (int pc = 0; pc < qt.nsplit; ++pc) {
      const float w = lc[pc] > 0.f ? fast_exp2(mc[pc] - mx) : 0.f;
      if (pc == qt.piece) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) osum[dt][e] = fmaf(w, oacc[dt][e], osum[dt][e]);
      } else {
        const float* po = part0 + (int64_t)pc * NW * (OF + 64) + wave * (OF + 64);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt)
#pragma unroll
          for (int e = 0; e < 16; ++e) osum[dt][e] = fmaf(w, ld_agent(po + (dt * 16 + e) * 64 + l), osum[dt][e]);
      }
      lsum = fmaf(w, lc[pc], lsum);
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] = osum[dt];
    l_tot = lsum;
    m_run = mx;
  }
  // O leaves through LDS as whole rows: each wave writes its 32 rows (8-byte
  // pieces into swizzled chunks) over the K / V tiles, then 16 lanes store
  // one row's D * 2 bytes together (the rows are scattered tokens, but each
  // row is contiguous).  Stored from the accumulators directly, every 8-byte
  // piece would touch its own row.
  {
    using GT = TileGeom<D, kSwz>;
    const float inv = qt.valid ? 1.f / l_tot : 0.f;
    if (qt.valid && g == 0) a.lse[(int64_t)hq * a.n + qt.r] = m_run + log2f(l_tot);
    __syncthreads();  // every wave is done with the K / V tiles
    bf16* const blk = reinterpret_cast<bf16*>(smem);  // NW * 32 rows in 64-row tiles
    const int row = 32 * wave + i;
    bf16* const orow = blk + (row >> 6) * GT::ELEMS;
    const int rr = row & 63;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        E4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (EL)(oacc[dt][4 * q4 + e] * inv);
        // d = 32 dt + 8 q4 + 4 g: half g of chunk 4 dt + q4
        *reinterpret_cast<E4*>(orow + GT::off(rr, 4 * dt + q4) + 4 * g) = v;
      }
    __syncthreads();
    constexpr int CHR = D / 8;           // 16-byte chunks per row
    constexpr int RPP = NW * 64 / CHR;   // rows per pass
    const int ch = threadIdx.x % CHR;
    const int nrow = qt.r_end - qt.r0;
    for (int r = threadIdx.x / CHR; r < nrow; r += RPP) {
      const int64_t tok = qt.rv.token(qt.r0 + r);
      const u32x4 v = *reinterpret_cast<const u32x4*>(blk + (r >> 6) * GT::ELEMS + GT::off(r & 63, ch));
      *reinterpret_cast<u32x4*>(a.o + (tok * a.hq + hq) * D + 8 * ch) = v;
    }
  }
}

template <int D>
constexpr size_t fwd_smem() { return (size_t)4 * TileGeom<D, kSwz>::ELEMS * sizeof(bf16); }

template <typename EL, int D, bool SPARSE, bool WINDOW>
static int launch_fwd(const AttnArgs& a_in, hipStream_t st) {
  AttnArgs a = a_in;
  const bool paired = a.nseq == 1 && a.n >= kFwdPairMinTokens;
  const int64_t rows = paired ? 2 * kBQ : kBQ;
  const int64_t ntmax = (a.n + rows - 1) / rows + a.nseq;
  if (WINDOW) a.split_cap = 0;
  else split_setup(a, paired ? 1 : 2, fwd_part_floats(D, paired ? 8 : 4));
  const int64_t nblk = std::max<int64_t>(ntmax, 2 * a.split_cap) * a.hq;
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "grid too large");
  if (paired) {
    auto kern = sq_fwd_pipe_kernel<EL, D, SPARSE, WINDOW, 8>;
    LOGO_HIP_CHECK(allow_smem(kern, fwd_smem<D>()));
    hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(512), fwd_smem<D>(), st, a);
  } else {
    auto kern = sq_fwd_pipe_kernel<EL, D, SPARSE, WINDOW, 4>;
    LOGO_HIP_CHECK(allow_smem(kern, fwd_smem<D>()));
    hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(256), fwd_smem<D>(), st, a);
  }
  LOGO_LAUNCH_CHECK("sq_fwd_pipe_kernel");
  return LOGO_OK;
}

template <int D, bool SPARSE, bool WINDOW>
static int launch_fwd_bf16(const AttnArgs& a, hipStream_t st) { return launch_fwd<bf16, D, SPARSE, WINDOW>(a, st); }

int sq_launch_fwd(const AttnArgs& a, hipStream_t st, int d, bool sparse, bool window, bool half) {
  if (window && swa_fwd_applies(a, sparse, half)) return swa_launch_fwd(a, st, d);
  if (half) return d == 128 ? launch_fwd<f16, 128, true, false>(a, st) : launch_fwd<f16, 64, true, false>(a, st);
  return LOGO_DISPATCH(launch_fwd_bf16, a, st, d, sparse, window);
}

}  // namespace logo
