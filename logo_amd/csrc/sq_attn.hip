// Query-sparse causal attention, forward and backward, for gfx950.
//
// Semantics follow logo/ops/selected_full_attn.py: selected ("compacted")
// query rows attend causally to every key of their own packed segment up to
// their real position (:33-121); the backward recomputes P from the stored
// log2-domain LSE (:141-228 dq, :231-337 dk/dv) with delta = rowsum(o * dO)
// (:124-138); dk/dv of a GQA group are summed over its query heads (:444-445).
// Differences in structure, not in results:
//   * the forward gathers q rows and scatters o rows inside the kernel (the
//     reference materialises q_sel / o_sel, :461 :469); the backward's delta
//     pass writes compacted, head-major copies of q and dO ([HQ, N, D]) so the
//     dq and dk/dv loops read contiguous rows (the reference's q_sel / do_sel,
//     :461 :483), and the dq kernel scatters dq rows itself (:487);
//   * the tile -> (sequence, block) map comes from device-side prefixes built
//     by the compaction kernels (no host list, :348 :413-414);
//   * the dk/dv kernel starts each key block at its exact first visible query
//     (the reference rounds down to a block, :374-402) and accumulates the GQA
//     sum in registers, storing bf16 once (no fp32 [N, HQ, D] buffers);
//   * an optional sliding window (keys [p - w, p]) turns the same kernels into
//     the local SWA branch (logo/layers/utils.py:144-147).
//
// Tiling (32x32x16 bf16 MFMA, wave64; kBQ = 128 compacted rows per fwd / dq
// workgroup, kBKV = 128 keys per dk/dv workgroup):
//   fwd   : 4 waves x 32 rows, two waves per SIMD; Q in registers as the B
//           operand, K/V streamed through double-buffered 64-key LDS tiles.
//           Each wave software-pipelines S of the next key tile against the
//           softmax of the current one.
//   dq    : 2 waves x 64 rows (two 32-row blocks), one wave per SIMD, so each
//           K / V operand read from LDS feeds two MFMAs; Q, dO and dQ in
//           AGPRs; S / dP of the next 32-key half pipelined against dS of the
//           current one.
//   dk/dv : 4 waves x 32 keys (K and V in registers), compacted query rows
//           streamed in double-buffered 64-row LDS tiles, GQA heads looped
//           inside the workgroup, an explicit MFMA / VALU / LDS slot schedule.
// S^T = K Q^T puts one query per lane pair, so the softmax row statistics need
// a single cross-lane exchange (lane ^ 32).  Transposed operands (V^T, K^T,
// Q^T, dO^T) come from the same row-major tiles through ds_read_b64_tr_b16.
#include <math.h>

#include <type_traits>

#include "capi.hpp"
#include "common.hpp"

namespace logo {

struct AttnArgs {
  const bf16* q;
  const bf16* k;
  const bf16* v;
  bf16* o;
  float* lse;
  const bf16* dout;
  float* delta;
  bf16* dq;
  bf16* dk;
  bf16* dv;
  bf16* q_sel;   // [HQ, N, D] compacted q rows (sparse backward)
  bf16* do_sel;  // [HQ, N, D] compacted dO rows (sparse backward)
  const int64_t* q_idx;
  const int32_t* pos;
  const int32_t* meta;
  const int32_t* cu;
  int64_t n;
  int nseq;
  int hq;
  int h;
  int g;
  int lanes;
  int meta_stride;
  float scale;
  float scale_log2;
  int window;
};

// Per-lane view of the compaction metadata.
template <bool SPARSE>
struct RowView {
  const int64_t* qi;
  const int32_t* ps;
  int bos;
  __device__ __forceinline__ int64_t token(int r) const { return SPARSE ? qi[r] : (int64_t)r; }
  __device__ __forceinline__ int posn(int r) const { return SPARSE ? ps[r] : r - bos; }
};

template <bool SPARSE>
__device__ __forceinline__ RowView<SPARSE> row_view(const AttnArgs& a, int lane_sel, int bos) {
  RowView<SPARSE> v;
  v.qi = SPARSE ? a.q_idx + (int64_t)lane_sel * a.n : nullptr;
  v.ps = SPARSE ? a.pos + (int64_t)lane_sel * a.n : nullptr;
  v.bos = bos;
  return v;
}

// Query-side rows (q or dO) of head hq as the backward reads them: compacted
// head-major copies [HQ, N, D] in sparse mode, the [N, HQ, D] inputs in dense
// mode (where the compacted row index is the token).
template <int D, bool SPARSE>
struct QSide {
  const bf16* base;
  int64_t stride;
  __device__ __forceinline__ QSide(const AttnArgs& a, const bf16* sel_buf, const bf16* full, int hq) {
    base = SPARSE ? sel_buf + (int64_t)hq * a.n * D : full + (int64_t)hq * D;
    stride = SPARSE ? (int64_t)D : (int64_t)a.hq * D;
  }
  __device__ __forceinline__ const bf16* row(int r) const { return base + (int64_t)r * stride; }
};

// Waves per SIMD each kernel is compiled for (caps VGPRs at 512 / waves).
#ifndef LOGO_OCC_FWD
#define LOGO_OCC_FWD __attribute__((amdgpu_waves_per_eu(2, 2)))
#endif
#ifndef LOGO_OCC_DQ64
#define LOGO_OCC_DQ64 __attribute__((amdgpu_waves_per_eu(1, 1)))
#endif
#ifndef LOGO_OCC_DKV
#define LOGO_OCC_DKV __attribute__((amdgpu_waves_per_eu(1, 1)))
#endif

extern __shared__ __attribute__((aligned(16))) char logo_smem[];
__device__ __forceinline__ bf16* dyn_smem() { return reinterpret_cast<bf16*>(logo_smem); }


// Shared front matter of the fwd and dq kernels: which compacted rows this
// workgroup and this lane own.  Returns false for a workgroup past the last
// tile (the grid is sized for the worst case).
template <bool SPARSE>
struct QTile {
  int hq, h, lane_sel, s, r0, r_end, bos, seqlen;
  int pmin, pmax, r, p, kv_lo, kv_hi;
  bool wave_active, valid;
  int64_t t;
  RowView<SPARSE> rv;

  // rpw: compacted rows per wave (32 or 64); r / t / p / valid describe the
  // lane's row in the wave's first 32-row block (row_at gives the others).
  // paired: the workgroup takes two consecutive kBQ-row tiles (a single
  // segment only, nseq == 1, so both tiles share one key range).
  __device__ __forceinline__ bool init(const AttnArgs& a, int wave, int i, bool window, int rpw = 32,
                                       bool paired = false) {
    int rank;
    xcd_remap(blockIdx.x, a.hq, rank, hq);
    lane_sel = a.lanes > 1 ? hq : 0;
    const int32_t* meta = a.meta + (int64_t)lane_sel * a.meta_stride;
    const int nt = paired ? (meta[1] + 1) >> 1 : meta[1];
    if (rank >= nt) return false;
    const int tile = nt - 1 - rank;  // heaviest (latest) blocks first
    const int32_t* cu_q = meta + kMetaHdr;
    const int32_t* cu_tq = cu_q + (a.nseq + 1);
    if (paired) {
      s = 0;
      r0 = cu_q[0] + tile * 2 * kBQ;
      r_end = min(r0 + 2 * kBQ, cu_q[1]);
    } else {
      s = seg_of(cu_tq, a.nseq, tile);
      r0 = cu_q[s] + (tile - cu_tq[s]) * kBQ;
      r_end = min(r0 + kBQ, cu_q[s + 1]);
    }
    bos = a.cu[s];
    seqlen = a.cu[s + 1] - bos;
    h = hq / a.g;
    rv = row_view<SPARSE>(a, lane_sel, bos);
    const int rw0 = r0 + rpw * wave;
    wave_active = rw0 < r_end;
    pmin = wave_active ? rv.posn(rw0) : 0;
    pmax = wave_active ? rv.posn(min(rw0 + rpw - 1, r_end - 1)) : -1;
    r = rw0 + i;
    valid = r < r_end;
    t = valid ? rv.token(r) : 0;
    p = valid ? rv.posn(r) : -1;
    kv_lo = window ? (max(0, rv.posn(r0) - a.window) & ~63) : 0;
    kv_hi = rv.posn(r_end - 1) + 1;
    return true;
  }
};

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <int B>
using BufTag = std::integral_constant<int, B>;

// ---------------------------------------------------------------------------
// Forward, software-pipelined inside each wave
// ---------------------------------------------------------------------------
// Iteration t of the workgroup loop (t = -1 .. nt - 1; key tile t starts at
// kv_lo + 64 t) runs two phases of MFMA slots on every wave:
//   X: the S^T MFMAs of tile t + 1 (K(t+1) rows from LDS), while the VALU turns
//      S(t) into P(t) = exp2(S c - base), sums it and packs it to bf16;
//   Y: the O += V(t)^T P(t) MFMAs, while the VALU masks S(t+1) and takes its
//      row max.
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
template <int D, bool SPARSE, bool WINDOW, int NW>
__global__ __launch_bounds__(64 * NW) LOGO_OCC_FWD void sq_fwd_pipe_kernel(const AttnArgs a) {
  constexpr int DS = D / 16, DT = D / 32;
  constexpr int NX = 2 * DS;   // S MFMAs per tile (two 32-key halves x DS k-steps)
  constexpr int NY = 4 * DT;   // PV MFMAs per tile (DT column blocks x 4 key steps)
  constexpr int IX = 32 / NX;  // softmax items per X slot
  constexpr int IY = 32 / NY;  // mask / max items per Y slot
  constexpr int PF = 4;        // operand prefetch distance, in slots
  using GT = TileGeom<D, kSwz>;
  bf16* const smem = dyn_smem();
  auto tileK = [&](int b) { return smem + b * GT::ELEMS; };
  auto tileV = [&](int b) { return smem + 2 * GT::ELEMS + b * GT::ELEMS; };

  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, i = l & 31, g = l >> 5;
  QTile<SPARSE> qt;
  if (!qt.init(a, wave, i, WINDOW, 32, NW == 8)) return;
  const int hq = qt.hq, p = qt.p, W = a.window;

  bf16x8 qreg[DS];
  {
    const bf16* qrow = a.q + (qt.t * a.hq + hq) * D + 8 * g;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds)
      qreg[ds] = qt.valid ? *reinterpret_cast<const bf16x8*>(qrow + 16 * ds) : bf16x8{};
  }

  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
  f32x16 sbuf[2][2];  // [t & 1][32-key half]: S of the current and the next tile
  bf16x8 pb[4];       // P(t) as the B operand of PV, one per 16-key step
  float m_run = -INFINITY, l_run = 0.f, base = 0.f;
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
  int tw_lo = 0, tw_hi = 0;  // tiles this wave's rows can see
  if (qt.wave_active) {
    tw_hi = ((qt.pmax - kv_lo) >> 6) + 1;
    tw_lo = WINDOW ? (max(0, qt.pmin - W - kv_lo) >> 6) : 0;
  }

  auto step = [&](auto par_tag, int t) {
    constexpr int PAR = decltype(par_tag)::value;  // t & 1
    if (t + 2 < nt) load_one(tileK(PAR), kbase, kv_lo + 64 * (t + 2));
    if (t + 1 < nt) load_one(tileV(PAR ^ 1), vbase, kv_lo + 64 * (t + 1));
    const bf16* kb = tileK(PAR ^ 1);
    const bf16* vb = tileV(PAR);
    const int j0n = kv_lo + 64 * (t + 1);

    auto body = [&](auto dos_tag, auto dopv_tag, auto mask_tag) {
      constexpr bool DOS = decltype(dos_tag)::value;    // S(t+1) and its statistics
      constexpr bool DOPV = decltype(dopv_tag)::value;  // P(t) and O += V^T P
      constexpr bool MASK = decltype(mask_tag)::value;  // S(t+1) crosses a mask edge
      // slot s < NX: K row operand (half s / DS, k-step s % DS);
      // slot s >= NX: V^T operand (column block (s - NX) / 4, key step (s - NX) % 4)
      bf16x8 op[NX + NY];
      auto load_op = [&](auto s_c) {
        constexpr int S = decltype(s_c)::value;
        if constexpr (S < NX) {
          if constexpr (DOS) op[S] = rd.row(kb, 32 * (S / DS), S % DS);
        } else {
          if constexpr (DOPV) op[S] = rd.tr(vb, 16 * ((S - NX) % 4), (S - NX) / 4);
        }
      };
      static_for<PF>([&](auto s_c) { load_op(s_c); });
      const int hi = p - j0n - 4 * g;  // mask bound of S(t+1) items
      float mx = -INFINITY, psum = 0.f;
      static_for<NX + NY>([&](auto s_c) {
        constexpr int S = decltype(s_c)::value;
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (S < NX) {
          if constexpr (DOS) {
            constexpr int KK = S / DS, DSI = S % DS;
            bf16x8 o = op[S];
            pin(o);
            sbuf[PAR ^ 1][KK] = mfma32(o, qreg[DSI], DSI == 0 ? f32x16{} : sbuf[PAR ^ 1][KK]);
          }
          if constexpr (DOPV) {
            static_for<IX>([&](auto e_c) {
              constexpr int IT = S * IX + decltype(e_c)::value;
              constexpr int KK = IT / 16, JJ = IT % 16;
              float sv = sbuf[PAR][KK][JJ];
              pin(sv);
              float pv = fast_exp2(fmaf(sv, c, -base));
              pin(pv);
              sbuf[PAR][KK][JJ] = pv;
              psum += pv;
              pin(psum);
              if constexpr (IT % 8 == 7) pb[IT / 8] = acc_to_bf16(sbuf[PAR][IT / 16], (IT / 8) & 1);
            });
          }
        } else {
          constexpr int Y = S - NX;
          if constexpr (DOPV) {
            bf16x8 o = op[S];
            pin(o);
            oacc[Y / 4] = mfma32(o, pb[Y % 4], oacc[Y / 4]);
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
                if (!vis) sv[E] = -INFINITY;
                sbuf[PAR ^ 1][KK][JJ] = sv[E];
              }
            });
#pragma unroll
            for (int e = 0; e < IY; e += 2) mx = max3_f32(mx, sv[e], sv[e + 1]);
          }
        }
        if constexpr (S + PF < NX + NY) load_op(std::integral_constant<int, S + PF>{});
      });
      __builtin_amdgcn_sched_barrier(0);
      if constexpr (DOPV) l_run += psum;
      if constexpr (DOS) {
        mx = pair_max(mx);
        const bool grow = (mx - m_run) * c > 8.f;
        const float m_new = __ballot(grow) ? fmaxf(m_run, mx) : m_run;
        const float nbase = (m_new == -INFINITY) ? 0.f : m_new * c;
        const float alpha = fast_exp2(m_run * c - nbase);
        l_run *= alpha;
        m_run = m_new;
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

  load_one(tileK(0), kbase, kv_lo);
  wait_vmem();
  __syncthreads();
  for (int t = -1; t < nt; t += 2) {
    step(BufTag<1>{}, t);
    if (t + 1 < nt) step(BufTag<0>{}, t + 1);
  }

  const float l_tot = pair_sum(l_run);
  if (qt.valid) {
    const float inv = 1.f / l_tot;
    bf16* orow = a.o + (qt.t * a.hq + hq) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (bf16)(oacc[dt][4 * q4 + e] * inv);
        *reinterpret_cast<bf16x4*>(orow + 32 * dt + 8 * q4 + 4 * g) = v;
      }
    if (g == 0) a.lse[(int64_t)hq * a.n + qt.r] = m_run * c + log2f(l_tot);
  }
}

// ---------------------------------------------------------------------------
// Backward preprocess: delta = rowsum(o * dO) per compacted row (fp32); in
// sparse mode also the compacted copies q_sel / do_sel.
// ---------------------------------------------------------------------------
template <int D, bool SPARSE>
__global__ __launch_bounds__(256) void sq_delta_kernel(const AttnArgs a) {
  constexpr int LPR = D / 8;          // lanes per row
  constexpr int RPB = 256 / LPR;      // rows per workgroup
  const int hq = blockIdx.y;
  const int lane_sel = a.lanes > 1 ? hq : 0;
  const int32_t* meta = a.meta + (int64_t)lane_sel * a.meta_stride;
  const int sq = meta[0];
  const int r = blockIdx.x * RPB + threadIdx.x / LPR;
  const int c = threadIdx.x % LPR;
  float acc = 0.f;
  if (r < sq) {
    const int64_t t = SPARSE ? a.q_idx[(int64_t)lane_sel * a.n + r] : (int64_t)r;
    const int64_t off = (t * a.hq + hq) * D + 8 * c;
    const bf16x8 ov = *reinterpret_cast<const bf16x8*>(a.o + off);
    const bf16x8 dv = *reinterpret_cast<const bf16x8*>(a.dout + off);
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf((float)ov[e], (float)dv[e], acc);
    if (SPARSE) {
      const int64_t soff = ((int64_t)hq * a.n + r) * D + 8 * c;
      *reinterpret_cast<bf16x8*>(a.do_sel + soff) = dv;
      *reinterpret_cast<bf16x8*>(a.q_sel + soff) = *reinterpret_cast<const bf16x8*>(a.q + off);
    }
  }
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
  if (r < sq && c == 0) a.delta[(int64_t)hq * a.n + r] = acc;
}

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
//      VALU forms P = exp2(S c - lse) and dS = P (dP - delta) of half (t, h);
//   Y: the dQ^T += K^T dS^T MFMAs of half (t, h).
// K and V tiles (64 keys) sit in two LDS slots each (slot = tile & 1).
// K(t + 1) is copied during step (t, 0), after K(t - 1)'s last read (step
// (t - 1, 1)); V(t + 2) during step (t, 1), after V(t)'s last read (step
// (t, 0)).  Every step ends with the copy wait and a barrier.
template <int D, bool SPARSE, bool WINDOW>
__global__ __launch_bounds__(128) LOGO_OCC_DQ64 void sq_dq64_kernel(const AttnArgs a) {
  constexpr int DS = D / 16, DT = D / 32;
  constexpr int NX = 2 * DS;    // X slots: K row operand (even), V row operand (odd)
  constexpr int NY = 2 * DT;    // Y slots: K^T operands (16-key step hh, column block dt)
  constexpr int IX = 16 / NX;   // VALU items per X slot and row block (16 per half)
  constexpr int PF = 3;         // operand prefetch distance, in slots
  using GT = TileGeom<D, kSwz>;
  bf16* const smem = dyn_smem();
  auto tileK = [&](int b) { return smem + b * GT::ELEMS; };
  auto tileV = [&](int b) { return smem + 2 * GT::ELEMS + b * GT::ELEMS; };

  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, i = l & 31, g = l >> 5;
  QTile<SPARSE> qt;
  if (!qt.init(a, wave, i, WINDOW, 64)) return;
  const int hq = qt.hq, W = a.window;
  int rr[2], pr[2];
  bool vr[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    rr[b] = qt.r0 + 64 * wave + 32 * b + i;
    vr[b] = rr[b] < qt.r_end;
    pr[b] = vr[b] ? qt.rv.posn(rr[b]) : -1;
  }

  bf16x8 qreg[2][DS], doreg[2][DS];
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
        qreg[b][ds] = vr[b] ? *reinterpret_cast<const bf16x8*>(qrow + 16 * ds) : bf16x8{};
        doreg[b][ds] = vr[b] ? *reinterpret_cast<const bf16x8*>(orow + 16 * ds) : bf16x8{};
      }
      lse_q[b] = vr[b] ? a.lse[(int64_t)hq * a.n + rr[b]] : 0.f;
      delta_q[b] = vr[b] ? a.delta[(int64_t)hq * a.n + rr[b]] : 0.f;
    }
  }
  const float c = a.scale_log2;

  f32x16 dqacc[2][DT];  // AGPRs
#pragma unroll
  for (int b = 0; b < 2; ++b)
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) dqacc[b][dt] = f32x16{};
  f32x16 sp[2][2][2];  // [half parity][row block][S, dP]
  bf16x8 dsb[2][2];    // dS of the current half as B operands [row block][16-key step]

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
  int hw_lo = 0, hw_hi = 0;  // 32-key halves this wave's rows can see
  if (qt.wave_active) {
    hw_hi = ((qt.pmax - kv_lo) >> 5) + 1;
    hw_lo = WINDOW ? (max(0, qt.pmin - W - kv_lo) >> 5) : 0;
  }

  // step (t, H): PAR = t & 1 (K / V slot of tile t)
  auto step = [&](auto par_tag, auto h_tag, int t) {
    constexpr int PAR = decltype(par_tag)::value, H = decltype(h_tag)::value;
    if (H == 0) {
      if (t + 1 < nt) load_one(tileK(PAR ^ 1), kbase, kv_lo + 64 * (t + 1));
    } else {
      if (t + 2 < nt) load_one(tileV(PAR), vbase, kv_lo + 64 * (t + 2));
    }
    // X reads the next half: rows 32 of tile t (H = 0) or rows 0 of tile t + 1
    const bf16* kx = tileK(H == 0 ? PAR : PAR ^ 1);
    const bf16* vx = tileV(H == 0 ? PAR : PAR ^ 1);
    constexpr int XR = H == 0 ? 32 : 0;
    const bf16* ky = tileK(PAR);  // K^T of the current half, rows 32 H
    const int hx = 2 * t + H;     // current half
    const int j0h = kv_lo + 32 * hx;

    auto body = [&](auto dox_tag, auto dov_tag, auto mask_tag) {
      constexpr bool DOX = decltype(dox_tag)::value;    // S / dP of the next half
      constexpr bool DOV = decltype(dov_tag)::value;    // dS and dQ of the current half
      constexpr bool MASK = decltype(mask_tag)::value;  // the current half crosses a mask edge
      bf16x8 op[NX + NY];
      auto load_op = [&](auto s_c) {
        constexpr int S = decltype(s_c)::value;
        if constexpr (S < NX) {
          if constexpr (DOX) op[S] = rd.row(S % 2 ? vx : kx, XR, S / 2);
        } else {
          constexpr int Y = S - NX;
          if constexpr (DOV) op[S] = rd.tr(ky, 32 * H + 16 * (Y / DT), Y % DT);
        }
      };
      static_for<PF>([&](auto s_c) { load_op(s_c); });
      int hi[2];
#pragma unroll
      for (int b = 0; b < 2; ++b) hi[b] = pr[b] - j0h - 4 * g;
      static_for<NX + NY>([&](auto s_c) {
        constexpr int S = decltype(s_c)::value;
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (S < NX) {
          // one wave per SIMD issues in order: each MFMA is followed by the
          // VALU items of its row block, which run under it
          constexpr int DSI = S / 2, KIND = S % 2;
          bf16x8 o;
          if constexpr (DOX) {
            o = op[S];
            pin(o);
          }
          static_for<2>([&](auto b_c) {
            constexpr int B = decltype(b_c)::value;
            if constexpr (B == 1) __builtin_amdgcn_sched_barrier(0);
            if constexpr (DOX) {
              const bf16x8 bop = KIND ? doreg[B][DSI] : qreg[B][DSI];
              sp[H ^ 1][B][KIND] = mfma32(o, bop, DSI == 0 ? f32x16{} : sp[H ^ 1][B][KIND]);
            }
            if constexpr (DOV) {
              static_for<IX>([&](auto e_c) {
                constexpr int JJ = S * IX + decltype(e_c)::value;
                float sv = sp[H][B][0][JJ], dpv = sp[H][B][1][JJ];
                pin(sv);
                pin(dpv);
                float pv = fast_exp2(fmaf(sv, c, -lse_q[B]));
                if constexpr (MASK) {
                  constexpr int off = 8 * (JJ / 4) + (JJ % 4);
                  bool vis = off <= hi[B];
                  if (WINDOW) vis = vis && off >= hi[B] - W;
                  if (!vis) pv = 0.f;
                }
                float dsv = pv * (dpv - delta_q[B]);
                pin(dsv);
                sp[H][B][0][JJ] = pv;
                sp[H][B][1][JJ] = dsv;
                if constexpr (JJ % 8 == 7) dsb[B][JJ / 8] = acc_to_bf16(sp[H][B][1], JJ / 8);
              });
            }
          });
        } else {
          constexpr int Y = S - NX;
          if constexpr (DOV) {
            bf16x8 o = op[S];
            pin(o);
            mfma32_agpr(dqacc[0][Y % DT], o, dsb[0][Y / DT]);
            mfma32_agpr(dqacc[1][Y % DT], o, dsb[1][Y / DT]);
          }
        }
        if constexpr (S + PF < NX + NY) load_op(std::integral_constant<int, S + PF>{});
      });
      __builtin_amdgcn_sched_barrier(0);
    };
    using T_ = std::true_type;
    using F_ = std::false_type;
    const bool dox = hx + 1 >= hw_lo && hx + 1 < hw_hi;
    const bool dov = hx >= hw_lo && hx < hw_hi;
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

  load_one(tileK(0), kbase, kv_lo);
  load_one(tileV(0), vbase, kv_lo);
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
#pragma unroll
  for (int b = 0; b < 2; ++b) {
    if (vr[b]) {
      const int64_t tok = qt.rv.token(rr[b]);
      bf16* dqrow = a.dq + (tok * a.hq + hq) * D;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int q4 = 0; q4 < 4; ++q4) {
          bf16x4 v;
#pragma unroll
          for (int e = 0; e < 4; ++e) v[e] = (bf16)(dqacc[b][dt][4 * q4 + e] * a.scale);
          *reinterpret_cast<bf16x4*>(dqrow + 32 * dt + 8 * q4 + 4 * g) = v;
        }
    }
  }
}

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

template <int D, bool SPARSE, bool WINDOW>
__global__ __launch_bounds__(256) LOGO_OCC_DKV void sq_dkv_kernel(const AttnArgs a) {
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

  bf16x8 kreg[DS], vreg[DS];
  {
    const int64_t off = ((int64_t)(bos + key) * a.h + h) * D + 8 * g;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      kreg[ds] = valid_k ? *reinterpret_cast<const bf16x8*>(a.k + off + 16 * ds) : bf16x8{};
      vreg[ds] = valid_k ? *reinterpret_cast<const bf16x8*>(a.v + off + 16 * ds) : bf16x8{};
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
    int rq0, rq_end;
    if (SPARSE) {
      rq0 = lower_bound_i32(rv.ps, q_lo, q_hi, k0);
      rq_end = WINDOW ? lower_bound_i32(rv.ps, rq0, q_hi, k_last + W + 1) : q_hi;
    } else {
      rq0 = min(q_lo + k0, q_hi);
      rq_end = WINDOW ? min(q_hi, q_lo + k_last + W + 1) : q_hi;
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
      const int p_first = pob[0];
      const int p_last = pob[last - rt];
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
        constexpr int PF = 6;       // operand prefetch distance, in slots
        constexpr int IPP = 16 / (2 * DS);  // P items per slot (over two blocks)
        constexpr int IPD = 16 / DS;        // dS items per slot (over one block)
        static_assert(IPP * 2 * DS == 16 && IPD * DS == 16, "a half has 16 row items per lane");
        f32x16 sacc[2], pacc[2];
        bf16x8 pbf[2][2], dbf[2][2];  // [half][hh]
        bf16x8 opA[NSUB * 2 * NS];    // S/dP operands: Q rows / dO rows
        bf16x8 opC[NSUB * 2 * NS];    // dV/dK operands: dO^T / Q^T
        f32x4 l4[NSUB][2][4], d4[NSUB][2][4];
        int4 p4[NSUB][2][4];
        // A operand a of sub-tile u: half a / NS; S (first DS) or dP (next DS), k-step a % DS
        auto load_a = [&](auto u_c, auto a_c) {
          constexpr int U = decltype(u_c)::value, A = decltype(a_c)::value;
          constexpr int QQ = A / NS, KK = A % NS;
          opA[U * 2 * NS + A] = rd.row(KK >= DS ? ob : qb, 64 * U + 32 * QQ, KK % DS);
        };
        // C operand c of sub-tile u: half c / NS; dV (first DS) or dK (next DS); hh, dt
        auto load_c = [&](auto u_c, auto c_c) {
          constexpr int U = decltype(u_c)::value, C = decltype(c_c)::value;
          constexpr int QQ = C / NS, KK = C % NS, HH = (KK % DS) / DT, DTI = KK % DT;
          opC[U * 2 * NS + C] = rd.tr(KK >= DS ? qb : ob, 64 * U + 16 * (2 * QQ + HH), DTI);
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
          l4[u][qq][m] = lds_load(reinterpret_cast<const f32x4*>(lb + qr));
          if constexpr (MASK) p4[u][qq][m] = lds_load(reinterpret_cast<const int4*>(pob + qr));
        };
        auto load_dstats = [&](int u, int qq, int m) {
          const int qr = 64 * u + 32 * qq + 8 * m + 4 * g;
          d4[u][qq][m] = lds_load(reinterpret_cast<const f32x4*>(dlb + qr));
        };
        auto mfma_a = [&](auto u_c, auto a_c) {
          constexpr int U = decltype(u_c)::value, A = decltype(a_c)::value;
          constexpr int QQ = A / NS, KK = A % NS;
          bf16x8 op = opA[U * 2 * NS + A];
          pin(op);
          if constexpr (KK < DS) {
            sacc[QQ] = mfma32(op, kreg[KK], KK == 0 ? f32x16{} : sacc[QQ]);
          } else {
            pacc[QQ] = mfma32(op, vreg[KK - DS], KK == DS ? f32x16{} : pacc[QQ]);
          }
        };
        auto mfma_c = [&](auto u_c, auto c_c) {
          constexpr int U = decltype(u_c)::value, C = decltype(c_c)::value;
          constexpr int QQ = C / NS, KK = C % NS, HH = (KK % DS) / DT, DTI = KK % DT;
          bf16x8 op = opC[U * 2 * NS + C];
          pin(op);
          if constexpr (KK < DS) mfma32_agpr(dvacc[DTI], op, pbf[QQ][HH]);
          else mfma32_agpr(dkacc[DTI], op, dbf[QQ][HH]);
        };
        // row item jj of half qq: items 4m..4m+3 are query rows 32qq + 8m + 4g + e.
        // P items leave P in sacc (fp32) and pack pairs into pbf; dS items leave
        // dS in pacc and pack pairs into dbf.
        auto p_item = [&](auto u_c, int qq, auto jj_c) {
          constexpr int U = decltype(u_c)::value, JJ = decltype(jj_c)::value;
          constexpr int M = JJ / 4, E = JJ % 4;
          float sv = sacc[qq][JJ];
          pin(sv);
          float pv = fast_exp2(fmaf(sv, c, -l4[U][qq][M][E]));
          if constexpr (MASK) {
            const int pq = p4[U][qq][M][E];
            bool vis = key <= pq;
            if (WINDOW) vis = vis && key >= pq - W;
            if (!vis) pv = 0.f;
          }
          pin(pv);
          sacc[qq][JJ] = pv;
          if constexpr (JJ % 2 == 1) {
            pbf[qq][JJ / 8][JJ % 8 - 1] = (bf16)sacc[qq][JJ - 1];
            pbf[qq][JJ / 8][JJ % 8] = (bf16)pv;
          }
        };
        auto ds_item = [&](auto u_c, int qq, auto jj_c) {
          constexpr int U = decltype(u_c)::value, JJ = decltype(jj_c)::value;
          constexpr int M = JJ / 4, E = JJ % 4;
          float pv = sacc[qq][JJ], dpv = pacc[qq][JJ];
          pin(pv);
          pin(dpv);
          float dsv = pv * (dpv - d4[U][qq][M][E]);
          pin(dsv);
          pacc[qq][JJ] = dsv;
          if constexpr (JJ % 2 == 1) {
            dbf[qq][JJ / 8][JJ % 8 - 1] = (bf16)pacc[qq][JJ - 1];
            dbf[qq][JJ / 8][JJ % 8] = (bf16)dsv;
          }
        };
        // stats of (sub-tile u, half qq, group m) are read DS/2 slots before
        // the first item of group m needs them; the P items of half qq start at
        // block 1 + 3qq, its dS items at block 3 + 3qq
        auto pstats_slot = [](int u, int qq, int m) { return SPT * u + DS * (1 + 3 * qq) + 4 * m / IPP - DS / 2; };
        auto dstats_slot = [](int u, int qq, int m) { return SPT * u + DS * (3 + 3 * qq) + 4 * m / IPD - DS / 2; };

        static_for<PF>([&](auto t_c) { load_for_slot(t_c); });
        static_for<NSUB * SPT>([&](auto s_c) {
          constexpr int S = decltype(s_c)::value, U = S / SPT, L = S % SPT;
          constexpr int BLK = L / DS, K = L % DS;
          using UC = std::integral_constant<int, U>;
          __builtin_amdgcn_sched_barrier(0);
          if constexpr (L < 2 * NS) mfma_a(UC{}, std::integral_constant<int, L>{});
          else mfma_c(UC{}, std::integral_constant<int, L - 2 * NS>{});
          if constexpr (S + PF < NSUB * SPT) load_for_slot(std::integral_constant<int, S + PF>{});
#pragma unroll
          for (int u = 0; u < NSUB; ++u)
#pragma unroll
            for (int qq = 0; qq < 2; ++qq)
#pragma unroll
              for (int m = 0; m < 4; ++m) {
                if (pstats_slot(u, qq, m) == S) load_pstats(u, qq, m);
                if (dstats_slot(u, qq, m) == S) load_dstats(u, qq, m);
              }
          if constexpr (BLK == 1 || BLK == 2 || BLK == 4 || BLK == 5) {
            constexpr int QQ = BLK >= 4, J0 = ((BLK - 1) % 3) * DS + K;
            static_for<IPP>([&](auto i_c) {
              p_item(UC{}, QQ, std::integral_constant<int, J0 * IPP + decltype(i_c)::value>{});
            });
          }
          if constexpr (BLK == 3 || BLK == 6) {
            constexpr int QQ = BLK == 6;
            static_for<IPD>([&](auto i_c) {
              ds_item(UC{}, QQ, std::integral_constant<int, K * IPD + decltype(i_c)::value>{});
            });
          }
        });
        __builtin_amdgcn_sched_barrier(0);
      };
      const bool skip = !wave_active || p_last < kw0 || (WINDOW && p_first > kw_last + W);
      if (!skip) {
        const bool need_mask = WINDOW || (p_first < kw_last) || (rt + RS > rq_end);
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
  if (valid_k) {
    const int64_t off = ((int64_t)(bos + key) * a.h + h) * D;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        bf16x4 kv, vv;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          kv[e] = (bf16)(dkacc[dt][4 * q4 + e] * a.scale);
          vv[e] = (bf16)dvacc[dt][4 * q4 + e];
        }
        *reinterpret_cast<bf16x4*>(a.dk + off + 32 * dt + 8 * q4 + 4 * g) = kv;
        *reinterpret_cast<bf16x4*>(a.dv + off + 32 * dt + 8 * q4 + 4 * g) = vv;
      }
  }
}

// ---------------------------------------------------------------------------
// Host launchers
// ---------------------------------------------------------------------------
template <int D>
constexpr size_t fwd_smem() { return (size_t)4 * TileGeom<D, kSwz>::ELEMS * sizeof(bf16); }
template <int D>
constexpr size_t dq_smem() { return (size_t)4 * TileGeom<D, kSwz>::ELEMS * sizeof(bf16); }
template <int D>
constexpr size_t dkv_smem() { return (size_t)kDkvStages * dkv_stage_bytes<D>(); }

template <typename K>
static hipError_t allow_smem(K kernel, size_t bytes) {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

static int check_common(int64_t n, int nseq, int hq, int h, int d, int v_dim, int lanes, int dtype) {
  LOGO_REQUIRE(n > 0 && n < ((int64_t)1 << 31), "n_tokens out of range: %lld", (long long)n);
  LOGO_REQUIRE(nseq >= 1, "nseq must be >= 1");
  LOGO_REQUIRE(h >= 1 && hq >= h && hq % h == 0, "HQ (%d) must be a multiple of H (%d)", hq, h);
  LOGO_REQUIRE(d == 64 || d == 128, "head dim %d unsupported (64 or 128)", d);
  // every kernel strides q, k, v, o and the gradients by the one head dim d
  LOGO_REQUIRE(v_dim == d, "value head dim %d must equal the key head dim %d", v_dim, d);
  LOGO_REQUIRE(lanes == 1 || lanes == hq, "lanes must be 1 or HQ");
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  return LOGO_OK;
}

// Single long sequences take 8-wave workgroups of two query tiles, which
// share each K / V tile copy between 256 rows (half the copy traffic and
// issue per row); packed or short inputs keep 4-wave single-tile workgroups,
// which give more workgroups where rows are few.
constexpr int64_t kFwdPairMinTokens = 16384;

template <int D, bool SPARSE, bool WINDOW>
static int launch_fwd(const AttnArgs& a, hipStream_t st) {
  const bool paired = a.nseq == 1 && a.n >= kFwdPairMinTokens;
  const int64_t rows = paired ? 2 * kBQ : kBQ;
  const int64_t ntmax = (a.n + rows - 1) / rows + a.nseq;
  const int64_t nblk = ntmax * a.hq;
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "grid too large");
  if (paired) {
    auto kern = sq_fwd_pipe_kernel<D, SPARSE, WINDOW, 8>;
    LOGO_HIP_CHECK(allow_smem(kern, fwd_smem<D>()));
    hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(512), fwd_smem<D>(), st, a);
  } else {
    auto kern = sq_fwd_pipe_kernel<D, SPARSE, WINDOW, 4>;
    LOGO_HIP_CHECK(allow_smem(kern, fwd_smem<D>()));
    hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(256), fwd_smem<D>(), st, a);
  }
  LOGO_LAUNCH_CHECK("sq_fwd_pipe_kernel");
  return LOGO_OK;
}

// Backward phases: 0 = delta, 1 = dq, 2 = dk/dv, -1 = all three in order.
template <int D, bool SPARSE, bool WINDOW>
static int launch_bwd_phase(const AttnArgs& a, hipStream_t st, int phase) {
  if (phase < 0 || phase == 0) {
    constexpr int RPB = 256 / (D / 8);
    dim3 grid((unsigned)((a.n + RPB - 1) / RPB), a.hq);
    hipLaunchKernelGGL((sq_delta_kernel<D, SPARSE>), grid, dim3(256), 0, st, a);
    LOGO_LAUNCH_CHECK("sq_delta_kernel");
  }
  if (phase < 0 || phase == 1) {
    const int64_t ntmax = (a.n + kBQ - 1) / kBQ + a.nseq;
    auto kern = sq_dq64_kernel<D, SPARSE, WINDOW>;
    LOGO_HIP_CHECK(allow_smem(kern, dq_smem<D>()));
    hipLaunchKernelGGL(kern, dim3((unsigned)(ntmax * a.hq)), dim3(128), dq_smem<D>(), st, a);
    LOGO_LAUNCH_CHECK("sq_dq64_kernel");
  }
  if (phase < 0 || phase == 2) {
    const int64_t ntmax = (a.n + kBKV - 1) / kBKV + a.nseq;
    auto kern = sq_dkv_kernel<D, SPARSE, WINDOW>;
    LOGO_HIP_CHECK(allow_smem(kern, dkv_smem<D>()));
    hipLaunchKernelGGL(kern, dim3((unsigned)(ntmax * a.h)), dim3(256), dkv_smem<D>(), st, a);
    LOGO_LAUNCH_CHECK("sq_dkv_kernel");
  }
  return LOGO_OK;
}

template <int D, bool SPARSE, bool WINDOW>
static int launch_bwd(const AttnArgs& a, hipStream_t st) { return launch_bwd_phase<D, SPARSE, WINDOW>(a, st, -1); }
template <int D, bool SPARSE, bool WINDOW>
static int launch_bwd_delta(const AttnArgs& a, hipStream_t st) { return launch_bwd_phase<D, SPARSE, WINDOW>(a, st, 0); }
template <int D, bool SPARSE, bool WINDOW>
static int launch_bwd_dq(const AttnArgs& a, hipStream_t st) { return launch_bwd_phase<D, SPARSE, WINDOW>(a, st, 1); }
template <int D, bool SPARSE, bool WINDOW>
static int launch_bwd_dkv(const AttnArgs& a, hipStream_t st) { return launch_bwd_phase<D, SPARSE, WINDOW>(a, st, 2); }

static AttnArgs make_args(const void* q, const void* k, const void* v, const int64_t* q_idx,
                          const int32_t* pos, const int32_t* meta, const int32_t* cu, int64_t n,
                          int nseq, int hq, int h, int lanes, float scale, int window) {
  AttnArgs a{};
  a.q = static_cast<const bf16*>(q);
  a.k = static_cast<const bf16*>(k);
  a.v = static_cast<const bf16*>(v);
  a.q_idx = q_idx;
  a.pos = pos;
  a.meta = meta;
  a.cu = cu;
  a.n = n;
  a.nseq = nseq;
  a.hq = hq;
  a.h = h;
  a.g = hq / h;
  a.lanes = lanes;
  a.meta_stride = LOGO_META_STRIDE(nseq);
  a.scale = scale;
  a.scale_log2 = scale * 1.4426950408889634f;
  a.window = window;
  return a;
}

#define LOGO_DISPATCH(FN, a, st, d, sparse, window)                                   \
  ((d) == 128 ? ((sparse) ? ((window) ? FN<128, true, true>(a, st) : FN<128, true, false>(a, st))   \
                          : ((window) ? FN<128, false, true>(a, st) : FN<128, false, false>(a, st))) \
              : ((sparse) ? ((window) ? FN<64, true, true>(a, st) : FN<64, true, false>(a, st))     \
                          : ((window) ? FN<64, false, true>(a, st) : FN<64, false, false>(a, st))))

}  // namespace logo

using namespace logo;

extern "C" int logo_sq_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                           const int64_t* q_idx, const int32_t* pos, const int32_t* meta,
                           const int32_t* cu, int64_t n_tokens, int nseq, int hq, int h, int d,
                           int v_dim, int lanes, float scale, int window, int dtype, void* stream) {
  int rc = check_common(n_tokens, nseq, hq, h, d, v_dim, lanes, dtype);
  if (rc != LOGO_OK) return rc;
  LOGO_REQUIRE(q && k && v && o && lse && meta && cu, "null pointer argument");
  LOGO_REQUIRE((q_idx == nullptr) == (pos == nullptr), "q_idx and pos must both be set or both be null");
  AttnArgs a = make_args(q, k, v, q_idx, pos, meta, cu, n_tokens, nseq, hq, h, lanes, scale, window);
  a.o = static_cast<bf16*>(o);
  a.lse = lse;
  const bool sparse = q_idx != nullptr;
  const bool win = window >= 0;
  return LOGO_DISPATCH(launch_fwd, a, as_stream(stream), d, sparse, win);
}

#define LOGO_BWD_PARAMS                                                                        \
  const void *q, const void *k, const void *v, const void *o, const void *dout, const float *lse, \
      float *delta, void *q_sel, void *do_sel, void *dq, void *dk, void *dv, const int64_t *q_idx, \
      const int32_t *pos, const int32_t *meta, const int32_t *cu, int64_t n_tokens, int nseq,      \
      int hq, int h, int d, int v_dim, int lanes, float scale, int window, int dtype, void *stream

#define LOGO_BWD_ARGS                                                                             \
  q, k, v, o, dout, lse, delta, q_sel, do_sel, dq, dk, dv, q_idx, pos, meta, cu, n_tokens, nseq, hq, \
      h, d, v_dim, lanes, scale, window, dtype, stream

static int bwd_entry(LOGO_BWD_PARAMS, int phase) {
  int rc = check_common(n_tokens, nseq, hq, h, d, v_dim, lanes, dtype);
  if (rc != LOGO_OK) return rc;
  LOGO_REQUIRE(q && k && v && o && dout && lse && delta && meta && cu, "null pointer argument");
  LOGO_REQUIRE(phase == 0 || (dq && dk && dv), "null gradient pointer");
  LOGO_REQUIRE((q_idx == nullptr) == (pos == nullptr), "q_idx and pos must both be set or both be null");
  LOGO_REQUIRE(q_idx == nullptr || (q_sel && do_sel), "sparse backward needs q_sel and do_sel workspaces");
  AttnArgs a = make_args(q, k, v, q_idx, pos, meta, cu, n_tokens, nseq, hq, h, lanes, scale, window);
  a.o = const_cast<bf16*>(static_cast<const bf16*>(o));
  a.dout = static_cast<const bf16*>(dout);
  a.lse = const_cast<float*>(lse);
  a.delta = delta;
  a.q_sel = static_cast<bf16*>(q_sel);
  a.do_sel = static_cast<bf16*>(do_sel);
  a.dq = static_cast<bf16*>(dq);
  a.dk = static_cast<bf16*>(dk);
  a.dv = static_cast<bf16*>(dv);
  const bool sparse = q_idx != nullptr;
  const bool win = window >= 0;
  hipStream_t st = as_stream(stream);
  switch (phase) {
    case 0: return LOGO_DISPATCH(launch_bwd_delta, a, st, d, sparse, win);
    case 1: return LOGO_DISPATCH(launch_bwd_dq, a, st, d, sparse, win);
    case 2: return LOGO_DISPATCH(launch_bwd_dkv, a, st, d, sparse, win);
    default: return LOGO_DISPATCH(launch_bwd, a, st, d, sparse, win);
  }
}

extern "C" int logo_sq_bwd(LOGO_BWD_PARAMS) { return bwd_entry(LOGO_BWD_ARGS, -1); }
extern "C" int logo_sq_bwd_delta(LOGO_BWD_PARAMS) { return bwd_entry(LOGO_BWD_ARGS, 0); }
extern "C" int logo_sq_bwd_dq(LOGO_BWD_PARAMS) { return bwd_entry(LOGO_BWD_ARGS, 1); }
extern "C" int logo_sq_bwd_dkv(LOGO_BWD_PARAMS) { return bwd_entry(LOGO_BWD_ARGS, 2); }
