// Sliding-window causal attention forward for gfx950 (the local branch:
// flash-attn window_size=(w, w), causal=True over every row, as called by
// logo/layers/utils.py:144-147, :166-178): row p attends keys [p - w, p] of
// its own segment.
//
// The generic forward kernel streams K / V through a software pipeline built
// for long key ranges; a window of at most 128 keys gives it 4-5 pipeline
// steps per 128-row tile, each waiting on its own copy, so it idles on load
// latency.  This kernel loads the whole key window of a 128-row query block
// (at most 256 keys: blocks b - 1 and b) into LDS in one burst, first K, and
// each wave scores only the 32-key chunks its 32 rows can see (five for
// w = 128: 160 keys for 129 visible).  The softmax is exact in two passes
// over registers (row max, then P = exp2(S c - m c)), with no rescaling.
// V's window is fetched into registers together with q and K, and written
// over K's LDS tiles once the scores are done (one 64 KB window at D = 128,
// so two workgroups share a CU; every load of a workgroup is in flight at
// once), then O = P V.  lse is written in the same log2 domain as the
// generic forward, so the backward kernels are unchanged.
//
// Layout as the generic kernels: q / k / v / o [N, heads, D] bf16, the tile
// -> (segment, block) map from the dense metadata (kBQ = 128 rows a tile).
#include "sq_attn.hpp"

namespace logo {

constexpr int kSwaMaxWindow = 128;  // keys [p - w, p] within blocks b - 1 and b
constexpr int kSwaChunks = 5;       // 32-key chunks a wave can see: (32 + 128) / 32

template <int D>
__global__ __launch_bounds__(256) void swa_fwd_kernel(const AttnArgs a) {
  constexpr int DS = D / 16, DT = D / 32;
  using GT = TileGeom<D, kSwz>;
  bf16* const smem = dyn_smem();
  auto tile = [&](int t) { return smem + t * GT::ELEMS; };  // K's window, then V's

  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, i = l & 31, g = l >> 5;
  QTile<false> qt;
  if (!qt.init(a, wave, i, true, 32)) return;
  const int hq = qt.hq, p = qt.p, W = a.window;
  const int kv_lo = qt.kv_lo;                       // 64-aligned, >= 0
  const int seqlen = qt.seqlen;

  // Loads in a fixed order, all unconditional: q rows, the four K tiles
  // (global -> LDS), the four V tiles (global -> registers).  Tiles past the
  // window (nt < 4) and keys past the segment are clamped to the segment's
  // last key (never read, or masked).
  bf16x8 qreg[DS];
  {
    const bf16* qrow = a.q + (qt.t * a.hq + hq) * D + 8 * g;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) qreg[ds] = qt.valid ? *reinterpret_cast<const bf16x8*>(qrow + 16 * ds) : bf16x8{};
  }
  const int64_t rstride = (int64_t)a.h * D;
  const bf16* kbase = a.k + ((int64_t)qt.bos * a.h + qt.h) * D;
  const bf16* vbase = a.v + ((int64_t)qt.bos * a.h + qt.h) * D;
  TileBufDma<D, 4> dma;
  dma.init((int)rstride);
  auto load_one = [&](bf16* tile, const bf16* src, int t) {
    const int j0 = min(kv_lo + 64 * t, seqlen - 1);
    dma.issue_clamped(tile, src + j0 * rstride, seqlen - 1 - j0);
  };
#pragma unroll
  for (int t = 0; t < 4; ++t) load_one(tile(t), kbase, t);
  Tile64<D> vreg[4];
#pragma unroll
  for (int t = 0; t < 4; ++t)
    vreg[t].load(tid, [&](int r) { return vbase + (int64_t)min(kv_lo + 64 * t + r, seqlen - 1) * rstride; });

  // the 32-key chunks (relative to kv_lo) this wave's rows can see
  int c_lo = 0, nch = 0;
  if (qt.wave_active) {
    c_lo = max(0, qt.pmin - W - kv_lo) >> 5;
    nch = min(kSwaChunks, ((qt.pmax - kv_lo) >> 5) + 1 - c_lo);
  }

  // q and K landed (the V loads, this thread's last 4 * RPT, may still be in
  // flight).  A bare barrier publishes the K tiles: the one in
  // __syncthreads() would first wait for every load, V's included.
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" ::"n"(4 * Tile64<D>::RPT) : "memory");

  TileReader<D, kSwz> rd;
  rd.init();
  const float c = a.scale_log2;
  f32x16 sc[kSwaChunks];
  float mx = -INFINITY;
#pragma unroll
  for (int k = 0; k < kSwaChunks; ++k) {
    sc[k] = f32x16{};
    if (k < nch) {
      const int ch = c_lo + k;
      const bf16* kt = tile(ch >> 1);
#pragma unroll
      for (int ds = 0; ds < DS; ++ds) sc[k] = mfma32(rd.row(kt, 32 * (ch & 1), ds), qreg[ds], sc[k]);
      // key kv_lo + 32 ch + rowmap(g, j) is visible iff it lies in [p - W, p]
      const int hi = p - (kv_lo + 32 * ch) - 4 * g;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int off = 8 * (j / 4) + (j % 4);
        const bool vis = off <= hi && off >= hi - W;
        sc[k][j] = vis ? sc[k][j] : -INFINITY;
        mx = fmaxf(mx, sc[k][j]);
      }
    }
  }
  const float mrow = pair_max(mx);
  const float base = mrow == -INFINITY ? 0.f : mrow * c;
  float lsum = 0.f;
  bf16x8 pb[2 * kSwaChunks];
#pragma unroll
  for (int k = 0; k < kSwaChunks; ++k) {
    if (k < nch) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float pv = fast_exp2(fmaf(sc[k][j], c, -base));
        sc[k][j] = pv;
        lsum += pv;
      }
      pb[2 * k] = acc_to<bf16>(sc[k], 0);
      pb[2 * k + 1] = acc_to<bf16>(sc[k], 1);
    }
  }
  const float l_tot = pair_sum(lsum);

  __syncthreads();  // every wave is done with K's tiles
#pragma unroll
  for (int t = 0; t < 4; ++t) vreg[t].template store<kSwz>(tile(t), tid);
  __syncthreads();
  f32x16 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x16{};
#pragma unroll
  for (int k = 0; k < kSwaChunks; ++k) {
    if (k < nch) {
      const int ch = c_lo + k;
      const bf16* vt = tile(ch >> 1);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) oacc[dt] = mfma32(rd.tr(vt, 32 * (ch & 1) + 16 * h, dt), pb[2 * k + h], oacc[dt]);
    }
  }

  // O leaves through LDS as whole rows: each wave writes its 32 rows (8-byte
  // pieces, swizzled chunks) over the V tiles, then 16 lanes store one row's
  // D * 2 bytes together.  Stored from the accumulators directly, every
  // 8-byte piece would touch its own row (32 rows per store instruction).
  const float inv = qt.valid ? 1.f / l_tot : 0.f;
  __syncthreads();  // every wave is done with V's tiles
  bf16* const ot = tile(0);  // 128 rows x D (two 64-row swizzled tiles)
  {
    const int row = 32 * wave + i;
    bf16* const orow = ot + (row >> 6) * GT::ELEMS;
    const int rr = row & 63;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt)
#pragma unroll
      for (int q4 = 0; q4 < 4; ++q4) {
        bf16x4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] = (bf16)(oacc[dt][4 * q4 + e] * inv);
        // d = 32 dt + 8 q4 + 4 g: half g of chunk 4 dt + q4
        *reinterpret_cast<bf16x4*>(orow + GT::off(rr, 4 * dt + q4) + 4 * g) = v;
      }
  }
  if (qt.valid && g == 0) a.lse[(int64_t)hq * a.n + qt.r] = base + log2f(l_tot);
  __syncthreads();
  {
    constexpr int CHR = D / 8;               // 16-byte chunks per row
    constexpr int RPP = 256 / CHR;           // rows per pass
    const int ch = tid % CHR;
    const int nrow = qt.r_end - qt.r0;
#pragma unroll
    for (int r = tid / CHR; r < 128; r += RPP) {
      if (r < nrow) {
        const u32x4 v = *reinterpret_cast<const u32x4*>(ot + (r >> 6) * GT::ELEMS + GT::off(r & 63, ch));
        // dense rows: row r0 + r is the token
        *reinterpret_cast<u32x4*>(a.o + ((int64_t)(qt.r0 + r) * a.hq + hq) * D + 8 * ch) = v;
      }
    }
  }
}

template <int D>
constexpr size_t swa_fwd_smem() { return (size_t)4 * TileGeom<D, kSwz>::ELEMS * sizeof(bf16); }

template <int D>
static int launch_swa_fwd(const AttnArgs& a, hipStream_t st) {
  const int64_t ntmax = (a.n + kBQ - 1) / kBQ + a.nseq;
  const int64_t nblk = ntmax * a.hq;
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "grid too large");
  auto kern = swa_fwd_kernel<D>;
  LOGO_HIP_CHECK(allow_smem(kern, swa_fwd_smem<D>()));
  hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(256), swa_fwd_smem<D>(), st, a);
  LOGO_LAUNCH_CHECK("swa_fwd_kernel");
  return LOGO_OK;
}

bool swa_fwd_applies(const AttnArgs& a, bool sparse, bool half) {
  return !sparse && !half && a.window >= 0 && a.window <= kSwaMaxWindow;
}

int swa_launch_fwd(const AttnArgs& a, hipStream_t st, int d) {
  return d == 128 ? launch_swa_fwd<128>(a, st) : launch_swa_fwd<64>(a, st);
}

}  // namespace logo
