// Fused LoGo attention epilogue for gfx950: gate threshold, the two branch
// context RMSNorms and the gated fusion, forward and backward.
//
// Forward, per element of a (token, head) row, with the eager bf16 rounding
// points of the reference kept (logo/modules/layernorm.py:17-22,
// logo/layers/logo.py:180-181, :225-226, :256-258):
//   Ln  = bf16(w_l * bf16(L * rsqrt(mean(L^2) + eps)))      (same for G)
//   g'  = gate < thres ? 0 : gate
//   out = bf16(bf16(bf16(1 - g') * Ln) + bf16(g' * Gn))
// One pass reads L, G and the gate and writes out (the reference makes about a
// dozen full passes).  Backward recomputes the norms in fp32 and returns dL,
// dG, dgate (zero where masked) and the weight gradients, reduced
// deterministically (per-workgroup partials, then a fixed-order sum).
//
// Rows are [N * H, D]; D/8 lanes own one row (8 elements each), so a
// 256-thread workgroup covers 256 / (D/8) rows and row reductions are lane
// shuffles inside the group.
#include <math.h>

#include "capi.hpp"
#include "common.hpp"

namespace logo {

struct EpiArgs {
  const bf16* L;
  const bf16* G;
  const bf16* gate;
  const void* thres;
  bool thres_bf16;
  const bf16* w_l;
  const bf16* w_g;
  bf16* out;
  const bf16* dout;
  bf16* dL;
  bf16* dG;
  bf16* dgate;
  bf16* dw_l;
  bf16* dw_g;
  float* dgate_part;  // [rows]
  float* dw_part;     // [grid, 2, D]
  int64_t rows;
  int heads;
  float eps;
};

constexpr int kEpiMaxGrid = 1024;

template <int D>
__global__ __launch_bounds__(256) void epi_fwd_kernel(const EpiArgs a) {
  constexpr int LPR = D / 8, RPB = 256 / LPR;
  const int64_t r0 = (int64_t)blockIdx.x * RPB + threadIdx.x / LPR;
  const int c = threadIdx.x % LPR;
  const bool ok = r0 < a.rows;
  // rows past the end compute on row 0 (every lane of a group joins the
  // shuffles) and store nothing
  const int64_t r = ok ? r0 : 0;
  const bf16x8 lv = *reinterpret_cast<const bf16x8*>(a.L + r * D + 8 * c);
  const bf16x8 gv = *reinterpret_cast<const bf16x8*>(a.G + r * D + 8 * c);
  const bf16x8 o = epi_fwd_chunk<D>(lv, gv, (float)a.gate[r / a.heads], load_thres(a.thres, a.thres_bf16),
                                    a.w_l, a.w_g, a.eps, c);
  if (ok) *reinterpret_cast<bf16x8*>(a.out + r * D + 8 * c) = o;
}

template <int D>
__global__ __launch_bounds__(256) void epi_bwd_kernel(const EpiArgs a) {
  constexpr int LPR = D / 8, RPB = 256 / LPR;
  __shared__ float red[2][RPB][D];
  const int c = threadIdx.x % LPR;
  const int rg_ = threadIdx.x / LPR;
  const bf16x8 wlv = *reinterpret_cast<const bf16x8*>(a.w_l + 8 * c);
  const bf16x8 wgv = *reinterpret_cast<const bf16x8*>(a.w_g + 8 * c);
  float wl[8], wg[8], dwl[8], dwg[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    wl[e] = (float)wlv[e];
    wg[e] = (float)wgv[e];
    dwl[e] = 0.f;
    dwg[e] = 0.f;
  }
  const float thres = load_thres(a.thres, a.thres_bf16);
  const int64_t nrb = (a.rows + RPB - 1) / RPB;
  for (int64_t rb = blockIdx.x; rb < nrb; rb += gridDim.x) {
    const int64_t r = rb * RPB + rg_;
    const bool ok = r < a.rows;
    bf16x8 lv{}, gv{}, dv{};
    if (ok) {
      lv = ld_nt(reinterpret_cast<const bf16x8*>(a.L + r * D + 8 * c));
      gv = ld_nt(reinterpret_cast<const bf16x8*>(a.G + r * D + 8 * c));
      dv = ld_nt(reinterpret_cast<const bf16x8*>(a.dout + r * D + 8 * c));
    }
    float xl[8], xg[8], dy[8];
    float ssl = 0.f, ssg = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      xl[e] = (float)lv[e];
      xg[e] = (float)gv[e];
      dy[e] = (float)dv[e];
      ssl = fmaf(xl[e], xl[e], ssl);
      ssg = fmaf(xg[e], xg[e], ssg);
    }
    ssl = group_sum<LPR>(ssl);
    ssg = group_sum<LPR>(ssg);
    const float rl = rsqrtf(ssl / (float)D + a.eps);
    const float rgn = rsqrtf(ssg / (float)D + a.eps);
    const float g = ok ? (float)a.gate[r / a.heads] : 0.f;
    const float gp = g < thres ? 0.f : g;
    float part = 0.f, dotl = 0.f, dotg = 0.f;
    float nl[8], ng[8], dnl[8], dng[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      nl[e] = xl[e] * rl;
      ng[e] = xg[e] * rgn;
      part = fmaf(dy[e], wg[e] * ng[e] - wl[e] * nl[e], part);
      const float dln = dy[e] * (1.f - gp);
      const float dgn = dy[e] * gp;
      dwl[e] = fmaf(dln, nl[e], dwl[e]);
      dwg[e] = fmaf(dgn, ng[e], dwg[e]);
      dnl[e] = dln * wl[e];
      dng[e] = dgn * wg[e];
      dotl = fmaf(dnl[e], nl[e], dotl);
      dotg = fmaf(dng[e], ng[e], dotg);
    }
    part = group_sum<LPR>(part);
    dotl = group_sum<LPR>(dotl) / (float)D;
    dotg = group_sum<LPR>(dotg) / (float)D;
    if (ok) {
      bf16x8 ol, og;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        ol[e] = (bf16)(rl * (dnl[e] - nl[e] * dotl));
        og[e] = (bf16)(rgn * (dng[e] - ng[e] * dotg));
      }
      st_nt(reinterpret_cast<bf16x8*>(a.dL + r * D + 8 * c), ol);
      st_nt(reinterpret_cast<bf16x8*>(a.dG + r * D + 8 * c), og);
      if (c == 0) a.dgate_part[r] = part;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    red[0][rg_][8 * c + e] = dwl[e];
    red[1][rg_][8 * c + e] = dwg[e];
  }
  __syncthreads();
  for (int k = threadIdx.x; k < 2 * D; k += 256) {
    const int br = k / D, d = k % D;
    float s = 0.f;
    for (int j = 0; j < RPB; ++j) s += red[br][j][d];
    a.dw_part[((int64_t)blockIdx.x * 2 + br) * D + d] = s;
  }
}

// dgate per token (sum of its heads' partials, zero where masked) and the
// weight gradients.  Workgroups past the token blocks each reduce 32 of the
// 2 * D (branch, column) weight sums: thread (column, group pg) adds the
// partials b = pg, pg + 8, ... with four independent accumulators, and the 8
// groups are combined in a fixed order, so the sums are deterministic and no
// thread walks all the partials in one dependent chain.
constexpr int kEpiDwCols = 32;

template <int D>
__global__ __launch_bounds__(256) void epi_bwd_finalize_kernel(const EpiArgs a, int64_t n_tokens, int nparts,
                                                               int tok_blocks) {
  if ((int)blockIdx.x >= tok_blocks) {
    __shared__ float red[8][kEpiDwCols];
    const int col = threadIdx.x % kEpiDwCols, pg = threadIdx.x / kEpiDwCols;
    const int k = ((int)blockIdx.x - tok_blocks) * kEpiDwCols + col;  // br * D + d
    const float* src = a.dw_part + k;
    float acc0 = 0.f, acc1 = 0.f, acc2 = 0.f, acc3 = 0.f;
    int b = pg;
    for (; b + 24 < nparts; b += 32) {
      acc0 += src[(int64_t)b * 2 * D];
      acc1 += src[(int64_t)(b + 8) * 2 * D];
      acc2 += src[(int64_t)(b + 16) * 2 * D];
      acc3 += src[(int64_t)(b + 24) * 2 * D];
    }
    for (; b < nparts; b += 8) acc0 += src[(int64_t)b * 2 * D];
    red[pg][col] = (acc0 + acc1) + (acc2 + acc3);
    __syncthreads();
    if (pg == 0) {
      float s = red[0][col];
#pragma unroll
      for (int j = 1; j < 8; ++j) s += red[j][col];
      (k < D ? a.dw_l : a.dw_g)[k % D] = (bf16)s;
    }
    return;
  }
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= n_tokens) return;
  const float g = (float)a.gate[t];
  float s = 0.f;
  if (!(g < load_thres(a.thres, a.thres_bf16))) {
    for (int h = 0; h < a.heads; ++h) s += a.dgate_part[t * a.heads + h];
  }
  a.dgate[t] = (bf16)s;
}

static int epi_check(int64_t n, int heads, int d, int dtype, int thres_dtype) {
  LOGO_REQUIRE(thres_dtype == LOGO_DTYPE_BF16 || thres_dtype == LOGO_DTYPE_F32, "thres_dtype must be bf16 or f32");
  LOGO_REQUIRE(n >= 0 && heads >= 1, "bad token / head counts");
  LOGO_REQUIRE(d == 64 || d == 128, "head dim %d unsupported (64 or 128)", d);
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  return LOGO_OK;
}

static int64_t epi_bwd_grid(int64_t rows, int d) {
  const int rpb = 256 / (d / 8);
  const int64_t nrb = (rows + rpb - 1) / rpb;
  return nrb < kEpiMaxGrid ? (nrb > 0 ? nrb : 1) : kEpiMaxGrid;
}

}  // namespace logo

using namespace logo;

extern "C" int logo_epilogue_fwd(const void* L, const void* G, const void* gate, const void* thres,
                                 int thres_dtype, const void* w_l, const void* w_g, void* out, int64_t n_tokens,
                                 int heads, int d, float eps, int dtype, void* stream) {
  int rc = epi_check(n_tokens, heads, d, dtype, thres_dtype);
  if (rc != LOGO_OK) return rc;
  if (n_tokens == 0) return LOGO_OK;
  LOGO_REQUIRE(L && G && gate && thres && w_l && w_g && out, "null pointer argument");
  EpiArgs a{};
  a.L = static_cast<const bf16*>(L);
  a.G = static_cast<const bf16*>(G);
  a.gate = static_cast<const bf16*>(gate);
  a.thres = thres;
  a.thres_bf16 = thres_dtype == LOGO_DTYPE_BF16;
  a.w_l = static_cast<const bf16*>(w_l);
  a.w_g = static_cast<const bf16*>(w_g);
  a.out = static_cast<bf16*>(out);
  a.rows = n_tokens * heads;
  a.heads = heads;
  a.eps = eps;
  const int rpb = 256 / (d / 8);
  const int64_t nblk = (a.rows + rpb - 1) / rpb;
  hipStream_t st = as_stream(stream);
  if (d == 128) hipLaunchKernelGGL(epi_fwd_kernel<128>, dim3((unsigned)nblk), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(epi_fwd_kernel<64>, dim3((unsigned)nblk), dim3(256), 0, st, a);
  LOGO_LAUNCH_CHECK("epi_fwd_kernel");
  return LOGO_OK;
}

extern "C" size_t logo_epilogue_bwd_workspace_bytes(int64_t n_tokens, int heads, int d) {
  const int64_t rows = n_tokens * heads;
  return (size_t)(rows > 0 ? rows : 1) * sizeof(float) +
         (size_t)epi_bwd_grid(rows, d) * 2 * (size_t)d * sizeof(float);
}

extern "C" int logo_epilogue_bwd(const void* L, const void* G, const void* gate, const void* thres,
                                 int thres_dtype, const void* w_l, const void* w_g, const void* dout, void* dL,
                                 void* dG, void* dgate, void* dw_l, void* dw_g, int64_t n_tokens,
                                 int heads, int d, float eps, void* workspace, int dtype,
                                 void* stream) {
  int rc = epi_check(n_tokens, heads, d, dtype, thres_dtype);
  if (rc != LOGO_OK) return rc;
  LOGO_REQUIRE(L && G && gate && thres && w_l && w_g && dout && dL && dG && dgate && dw_l && dw_g &&
                   workspace,
               "null pointer argument");
  EpiArgs a{};
  a.L = static_cast<const bf16*>(L);
  a.G = static_cast<const bf16*>(G);
  a.gate = static_cast<const bf16*>(gate);
  a.thres = thres;
  a.thres_bf16 = thres_dtype == LOGO_DTYPE_BF16;
  a.w_l = static_cast<const bf16*>(w_l);
  a.w_g = static_cast<const bf16*>(w_g);
  a.dout = static_cast<const bf16*>(dout);
  a.dL = static_cast<bf16*>(dL);
  a.dG = static_cast<bf16*>(dG);
  a.dgate = static_cast<bf16*>(dgate);
  a.dw_l = static_cast<bf16*>(dw_l);
  a.dw_g = static_cast<bf16*>(dw_g);
  a.rows = n_tokens * heads;
  a.heads = heads;
  a.eps = eps;
  a.dgate_part = static_cast<float*>(workspace);
  a.dw_part = a.dgate_part + (a.rows > 0 ? a.rows : 1);
  const int64_t grid = epi_bwd_grid(a.rows, d);
  hipStream_t st = as_stream(stream);
  if (d == 128) hipLaunchKernelGGL(epi_bwd_kernel<128>, dim3((unsigned)grid), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(epi_bwd_kernel<64>, dim3((unsigned)grid), dim3(256), 0, st, a);
  LOGO_LAUNCH_CHECK("epi_bwd_kernel");
  const int tok_blocks = (int)((n_tokens + 255) / 256);
  const int fblk = tok_blocks + 2 * d / kEpiDwCols;
  if (d == 128)
    hipLaunchKernelGGL(epi_bwd_finalize_kernel<128>, dim3((unsigned)fblk), dim3(256), 0, st, a, n_tokens, (int)grid,
                       tok_blocks);
  else
    hipLaunchKernelGGL(epi_bwd_finalize_kernel<64>, dim3((unsigned)fblk), dim3(256), 0, st, a, n_tokens, (int)grid,
                       tok_blocks);
  LOGO_LAUNCH_CHECK("epi_bwd_finalize_kernel");
  return LOGO_OK;
}
