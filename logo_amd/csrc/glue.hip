// Fused glue of the LoGo layer and model for gfx950: rotary embedding and
// RMSNorm, each in one launch instead of a chain of eager element-wise ops.
//
// RoPE (logo/modules/rotary.py:81-106): x' = bf16(bf16(x * cos) +
// bf16(rotate_half(x) * sin)) with rotate_half(x) = [-x2, x1], the rounding
// points of the reference's eager bf16 ops kept (products of two bf16 values
// are exact in fp32, so each rounds exactly as the eager op does).  Up to four
// [N, H_i, D] tensors (q, k and the global q, k) are rotated with one [N, D]
// cos / sin pair, in place or into separate outputs.  The inverse rotation is
// the backward: eager autograd of the forward gives
//   dx1 = bf16(bf16(dy1 * cos1) + bf16(dy2 * sin2))
//   dx2 = bf16(bf16(dy2 * cos2) + bf16(-(dy1 * sin1)))
// (mul backward rounds each product; rotate_half's cat / neg backward moves
// and negates exactly; the two contributions are summed in bf16), and the
// kernel keeps those rounding points too.
//
// RMSNorm (logo/modules/layernorm.py:17-22): y = bf16(w * bf16(x *
// rsqrt(mean(x^2) + eps))), the mean taken in fp32.
//
// Per-head projection for a few tokens (the LoGo global re-parameterisation
// at decode, logo/layers/logo.py:86-94: gq = q W_q[h], gk = k W_k[h],
// gv = v W_v[h] per head): one launch for the three tensors instead of three
// batched GEMMs and six layout copies; fp32 accumulation, one bf16 rounding.
#include <math.h>

#include "capi.hpp"
#include "common.hpp"

// every product and sum rounds as its own eager bf16 op (no fma contraction)
#pragma clang fp contract(off)

namespace logo {

struct RopeArgs {
  const bf16* x[4];
  bf16* y[4];
  int heads[4];
  int nt;  // tensors in use
  const bf16* cos;
  const bf16* sin;
  int64_t n;  // rows (tokens)
};

__device__ __forceinline__ float bfr_g(float x) { return (float)(bf16)x; }

// One thread per (tensor, token, head, 8-element chunk of the first half):
// it rotates the pair of chunks (c, c + D/16) together (reading both before
// writing either, so x == y is allowed).
template <int D, bool INV>
__global__ __launch_bounds__(256) void rope_kernel(const RopeArgs a, int64_t per_tensor_max) {
  constexpr int HC = D / 16;  // chunks of 8 in each half
  const int ti = blockIdx.y;
  if (ti >= a.nt) return;
  const int H = a.heads[ti];
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t total = a.n * H * HC;
  if (idx >= total || idx >= per_tensor_max) return;
  const int c = (int)(idx % HC);
  const int64_t row = idx / HC;  // token * H + head
  const int64_t tok = row / H;
  const bf16* xr = a.x[ti] + row * D;
  bf16* yr = a.y[ti] + row * D;
  const bf16x8 x1 = ld_nt(reinterpret_cast<const bf16x8*>(xr + 8 * c));
  const bf16x8 x2 = ld_nt(reinterpret_cast<const bf16x8*>(xr + D / 2 + 8 * c));
  const bf16x8 c1 = *reinterpret_cast<const bf16x8*>(a.cos + tok * D + 8 * c);
  const bf16x8 c2 = *reinterpret_cast<const bf16x8*>(a.cos + tok * D + D / 2 + 8 * c);
  const bf16x8 s1 = *reinterpret_cast<const bf16x8*>(a.sin + tok * D + 8 * c);
  const bf16x8 s2 = *reinterpret_cast<const bf16x8*>(a.sin + tok * D + D / 2 + 8 * c);
  bf16x8 y1, y2;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if constexpr (!INV) {
      // first half:  x1 * cos1 + (-x2) * sin1;  second half: x2 * cos2 + x1 * sin2
      const float a1 = bfr_g((float)x1[e] * (float)c1[e]);
      const float b1 = bfr_g(-(float)x2[e] * (float)s1[e]);
      const float a2 = bfr_g((float)x2[e] * (float)c2[e]);
      const float b2 = bfr_g((float)x1[e] * (float)s2[e]);
      y1[e] = (bf16)(a1 + b1);
      y2[e] = (bf16)(a2 + b2);
    } else {
      // transpose of the rotation: x1 * cos1 + x2 * sin2;  x2 * cos2 - x1 * sin1
      const float a1 = bfr_g((float)x1[e] * (float)c1[e]);
      const float b1 = bfr_g((float)x2[e] * (float)s2[e]);
      const float a2 = bfr_g((float)x2[e] * (float)c2[e]);
      const float b2 = -bfr_g((float)x1[e] * (float)s1[e]);
      y1[e] = (bf16)(a1 + b1);
      y2[e] = (bf16)(a2 + b2);
    }
  }
  st_nt(reinterpret_cast<bf16x8*>(yr + 8 * c), y1);
  st_nt(reinterpret_cast<bf16x8*>(yr + D / 2 + 8 * c), y2);
}

// One wave per row; rows of `cols` bf16 (a multiple of 8, at most 64 * 8 * 8).
template <int VPL>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const bf16* x, const bf16* w, bf16* y, int64_t rows,
                                                      int cols, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  if (row >= rows) return;
  const bf16* xr = x + row * cols;
  bf16x8 v[VPL];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int col = 8 * (l + 64 * k);
    v[k] = col < cols ? *reinterpret_cast<const bf16x8*>(xr + col) : bf16x8{};
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf((float)v[k][e], (float)v[k][e], ss);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  const float r = rsqrtf(ss / (float)cols + eps);
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int col = 8 * (l + 64 * k);
    if (col < cols) {
      const bf16x8 wv = *reinterpret_cast<const bf16x8*>(w + col);
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)((float)wv[e] * bfr_g((float)v[k][e] * r));
      *reinterpret_cast<bf16x8*>(y + row * cols + col) = o;
    }
  }
}

struct HeadProjArgs {
  const bf16* x[3];  // [T, H_i, D]
  const bf16* w[3];  // [H_i, D, E]
  bf16* y[3];        // [T, H_i, E]
  int heads[3];
  int head0[4];      // prefix of heads over the tensors
  int nt, t, d, e;
};

constexpr int kHpTok = 8;  // tokens per workgroup

// Workgroup (global head gh, token block): thread n computes output column n
// of kHpTok tokens; W's row k is read once per block (coalesced over n) and
// the tokens' x rows sit in LDS.
__global__ __launch_bounds__(128) void head_proj_kernel(const HeadProjArgs a) {
  const int gh = blockIdx.x;
  int ti = 0;
  while (ti + 1 < a.nt && gh >= a.head0[ti + 1]) ++ti;
  const int h = gh - a.head0[ti], H = a.heads[ti];
  const int t0 = blockIdx.y * kHpTok;
  const int n = threadIdx.x;
  __shared__ float xs[kHpTok][256];
  for (int idx = threadIdx.x; idx < kHpTok * a.d; idx += 128) {
    const int tt = idx / a.d, k = idx % a.d;
    const int t = t0 + tt;
    xs[tt][k] = t < a.t ? (float)a.x[ti][((int64_t)t * H + h) * a.d + k] : 0.f;
  }
  __syncthreads();
  if (n >= a.e) return;
  const bf16* w = a.w[ti] + (int64_t)h * a.d * a.e + n;
  float acc[kHpTok];
#pragma unroll
  for (int tt = 0; tt < kHpTok; ++tt) acc[tt] = 0.f;
  for (int k = 0; k < a.d; ++k) {
    const float wk = (float)w[(int64_t)k * a.e];
#pragma unroll
    for (int tt = 0; tt < kHpTok; ++tt) acc[tt] = fmaf(xs[tt][k], wk, acc[tt]);
  }
#pragma unroll
  for (int tt = 0; tt < kHpTok; ++tt) {
    const int t = t0 + tt;
    if (t < a.t) a.y[ti][((int64_t)t * H + h) * a.e + n] = (bf16)acc[tt];
  }
}

// Residual add + RMSNorm of the decoder (logo/modeling_logo.py:60-66 with
// logo/modules/layernorm.py:17-22): s = bf16(r + x) (the eager bf16 add) and
// y = bf16(w * bf16(s * rsqrt(mean(s^2) + eps))), one wave per row.
template <int VPL>
__global__ __launch_bounds__(256) void add_rmsnorm_kernel(const bf16* r, const bf16* x, const bf16* w, bf16* s_out,
                                                          bf16* y, int64_t rows, int cols, float eps) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  if (row >= rows) return;
  bf16x8 v[VPL];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int col = 8 * (l + 64 * k);
    if (col < cols) {
      const bf16x8 rv = *reinterpret_cast<const bf16x8*>(r + row * cols + col);
      const bf16x8 xv = *reinterpret_cast<const bf16x8*>(x + row * cols + col);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[k][e] = (bf16)((float)rv[e] + (float)xv[e]);
      *reinterpret_cast<bf16x8*>(s_out + row * cols + col) = v[k];
    } else {
      v[k] = bf16x8{};
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) ss = fmaf((float)v[k][e], (float)v[k][e], ss);
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) ss += __shfl_xor(ss, off);
  const float rs = rsqrtf(ss / (float)cols + eps);
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int col = 8 * (l + 64 * k);
    if (col < cols) {
      const bf16x8 wv = *reinterpret_cast<const bf16x8*>(w + col);
      bf16x8 o;
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = (bf16)((float)wv[e] * bfr_g((float)v[k][e] * rs));
      *reinterpret_cast<bf16x8*>(y + row * cols + col) = o;
    }
  }
}

// SwiGLU activation of logo/modules/mlp.py:24-27: y = bf16(bf16(silu(g)) * u)
// with silu(g) = g / (1 + exp(-g)) in fp32 (the rounding of the eager bf16
// F.silu and mul); g and u are the two halves of a stacked projection row.
__global__ __launch_bounds__(256) void silu_mul_kernel(const bf16* gu, int64_t ld, bf16* y, int64_t rows,
                                                       int cols) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = idx / (cols / 8);
  const int c8 = (int)(idx % (cols / 8)) * 8;
  if (row >= rows) return;
  const bf16x8 g = *reinterpret_cast<const bf16x8*>(gu + row * ld + c8);
  const bf16x8 u = *reinterpret_cast<const bf16x8*>(gu + row * ld + cols + c8);
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float gf = (float)g[e];
    const float sg = bfr_g(gf / (1.f + expf(-gf)));
    o[e] = (bf16)(sg * (float)u[e]);
  }
  *reinterpret_cast<bf16x8*>(y + row * cols + c8) = o;
}

// One decode step's q / k / v transform for a LoGo layer: from the stacked
// projection output row of each token ([q | k | v], row stride ldq), the
// global projections (as head_proj), RoPE of q, k, gq, gk (the rounding of
// rope_kernel) and both cache appends (k, v into the local ring at pos % ring,
// gk, gv into the global cache at pos), replacing head_proj, rope and two
// cache_append launches.  Outputs q (local, rotated) and gq (rotated), and,
// when gate_out is set, the gate sigmoid(qkv[b, gate_col]) of each token.
// Each workgroup stages its head's [D, D] projection in LDS with 16-byte
// loads (all in flight at once), then every thread runs the same sequential
// fp32 k-loop as head_proj_kernel for its output column.
struct DecQkvArgs {
  const bf16* qkv;
  int64_t ldq;
  const bf16* w[3];  // [H, D, D], [HK, D, D], [HK, D, D]
  const bf16* cos;   // [B, D]
  const bf16* sin;
  const int32_t* pos;
  bf16* q_out;       // [B, H, D]
  bf16* gq_out;
  bf16* lk;          // [B, HK, ring, D]
  bf16* lv;
  bf16* gk;          // [B, HK, t_cap, D]
  bf16* gv;
  bf16* gate_out;    // [B] or null
  int64_t gate_col;
  int b, h, hk, ring;
  int64_t t_cap;
};

constexpr int kDqTok = 2;  // tokens per decode_qkv workgroup (more workgroups, short k-chains)

template <int D>
__global__ __launch_bounds__(D) void decode_qkv_kernel(const DecQkvArgs a) {
  // blockIdx.x: heads of q (0 .. H-1), then k (H .. H+HK-1), then v
  const int gh = blockIdx.x;
  const int ti = gh < a.h ? 0 : (gh < a.h + a.hk ? 1 : 2);
  const int hh = ti == 0 ? gh : (ti == 1 ? gh - a.h : gh - a.h - a.hk);
  const int col0 = ti == 0 ? hh * D : (ti == 1 ? (a.h + hh) * D : (a.h + a.hk + hh) * D);
  const int t0 = blockIdx.y * kDqTok;
  const int n = threadIdx.x;
  __shared__ bf16x8 wsm[D * D / 8];  // this head's projection, [k][n]
  __shared__ float xs[kDqTok][D];
  __shared__ float ys[kDqTok][D];
  {
    const bf16x8* wsrc = reinterpret_cast<const bf16x8*>(a.w[ti] + (int64_t)hh * D * D);
    bf16x8 wv[D / 8];
#pragma unroll
    for (int i = 0; i < D / 8; ++i) wv[i] = wsrc[i * D + n];
#pragma unroll
    for (int i = 0; i < D / 8; ++i) wsm[i * D + n] = wv[i];
  }
  for (int idx = threadIdx.x; idx < kDqTok * D; idx += D) {
    const int tt = idx / D, k = idx % D;
    const int t = t0 + tt;
    xs[tt][k] = t < a.b ? (float)a.qkv[(int64_t)t * a.ldq + col0 + k] : 0.f;
  }
  if (a.gate_out != nullptr && gh == 0 && n < kDqTok && t0 + n < a.b) {
    const float z = (float)a.qkv[(int64_t)(t0 + n) * a.ldq + a.gate_col];
    a.gate_out[t0 + n] = (bf16)(1.f / (1.f + expf(-z)));
  }
  __syncthreads();
  const bf16* w = reinterpret_cast<const bf16*>(wsm) + n;
  float acc[kDqTok];
#pragma unroll
  for (int tt = 0; tt < kDqTok; ++tt) acc[tt] = 0.f;
  for (int k = 0; k < D; ++k) {
    const float wk = (float)w[k * D];
#pragma unroll
    for (int tt = 0; tt < kDqTok; ++tt) acc[tt] = fmaf(xs[tt][k], wk, acc[tt]);
  }
#pragma unroll
  for (int tt = 0; tt < kDqTok; ++tt) ys[tt][n] = (float)(bf16)acc[tt];
  __syncthreads();
  const int pn = n < D / 2 ? n + D / 2 : n - D / 2;
  for (int tt = 0; tt < kDqTok; ++tt) {
    const int t = t0 + tt;
    if (t >= a.b) break;
    const float x = xs[tt][n], xp = xs[tt][pn];
    const float y = ys[tt][n], yp = ys[tt][pn];
    float xo = x, yo = y;
    if (ti < 2) {
      const float c = (float)a.cos[(int64_t)t * D + n], s = (float)a.sin[(int64_t)t * D + n];
      // first half: v * cos + (-v[n + D/2]) * sin; second half: v * cos + v[n - D/2] * sin
      const float sg = n < D / 2 ? -1.f : 1.f;
      xo = bfr_g(bfr_g(x * c) + bfr_g(sg * xp * s));
      yo = bfr_g(bfr_g(y * c) + bfr_g(sg * yp * s));
    }
    if (ti == 0) {
      const int64_t o = ((int64_t)t * a.h + hh) * D + n;
      a.q_out[o] = (bf16)xo;
      a.gq_out[o] = (bf16)yo;
    } else {
      const int p = a.pos[t];
      const int64_t row = (int64_t)t * a.hk + hh;
      bf16* lc = ti == 1 ? a.lk : a.lv;
      bf16* gc = ti == 1 ? a.gk : a.gv;
      lc[(row * a.ring + p % a.ring) * D + n] = (bf16)xo;
      gc[(row * a.t_cap + p) * D + n] = (bf16)yo;
    }
  }
}

}  // namespace logo

using namespace logo;

static int rope_launch(const void* const xs[4], void* const ys[4], const int hs[4], const void* cos,
                       const void* sin, int64_t n_tokens, int d, int inverse, int dtype, void* stream) {
  LOGO_REQUIRE(d == 64 || d == 128, "head dim %d unsupported (64 or 128)", d);
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  LOGO_REQUIRE(n_tokens >= 0, "n_tokens must be >= 0");
  LOGO_REQUIRE(cos && sin, "null cos / sin");
  RopeArgs a{};
  int hmax = 0;
  for (int i = 0; i < 4; ++i) {
    if (xs[i] == nullptr) continue;
    LOGO_REQUIRE(ys[i] != nullptr, "tensor %d: null output", i);
    LOGO_REQUIRE(hs[i] >= 1, "tensor %d: heads must be >= 1", i);
    a.x[a.nt] = static_cast<const bf16*>(xs[i]);
    a.y[a.nt] = static_cast<bf16*>(ys[i]);
    a.heads[a.nt] = hs[i];
    ++a.nt;
    hmax = hs[i] > hmax ? hs[i] : hmax;
  }
  if (a.nt == 0 || n_tokens == 0) return LOGO_OK;
  a.cos = static_cast<const bf16*>(cos);
  a.sin = static_cast<const bf16*>(sin);
  a.n = n_tokens;
  const int64_t per = n_tokens * hmax * (d / 16);
  const int64_t nblk = (per + 255) / 256;
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "too many rows");
  hipStream_t st = as_stream(stream);
  const dim3 grid((unsigned)nblk, a.nt);
  if (d == 128) {
    if (inverse) hipLaunchKernelGGL((rope_kernel<128, true>), grid, dim3(256), 0, st, a, per);
    else hipLaunchKernelGGL((rope_kernel<128, false>), grid, dim3(256), 0, st, a, per);
  } else {
    if (inverse) hipLaunchKernelGGL((rope_kernel<64, true>), grid, dim3(256), 0, st, a, per);
    else hipLaunchKernelGGL((rope_kernel<64, false>), grid, dim3(256), 0, st, a, per);
  }
  LOGO_LAUNCH_CHECK("rope_kernel");
  return LOGO_OK;
}

extern "C" int logo_rope_apply(void* x0, int h0, void* x1, int h1, void* x2, int h2, void* x3, int h3,
                               const void* cos, const void* sin, int64_t n_tokens, int d, int dtype,
                               void* stream) {
  const void* xs[4] = {x0, x1, x2, x3};
  void* ys[4] = {x0, x1, x2, x3};
  const int hs[4] = {h0, h1, h2, h3};
  return rope_launch(xs, ys, hs, cos, sin, n_tokens, d, 0, dtype, stream);
}

extern "C" int logo_rope(const void* x0, void* y0, int h0, const void* x1, void* y1, int h1, const void* x2,
                         void* y2, int h2, const void* x3, void* y3, int h3, const void* cos, const void* sin,
                         int64_t n_tokens, int d, int inverse, int dtype, void* stream) {
  const void* xs[4] = {x0, x1, x2, x3};
  void* ys[4] = {y0, y1, y2, y3};
  const int hs[4] = {h0, h1, h2, h3};
  return rope_launch(xs, ys, hs, cos, sin, n_tokens, d, inverse, dtype, stream);
}

extern "C" int logo_rmsnorm(const void* x, const void* w, void* y, int64_t rows, int cols, float eps, int dtype,
                            void* stream) {
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  LOGO_REQUIRE(rows >= 0, "rows must be >= 0");
  LOGO_REQUIRE(cols >= 8 && cols % 8 == 0 && cols <= 64 * 8 * 8, "cols must be a multiple of 8 in [8, 4096]");
  LOGO_REQUIRE(x && w && y, "null pointer argument");
  if (rows == 0) return LOGO_OK;
  const int64_t nblk = (rows + 3) / 4;
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "too many rows");
  hipStream_t st = as_stream(stream);
  const int vpl = (cols + 511) / 512;
  const auto xb = static_cast<const bf16*>(x);
  const auto wb = static_cast<const bf16*>(w);
  const auto yb = static_cast<bf16*>(y);
  if (vpl <= 1)
    hipLaunchKernelGGL(rmsnorm_kernel<1>, dim3((unsigned)nblk), dim3(256), 0, st, xb, wb, yb, rows, cols, eps);
  else if (vpl <= 2)
    hipLaunchKernelGGL(rmsnorm_kernel<2>, dim3((unsigned)nblk), dim3(256), 0, st, xb, wb, yb, rows, cols, eps);
  else if (vpl <= 4)
    hipLaunchKernelGGL(rmsnorm_kernel<4>, dim3((unsigned)nblk), dim3(256), 0, st, xb, wb, yb, rows, cols, eps);
  else
    hipLaunchKernelGGL(rmsnorm_kernel<8>, dim3((unsigned)nblk), dim3(256), 0, st, xb, wb, yb, rows, cols, eps);
  LOGO_LAUNCH_CHECK("rmsnorm_kernel");
  return LOGO_OK;
}

extern "C" int logo_head_proj(const void* x0, const void* w0, void* y0, int h0, const void* x1, const void* w1,
                              void* y1, int h1, const void* x2, const void* w2, void* y2, int h2, int n_tokens,
                              int d, int e, int dtype, void* stream) {
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  LOGO_REQUIRE(n_tokens >= 0 && n_tokens <= 4096, "n_tokens (%d) must be in [0, 4096]", n_tokens);
  LOGO_REQUIRE(d >= 1 && d <= 256 && e >= 1 && e <= 128, "d must be in [1, 256] and e in [1, 128] (d %d, e %d)", d,
               e);
  HeadProjArgs a{};
  const void* xs[3] = {x0, x1, x2};
  const void* ws[3] = {w0, w1, w2};
  void* ys[3] = {y0, y1, y2};
  const int hs[3] = {h0, h1, h2};
  int total = 0;
  for (int i = 0; i < 3; ++i) {
    if (xs[i] == nullptr) continue;
    LOGO_REQUIRE(ws[i] && ys[i] && hs[i] >= 1, "tensor %d: null weight / output or no heads", i);
    a.x[a.nt] = static_cast<const bf16*>(xs[i]);
    a.w[a.nt] = static_cast<const bf16*>(ws[i]);
    a.y[a.nt] = static_cast<bf16*>(ys[i]);
    a.heads[a.nt] = hs[i];
    a.head0[a.nt] = total;
    total += hs[i];
    ++a.nt;
  }
  a.head0[a.nt] = total;
  if (a.nt == 0 || n_tokens == 0) return LOGO_OK;
  a.t = n_tokens;
  a.d = d;
  a.e = e;
  const dim3 grid((unsigned)total, (unsigned)((n_tokens + kHpTok - 1) / kHpTok));
  hipLaunchKernelGGL(head_proj_kernel, grid, dim3(128), 0, as_stream(stream), a);
  LOGO_LAUNCH_CHECK("head_proj_kernel");
  return LOGO_OK;
}

extern "C" int logo_decode_qkv(const void* qkv, int64_t ldq, const void* wq, const void* wk, const void* wv,
                               const void* cos, const void* sin, const int32_t* pos, void* q_out, void* gq_out,
                               void* local_k, void* local_v, void* global_k, void* global_v, int64_t gate_col,
                               void* gate_out, int batch, int h, int hk, int d, int ring, int64_t t_cap, int dtype,
                               void* stream) {
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  LOGO_REQUIRE(d == 64 || d == 128, "head dim %d unsupported (64 or 128)", d);
  LOGO_REQUIRE(batch >= 0 && batch <= 4096 && h >= 1 && hk >= 1 && h % hk == 0, "bad batch / head counts");
  LOGO_REQUIRE(ldq >= (int64_t)(h + 2 * hk) * d, "ldq (%lld) shorter than the stacked q | k | v row",
               (long long)ldq);
  LOGO_REQUIRE(ring >= 1 && t_cap >= 1, "ring and t_cap must be positive");
  LOGO_REQUIRE(gate_out == nullptr || (gate_col >= 0 && gate_col < ldq), "gate_col outside the row");
  LOGO_REQUIRE(qkv && wq && wk && wv && cos && sin && pos && q_out && gq_out && local_k && local_v && global_k &&
                   global_v,
               "null pointer argument");
  if (batch == 0) return LOGO_OK;
  DecQkvArgs a{};
  a.qkv = static_cast<const bf16*>(qkv);
  a.ldq = ldq;
  a.w[0] = static_cast<const bf16*>(wq);
  a.w[1] = static_cast<const bf16*>(wk);
  a.w[2] = static_cast<const bf16*>(wv);
  a.cos = static_cast<const bf16*>(cos);
  a.sin = static_cast<const bf16*>(sin);
  a.pos = pos;
  a.q_out = static_cast<bf16*>(q_out);
  a.gq_out = static_cast<bf16*>(gq_out);
  a.lk = static_cast<bf16*>(local_k);
  a.lv = static_cast<bf16*>(local_v);
  a.gk = static_cast<bf16*>(global_k);
  a.gv = static_cast<bf16*>(global_v);
  a.gate_out = static_cast<bf16*>(gate_out);
  a.gate_col = gate_col;
  a.b = batch;
  a.h = h;
  a.hk = hk;
  a.ring = ring;
  a.t_cap = t_cap;
  const dim3 grid((unsigned)(h + 2 * hk), (unsigned)((batch + kDqTok - 1) / kDqTok));
  hipStream_t st = as_stream(stream);
  if (d == 128) hipLaunchKernelGGL(decode_qkv_kernel<128>, grid, dim3(128), 0, st, a);
  else hipLaunchKernelGGL(decode_qkv_kernel<64>, grid, dim3(64), 0, st, a);
  LOGO_LAUNCH_CHECK("decode_qkv_kernel");
  return LOGO_OK;
}

extern "C" int logo_add_rmsnorm(const void* r, const void* x, const void* w, void* s_out, void* y, int64_t rows,
                                int cols, float eps, int dtype, void* stream) {
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  LOGO_REQUIRE(rows >= 0, "rows must be >= 0");
  LOGO_REQUIRE(cols >= 8 && cols % 8 == 0 && cols <= 64 * 8 * 8, "cols must be a multiple of 8 in [8, 4096]");
  LOGO_REQUIRE(r && x && w && s_out && y, "null pointer argument");
  if (rows == 0) return LOGO_OK;
  const int64_t nblk = (rows + 3) / 4;
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "too many rows");
  hipStream_t st = as_stream(stream);
  const int vpl = (cols + 511) / 512;
  const auto rb = static_cast<const bf16*>(r);
  const auto xb = static_cast<const bf16*>(x);
  const auto wb = static_cast<const bf16*>(w);
  const auto sb = static_cast<bf16*>(s_out);
  const auto yb = static_cast<bf16*>(y);
  if (vpl <= 1)
    hipLaunchKernelGGL(add_rmsnorm_kernel<1>, dim3((unsigned)nblk), dim3(256), 0, st, rb, xb, wb, sb, yb, rows, cols, eps);
  else if (vpl <= 2)
    hipLaunchKernelGGL(add_rmsnorm_kernel<2>, dim3((unsigned)nblk), dim3(256), 0, st, rb, xb, wb, sb, yb, rows, cols, eps);
  else if (vpl <= 4)
    hipLaunchKernelGGL(add_rmsnorm_kernel<4>, dim3((unsigned)nblk), dim3(256), 0, st, rb, xb, wb, sb, yb, rows, cols, eps);
  else
    hipLaunchKernelGGL(add_rmsnorm_kernel<8>, dim3((unsigned)nblk), dim3(256), 0, st, rb, xb, wb, sb, yb, rows, cols, eps);
  LOGO_LAUNCH_CHECK("add_rmsnorm_kernel");
  return LOGO_OK;
}

extern "C" int logo_silu_mul(const void* gu, int64_t ld, void* y, int64_t rows, int cols, int dtype, void* stream) {
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  LOGO_REQUIRE(rows >= 0 && cols >= 8 && cols % 8 == 0, "cols must be a positive multiple of 8");
  LOGO_REQUIRE(ld >= 2 * (int64_t)cols && ld % 8 == 0, "ld must hold both halves and be a multiple of 8");
  LOGO_REQUIRE(gu && y, "null pointer argument");
  if (rows == 0) return LOGO_OK;
  const int64_t total = rows * (cols / 8);
  const int64_t nblk = (total + 255) / 256;
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "too many rows");
  hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)nblk), dim3(256), 0, as_stream(stream),
                     static_cast<const bf16*>(gu), ld, static_cast<bf16*>(y), rows, cols);
  LOGO_LAUNCH_CHECK("silu_mul_kernel");
  return LOGO_OK;
}
