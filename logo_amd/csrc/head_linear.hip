// Per-head linear maps of LoGo's global re-parameterisation at training sizes,
// on the [N, H, D] activation layout in place (logo/layers/logo.py:86-94,
// einsum("bthd,hde->bthe") with one [D, D] matrix per head).
//
// The eager formulation moves every activation to a head-major copy for a
// batched GEMM and back (two full copies per projection forward, more in the
// backward).  Here:
//   * head_linear_kernel: y[n, h, :] = x[n, h, :] W_h (or W_h^T for the input
//     gradient), reading x rows with their head offset and writing y rows the
//     same way.  A workgroup stages W_h in LDS once (rows padded, conflict-free
//     16-byte reads) and runs up to kHlMaxPasses passes of 128 tokens (32 per wave, one
//     32x32x16 MFMA chain per 32 output columns), each wave loading its next
//     pass's rows while it computes the current one; each wave's output tile
//     goes through LDS so the stores are 16-byte row chunks.
//     With an addend (ADD), each stored element is bf16(bf16(y) + a): the
//     input gradient summed with the other gradient of the same tensor, with
//     the two roundings of a bf16 product followed by an eager bf16 add, in
//     place of a separate add pass (a may alias y: each lane reads its chunk
//     of a before it writes the same chunk of y).
//   * head_linear_dw_kernel: the weight gradient dW_h = X_h^T dY_h over a chunk
//     of tokens per workgroup (64-token tiles of X_h and dY_h copied global ->
//     LDS, both operands read transposed), fp32 partials per chunk, then
//     head_linear_dw_reduce_kernel sums the chunks in a fixed order
//     (deterministic; no cross-workgroup synchronisation).
#include "capi.hpp"
#include "common.hpp"

namespace logo {

int device_cus();  // sq_attn.hip

constexpr int kHlRows = 128;     // tokens per pass (4 waves x 32)
constexpr int kHlMaxPasses = 8;  // passes per workgroup (W_h staged once)
constexpr int kHlWgsPerCu = 2;   // 66 KB of LDS per workgroup
constexpr int kHlChunk = 1024;  // tokens per weight-gradient workgroup

struct HlArgs {
  const bf16* x;  // x[n * ldx + h * D + k]
  int64_t ldx;
  const bf16* w;  // [H, D, D]
  bf16* y;        // y[n * ldy + h * D + c]
  int64_t ldy;
  int64_t n;
  const bf16* add;  // ADD: add[n * ldadd + h * D + c]
  int64_t ldadd;
  int passes;       // 128-token passes per workgroup
};

// TW = false: y = x W_h;  TW = true: y = x W_h^T.  ADD: y = bf16(bf16(y) + add).
template <int D, bool TW, bool ADD = false>
__global__ __launch_bounds__(256) void head_linear_kernel(const HlArgs a) {
  constexpr int RS = D + 8;  // padded LDS row (elements)
  constexpr int DS = D / 16, CT = D / 32;
  // wb[c][k]: the MFMA's B operand, output column c, contraction index k
  __shared__ __attribute__((aligned(16))) bf16 wb[D * RS];
  __shared__ __attribute__((aligned(16))) bf16 ys[4][32 * RS];
  const int h = blockIdx.y;
  const bf16* wh = a.w + (int64_t)h * D * D;
  for (int idx = threadIdx.x; idx < D * D / 8; idx += 256) {
    const int r = idx / (D / 8), c8 = (idx % (D / 8)) * 8;  // W_h[r][c8 .. c8 + 7]
    const bf16x8 v = *reinterpret_cast<const bf16x8*>(wh + r * D + c8);
    if constexpr (TW) {
      *reinterpret_cast<bf16x8*>(wb + r * RS + c8) = v;  // B[k][c] = W[c][k]
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) wb[(c8 + j) * RS + r] = v[j];  // B[k][c] = W[k][c]
    }
  }
  __syncthreads();
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, i = l & 31, g = l >> 5;
  bf16* yw = ys[wave];
  // rows past n read the last row; they are not stored
  auto row_of = [&](int pass) { return ((int64_t)blockIdx.x * a.passes + pass) * kHlRows + 32 * wave; };
  auto load_x = [&](int64_t r0, bf16x8* dst) {
    const bf16* xr = a.x + (r0 + i < a.n ? r0 + i : a.n - 1) * a.ldx + (int64_t)h * D + 8 * g;
#pragma unroll
    for (int s = 0; s < DS; ++s) dst[s] = *reinterpret_cast<const bf16x8*>(xr + 16 * s);
  };
  bf16x8 nx[DS];  // the next pass's rows, loaded while this pass computes
  if (row_of(0) < a.n) load_x(row_of(0), nx);
  for (int pass = 0; pass < a.passes; ++pass) {
    const int64_t r0 = row_of(pass);
    if (r0 >= a.n) break;  // wave-uniform; no barrier follows
    bf16x8 av[DS];
#pragma unroll
    for (int s = 0; s < DS; ++s) av[s] = nx[s];
    if (pass + 1 < a.passes && row_of(pass + 1) < a.n) load_x(row_of(pass + 1), nx);
    // ADD: this pass's addend chunks (the ones this lane stores below), all
    // loaded before the MFMAs; loaded in the store loop, each would wait out
    // its own latency (y may alias add, so no load moves above a store)
    constexpr int NIT = 32 * D / 8 / 64;
    bf16x8 adv[ADD ? NIT : 1];
    if constexpr (ADD) {
#pragma unroll
      for (int it = 0; it < NIT; ++it) {
        const int idx = it * 64 + l, rr = idx / (D / 8), c8 = (idx % (D / 8)) * 8;
        const int64_t row = r0 + rr < a.n ? r0 + rr : a.n - 1;
        adv[it] = *reinterpret_cast<const bf16x8*>(a.add + row * a.ldadd + (int64_t)h * D + c8);
      }
    }
    f32x16 acc[CT];
#pragma unroll
    for (int ct = 0; ct < CT; ++ct) {
      acc[ct] = f32x16{};
#pragma unroll
      for (int s = 0; s < DS; ++s) {
        const bf16x8 bv = lds_load(reinterpret_cast<const bf16x8*>(wb + (32 * ct + i) * RS + 16 * s + 8 * g));
        acc[ct] = mfma32(av[s], bv, acc[ct]);
      }
    }
    // acc[ct] item 4m + e of lane (i, g): token r0 + 8m + 4g + e, column 32ct + i
#pragma unroll
    for (int ct = 0; ct < CT; ++ct)
#pragma unroll
      for (int jj = 0; jj < 16; ++jj) yw[(8 * (jj / 4) + 4 * g + (jj % 4)) * RS + 32 * ct + i] = (bf16)acc[ct][jj];
    // each lane stores 16-byte chunks of the wave's 32 output rows
#pragma unroll
    for (int it = 0; it < NIT; ++it) {
      const int idx = it * 64 + l, rr = idx / (D / 8), c8 = (idx % (D / 8)) * 8;
      bf16x8 v = lds_load(reinterpret_cast<const bf16x8*>(yw + rr * RS + c8));
      if (r0 + rr < a.n) {
        if constexpr (ADD) {
#pragma unroll
          for (int j = 0; j < 8; ++j) v[j] = (bf16)((float)v[j] + (float)adv[it][j]);
        }
        *reinterpret_cast<bf16x8*>(a.y + (r0 + rr) * a.ldy + (int64_t)h * D + c8) = v;
      }
    }
  }
}

struct HlwArgs {
  const bf16* x;  // x[n * ldx + h * D + d]
  int64_t ldx;
  const bf16* dy;  // dy[n * ldy + h * D + e]
  int64_t ldy;
  float* part;  // [H, nchunk, D, D]
  int64_t n;
  int nchunk;
};

template <int D>
__global__ __launch_bounds__(256) void head_linear_dw_kernel(const HlwArgs a) {
  static_assert(D == 128, "one 32-row block of dW per wave");
  constexpr int TILE = 64 * D;  // elements of one swizzled 64-row tile
  extern __shared__ __attribute__((aligned(16))) char hl_smem[];
  bf16* const smem = reinterpret_cast<bf16*>(hl_smem);
  auto tx = [&](int b) { return smem + 2 * b * TILE; };
  auto tdy = [&](int b) { return smem + (2 * b + 1) * TILE; };
  const int c = blockIdx.x, h = blockIdx.y;
  const int64_t t_lo = (int64_t)c * kHlChunk;
  const int64_t t_hi = t_lo + kHlChunk < a.n ? t_lo + kHlChunk : a.n;
  const int ntile = (int)((t_hi - t_lo + 63) / 64);
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, i = l & 31, g = l >> 5;
  TileBufDma<D> dx, ddy;
  dx.init((int)a.ldx);
  ddy.init((int)a.ldy);
  TileReader<D, kSwz> rd;
  rd.init();
  auto load = [&](int it, int b) {
    const int64_t t0 = t_lo + 64 * it;
    const bf16* xs = a.x + t0 * a.ldx + (int64_t)h * D;
    const bf16* ds = a.dy + t0 * a.ldy + (int64_t)h * D;
    if (t0 + 64 <= t_hi) {
      dx.issue(tx(b), xs);
      ddy.issue(tdy(b), ds);
    } else {
      dx.issue_clamped(tx(b), xs, (int)(t_hi - 1 - t0));
      ddy.issue_clamped(tdy(b), ds, (int)(t_hi - 1 - t0));
    }
  };
  f32x16 acc[D / 32];
#pragma unroll
  for (int eb = 0; eb < D / 32; ++eb) acc[eb] = f32x16{};
  load(0, 0);
  for (int it = 0; it < ntile; ++it) {
    const int b = it & 1;
    wait_vmem();
    __syncthreads();  // tile it landed for every wave; tile it - 1's buffer is free
    if (it + 1 < ntile) load(it + 1, b ^ 1);
    const int valid = (int)(t_hi - (t_lo + 64 * it));
    if (valid < 64) {
      // clamped rows repeat the last token: zero their dY so they add nothing
      for (int idx = threadIdx.x; idx < (64 - valid) * D / 8; idx += 256)
        *reinterpret_cast<bf16x8*>(tdy(b) + valid * D + 8 * idx) = bf16x8{};
      __syncthreads();
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const bf16x8 av = rd.tr(tx(b), 16 * ks, wave);  // X^T: d = 32 wave + i
#pragma unroll
      for (int eb = 0; eb < D / 32; ++eb) acc[eb] = mfma32(av, rd.tr(tdy(b), 16 * ks, eb), acc[eb]);
    }
  }
  // acc[eb] item 4m + e of lane (i, g): d = 32 wave + 8m + 4g + e, column e' = 32 eb + i
  float* p = a.part + (((int64_t)h * a.nchunk + c) * D) * D;
#pragma unroll
  for (int eb = 0; eb < D / 32; ++eb)
#pragma unroll
    for (int jj = 0; jj < 16; ++jj) p[(32 * wave + 8 * (jj / 4) + 4 * g + (jj % 4)) * D + 32 * eb + i] = acc[eb][jj];
}

// dw[h, d, e] = sum over chunks, in chunk order.
template <int D>
__global__ __launch_bounds__(256) void head_linear_dw_reduce_kernel(const float* part, bf16* dw, int h, int nchunk) {
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)h * D * D) return;
  const int64_t hh = idx / (D * D), de = idx % (D * D);
  const float* p = part + hh * nchunk * D * D + de;
  float s = 0.f;
  for (int k = 0; k < nchunk; ++k) s += p[(int64_t)k * D * D];
  dw[idx] = (bf16)s;
}

}  // namespace logo

using namespace logo;

static constexpr size_t kHlDwSmem = (size_t)4 * 64 * 128 * sizeof(bf16);

static int head_linear_launch(const void* x, int64_t ldx, const void* w, const void* add, int64_t ldadd, void* y,
                              int64_t ldy, int64_t n_tokens, int heads, int d, int transpose_w, int dtype,
                              void* stream) {
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  LOGO_REQUIRE(d == 64 || d == 128, "head dim %d unsupported (64 or 128)", d);
  LOGO_REQUIRE(n_tokens >= 0 && heads >= 1, "bad token / head counts");
  LOGO_REQUIRE(ldx >= (int64_t)heads * d && ldy >= (int64_t)heads * d && ldx % 8 == 0 && ldy % 8 == 0,
               "row strides must cover heads * d and be multiples of 8");
  LOGO_REQUIRE(x && w && y, "null pointer argument");
  LOGO_REQUIRE(((uintptr_t)x | (uintptr_t)w | (uintptr_t)y) % 16 == 0, "x, w, y must be 16-byte aligned");
  if (add) {
    LOGO_REQUIRE(ldadd >= (int64_t)heads * d && ldadd % 8 == 0 && (uintptr_t)add % 16 == 0,
                 "the addend's row stride must cover heads * d and be a multiple of 8, the addend 16-byte aligned");
    LOGO_REQUIRE(transpose_w, "the addend form is the input gradient (transpose_w = 1)");
  }
  if (n_tokens == 0) return LOGO_OK;
  HlArgs a{};
  a.x = static_cast<const bf16*>(x);
  a.ldx = ldx;
  a.w = static_cast<const bf16*>(w);
  a.y = static_cast<bf16*>(y);
  a.ldy = ldy;
  a.n = n_tokens;
  a.add = static_cast<const bf16*>(add);
  a.ldadd = ldadd;
  // as many passes as fill every workgroup slot once (W_h staged fewer times:
  // at 32K tokens x 16 heads, 8 passes took 54 / 49 / 96 us for the forward,
  // input gradient and addend form against 58 / 55 / 108 us with 4)
  const int cus = device_cus();
  const int64_t fill = cus > 0 ? n_tokens * heads / ((int64_t)kHlRows * kHlWgsPerCu * cus) : 4;
  a.passes = (int)std::min<int64_t>(kHlMaxPasses, std::max<int64_t>(1, fill));
  const int64_t per = (int64_t)kHlRows * a.passes;
  const int64_t nblk = (n_tokens + per - 1) / per;
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "too many tokens");
  const dim3 grid((unsigned)nblk, (unsigned)heads);
  hipStream_t st = as_stream(stream);
  if (d == 128) {
    if (add) hipLaunchKernelGGL((head_linear_kernel<128, true, true>), grid, dim3(256), 0, st, a);
    else if (transpose_w) hipLaunchKernelGGL((head_linear_kernel<128, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((head_linear_kernel<128, false>), grid, dim3(256), 0, st, a);
  } else {
    if (add) hipLaunchKernelGGL((head_linear_kernel<64, true, true>), grid, dim3(256), 0, st, a);
    else if (transpose_w) hipLaunchKernelGGL((head_linear_kernel<64, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((head_linear_kernel<64, false>), grid, dim3(256), 0, st, a);
  }
  LOGO_LAUNCH_CHECK("head_linear_kernel");
  return LOGO_OK;
}

extern "C" int logo_head_linear(const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int64_t n_tokens,
                                int heads, int d, int transpose_w, int dtype, void* stream) {
  return head_linear_launch(x, ldx, w, nullptr, 0, y, ldy, n_tokens, heads, d, transpose_w, dtype, stream);
}

extern "C" int logo_head_linear_grad_acc(const void* dy, int64_t lddy, const void* w, const void* add,
                                         int64_t ldadd, void* dx, int64_t lddx, int64_t n_tokens, int heads, int d,
                                         int dtype, void* stream) {
  LOGO_REQUIRE(add, "null pointer argument");
  return head_linear_launch(dy, lddy, w, add, ldadd, dx, lddx, n_tokens, heads, d, 1, dtype, stream);
}

extern "C" size_t logo_head_linear_dw_workspace_bytes(int64_t n_tokens, int heads, int d) {
  const int64_t nchunk = n_tokens > 0 ? (n_tokens + kHlChunk - 1) / kHlChunk : 1;
  return (size_t)heads * nchunk * d * d * sizeof(float);
}

extern "C" int logo_head_linear_dw(const void* x, int64_t ldx, const void* dy, int64_t ldy, void* dw, void* workspace,
                                   int64_t n_tokens, int heads, int d, int dtype, void* stream) {
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  LOGO_REQUIRE(d == 128, "head dim %d unsupported (128)", d);
  LOGO_REQUIRE(n_tokens >= 1 && heads >= 1, "bad token / head counts");
  LOGO_REQUIRE(ldx >= (int64_t)heads * d && ldy >= (int64_t)heads * d && ldx % 8 == 0 && ldy % 8 == 0,
               "row strides must cover heads * d and be multiples of 8");
  LOGO_REQUIRE(64 * ldx * 2 < ((int64_t)1 << 31) && 64 * ldy * 2 < ((int64_t)1 << 31), "row strides too large");
  LOGO_REQUIRE(x && dy && dw && workspace, "null pointer argument");
  LOGO_REQUIRE(((uintptr_t)x | (uintptr_t)dy) % 16 == 0, "x and dy must be 16-byte aligned");
  const int64_t nchunk = (n_tokens + kHlChunk - 1) / kHlChunk;
  LOGO_REQUIRE(nchunk < ((int64_t)1 << 31), "too many tokens");
  HlwArgs a{};
  a.x = static_cast<const bf16*>(x);
  a.ldx = ldx;
  a.dy = static_cast<const bf16*>(dy);
  a.ldy = ldy;
  a.part = static_cast<float*>(workspace);
  a.n = n_tokens;
  a.nchunk = (int)nchunk;
  hipStream_t st = as_stream(stream);
  auto kern = head_linear_dw_kernel<128>;
  LOGO_HIP_CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, (int)kHlDwSmem));
  hipLaunchKernelGGL(kern, dim3((unsigned)nchunk, (unsigned)heads), dim3(256), kHlDwSmem, st, a);
  LOGO_LAUNCH_CHECK("head_linear_dw_kernel");
  const int64_t total = (int64_t)heads * d * d;
  hipLaunchKernelGGL(head_linear_dw_reduce_kernel<128>, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st,
                     a.part, static_cast<bf16*>(dw), heads, (int)nchunk);
  LOGO_LAUNCH_CHECK("head_linear_dw_reduce_kernel");
  return LOGO_OK;
}
