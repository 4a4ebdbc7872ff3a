// Gate-aware decode attention for gfx950 (one new query token per sequence).
//
// The reference's decode step (logo/layers/logo.py:228-249) syncs the host on
// active.any() and, if any row's gate passes, runs dense attention over the
// whole global KV cache for every row, then masks the inactive rows to zero.
// Here each (sequence, head) reads the cache only if its gate passes
// (gate >= thres, decided on the device), so HBM traffic scales with the
// number of active rows.  The same kernel serves the local branch over the
// 129-slot window ring (all rows active).
//
// Cache layout is logo/cache.py's: K/V [B, H, T, D] per layer (preallocated to
// T_cap instead of grown with torch.cat, logo/cache.py:115-118).
//
// Split-K: a 256-thread workgroup takes 256 keys of one (b, kv-head); each wave
// takes 64 of them with lane l owning key 4s + l/16 (s = 0..15) and the 16-byte
// column chunk l % 16, so every K/V load is a contiguous 256-byte row per 16
// lanes.  The keys stay in registers while the workgroup serves every query
// head of the GQA group in turn (one cache read per group, not per query
// head).  Per query head, the waves merge through LDS into one (max, sum,
// o[D]) partial; a combine kernel merges the partials of a row and normalises.
#include <math.h>

#include "capi.hpp"
#include "common.hpp"

namespace logo {

constexpr int kDecKeysPerWave = 64;
constexpr int kDecKeysPerWG = 256;
constexpr int kDecHeadsPerPass = 8;  // query heads merged per barrier (LDS: 8 x 4 x D floats)

struct DecArgs {
  const bf16* q;        // [B, HQ, D]
  const bf16* k;        // [B, H, T_cap, D]
  const bf16* v;
  const int32_t* lens;  // [B] keys per row
  const bf16* gate;     // [B] or null (all active)
  const void* thres;
  bool thres_bf16;
  bf16* out;            // [B, HQ, D]
  float* part;          // [B*HQ, nsplit, D + 2]
  int batch, hq, h, g, nsplit;
  int64_t t_cap;
  float scale_log2;
};

__device__ __forceinline__ bool dec_active(const DecArgs& a, int b) {
  return a.gate == nullptr || !((float)a.gate[b] < load_thres(a.thres, a.thres_bf16));
}

// One workgroup's split: keys [256 split, 256 split + 256) of kv row
// bh = b * H + h, for the query heads hq = h * G .. h * G + G - 1 (rows
// bq = b * HQ + hq).
// GQA: groups of more than one query head (the keys stay live across the
// heads; G = 1 lets them die after scoring, for a higher occupancy).
template <int D, bool GQA>
__device__ __forceinline__ void dec_split(const DecArgs& a, const int split, const int bh) {
  constexpr int CH = D / 8;                 // 16-byte chunks per row
  constexpr int KPS = 64 / CH;              // keys per load step (4 for D=128)
  constexpr int STEPS = kDecKeysPerWave / KPS;
  const int b = bh / a.h, h = bh % a.h;
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63;
  const int len = a.lens[b];
  const int k0 = split * kDecKeysPerWG;
  // a single split writes the output itself (no combine launch)
  if (!dec_active(a, b) || k0 >= len) {
    if (a.nsplit == 1 && tid < D)
      for (int j = 0; j < a.g; ++j) a.out[((int64_t)b * a.hq + h * a.g + j) * D + tid] = (bf16)0.f;
    return;
  }
  const int c = l % CH, kk = l / CH;
  const int kw = k0 + wave * kDecKeysPerWave;

  const bf16* kb = a.k + ((int64_t)b * a.h + h) * a.t_cap * D + 8 * c;
  const bf16* vb = a.v + ((int64_t)b * a.h + h) * a.t_cap * D + 8 * c;

  // The cache rows are streamed once per step: non-temporal loads (a
  // streaming read of the decode layer's bytes runs at ~7.1 TB/s with them,
  // ~6.3 TB/s without, on one MI355X)
  bf16x8 kr[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int key = kw + KPS * s + kk;
    kr[s] = key < len ? __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(kb + (int64_t)key * D)) : bf16x8{};
  }
  bf16x8 vr[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int key = kw + KPS * s + kk;
    vr[s] = key < len ? __builtin_nontemporal_load(reinterpret_cast<const bf16x8*>(vb + (int64_t)key * D)) : bf16x8{};
  }
  // Query heads in chunks of kDecHeadsPerPass: each head's wave partials go
  // to LDS, and one barrier later the chunk's rows are merged together; the
  // next head's q is loaded while the current one is scored.
  __shared__ float sm[kDecHeadsPerPass][4], sl[kDecHeadsPerPass][4];
  __shared__ float so[kDecHeadsPerPass][4][D];
  const bf16* qg = a.q + ((int64_t)b * a.hq + h * a.g) * D + 8 * c;
  bf16x8 qn = *reinterpret_cast<const bf16x8*>(qg);
  const int G = GQA ? a.g : 1;
  for (int j0 = 0; j0 < G; j0 += kDecHeadsPerPass) {
    const int nj = GQA ? min(kDecHeadsPerPass, G - j0) : 1;
    if (j0 > 0) __syncthreads();  // the previous chunk's merge has read so / sm / sl
    for (int jj = 0; jj < nj; ++jj) {
      // keep the keys and values packed across heads (converting them once
      // for all heads would hold 8x their registers)
      if constexpr (GQA) {
#pragma unroll
        for (int s = 0; s < STEPS; ++s) {
          pin(kr[s]);
          pin(vr[s]);
        }
      }
      float qv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) qv[e] = (float)qn[e] * a.scale_log2;
      if (GQA && j0 + jj + 1 < G) qn = *reinterpret_cast<const bf16x8*>(qg + (int64_t)(j0 + jj + 1) * D);
      float sc[STEPS];
      float m = -INFINITY;
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) part = fmaf(qv[e], (float)kr[s][e], part);
#pragma unroll
        for (int off = CH / 2; off > 0; off >>= 1) part += __shfl_xor(part, off);
        const int key = kw + KPS * s + kk;
        sc[s] = key < len ? part : -INFINITY;
        m = fmaxf(m, sc[s]);
      }
#pragma unroll
      for (int off = CH; off < 64; off <<= 1) m = fmaxf(m, __shfl_xor(m, off));
      const float base = m == -INFINITY ? 0.f : m;
      float lsum = 0.f;
      float o[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) o[e] = 0.f;
#pragma unroll
      for (int s = 0; s < STEPS; ++s) {
        const float p = fast_exp2(sc[s] - base);
        lsum += p;
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = fmaf(p, (float)vr[s][e], o[e]);
      }
#pragma unroll
      for (int off = CH; off < 64; off <<= 1) {
        lsum += __shfl_xor(lsum, off);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] += __shfl_xor(o[e], off);
      }
      if (l < CH) {
#pragma unroll
        for (int e = 0; e < 8; ++e) so[jj][wave][8 * c + e] = o[e];
      }
      if (l == 0) {
        sm[jj][wave] = m;
        sl[jj][wave] = lsum;
      }
    }
    __syncthreads();
    for (int idx = tid; idx < nj * D; idx += 256) {
      const int jj = idx / D, d = idx % D;
      const int bq = b * a.hq + h * a.g + j0 + jj;
      float M = -INFINITY;
      for (int w = 0; w < 4; ++w) M = fmaxf(M, sm[jj][w]);
      const float Mb = M == -INFINITY ? 0.f : M;
      float L = 0.f, O = 0.f;
      for (int w = 0; w < 4; ++w) {
        const float f = fast_exp2(sm[jj][w] - Mb);
        L += f * sl[jj][w];
        O += f * so[jj][w][d];
      }
      if (a.nsplit == 1) {
        a.out[(int64_t)bq * D + d] = (bf16)(L > 0.f ? O / L : 0.f);
      } else {
        float* pp = a.part + ((int64_t)bq * a.nsplit + split) * (D + 2);
        pp[2 + d] = O;
        if (d == 0) {
          pp[0] = M;
          pp[1] = L;
        }
      }
    }
  }
}

template <int D, bool GQA>
__global__ __launch_bounds__(256) void decode_split_kernel(const DecArgs a) {
  dec_split<D, GQA>(a, blockIdx.x, blockIdx.y);
}

// Both branches of a decode step in one launch: x < glo.nsplit are the global
// branch's splits, x == glo.nsplit the local window's single split (at most
// 256 keys), which writes its output row itself.
template <int D, bool GQA>
__global__ __launch_bounds__(256) void decode_dual_split_kernel(const DecArgs loc, const DecArgs glo) {
  if ((int)blockIdx.x == glo.nsplit) dec_split<D, GQA>(loc, 0, blockIdx.y);
  else dec_split<D, GQA>(glo, blockIdx.x, blockIdx.y);
}

// Merge the split partials of one (b, q-head) row: the splits' maxima and
// sums are reduced across the workgroup, then thread (group gi, column d)
// sums the rescaled partial outputs of splits gi, gi + G, ... with
// independent loads, and the groups are added through LDS.  The bf16 output
// row goes to out (global memory) or, with out == nullptr, to sout (LDS).
constexpr int kCombThreads = 1024;  // combine workgroup: enough column groups that each
                                    // thread's split loads go out together
template <int D>
__device__ __forceinline__ void dec_combine(const DecArgs& a, const int bq, bf16* out, bf16* sout) {
  constexpr int G = kCombThreads / D;  // split groups
  constexpr int NWV = kCombThreads / 64;
  const int b = bq / a.hq;
  const int tid = threadIdx.x, l = tid & 63, wave = tid >> 6;
  if (!dec_active(a, b)) {
    if (tid < D) (out ? out : sout)[tid] = (bf16)0.f;
    return;
  }
  const int len = a.lens[b];
  const int ns = min(a.nsplit, (len + kDecKeysPerWG - 1) / kDecKeysPerWG);
  const float* pp = a.part + (int64_t)bq * a.nsplit * (D + 2);
  __shared__ float red[NWV];
  __shared__ float so[G][D];
  float m = -INFINITY;
  for (int s = tid; s < ns; s += kCombThreads) m = fmaxf(m, pp[(int64_t)s * (D + 2)]);
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) m = fmaxf(m, __shfl_xor(m, off));
  if (l == 0) red[wave] = m;
  __syncthreads();
  float M = red[0];
#pragma unroll
  for (int w = 1; w < NWV; ++w) M = fmaxf(M, red[w]);
  const float Mb = M == -INFINITY ? 0.f : M;
  __syncthreads();
  float lsum = 0.f;
  for (int s = tid; s < ns; s += kCombThreads) {
    const float* ps = pp + (int64_t)s * (D + 2);
    lsum += fast_exp2(ps[0] - Mb) * ps[1];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) lsum += __shfl_xor(lsum, off);
  if (l == 0) red[wave] = lsum;
  const int gi = tid / D, d = tid % D;
  float o = 0.f;
#pragma unroll 8
  for (int s = gi; s < ns; s += G) {
    const float* ps = pp + (int64_t)s * (D + 2);
    o = fmaf(fast_exp2(ps[0] - Mb), ps[2 + d], o);
  }
  so[gi][d] = o;
  __syncthreads();
  if (tid < D) {
    float L = 0.f;
#pragma unroll
    for (int w = 0; w < NWV; ++w) L += red[w];
    float O = 0.f;
#pragma unroll
    for (int k = 0; k < G; ++k) O += so[k][tid];
    (out ? out : sout)[tid] = (bf16)(L > 0.f ? O / L : 0.f);
  }
}

template <int D>
__global__ __launch_bounds__(kCombThreads) void decode_combine_kernel(const DecArgs a) {
  dec_combine<D>(a, blockIdx.x, a.out + (int64_t)blockIdx.x * D, nullptr);
}

// The global branch's combine and the fused epilogue (context norms, gate
// mask, fusion; the same arithmetic as the epilogue kernel) of one (b, q-head)
// row: the global row stays in LDS, the local row comes from the dual split.
struct DecEpiArgs {
  const bf16* local;  // [B * HQ, D], the local branch's output
  const bf16* w_l;
  const bf16* w_g;
  bf16* out;          // [B * HQ, D]
  float eps;
};

template <int D>
__global__ __launch_bounds__(kCombThreads) void decode_combine_epi_kernel(const DecArgs glo, const DecEpiArgs e) {
  const int bq = blockIdx.x, b = bq / glo.hq;
  __shared__ bf16x8 sg[D / 8];
  bf16* sgb = reinterpret_cast<bf16*>(sg);
  if (glo.nsplit > 1) {
    dec_combine<D>(glo, bq, nullptr, sgb);
  } else if (threadIdx.x < D) {  // the single split wrote the row already
    sgb[threadIdx.x] = glo.out[(int64_t)bq * D + threadIdx.x];
  }
  __syncthreads();
  constexpr int LPR = D / 8;
  if (threadIdx.x < LPR) {
    const int c = threadIdx.x;
    const bf16x8 lv = *reinterpret_cast<const bf16x8*>(e.local + (int64_t)bq * D + 8 * c);
    const bf16x8 o = epi_fwd_chunk<D>(lv, sg[c], (float)glo.gate[b], load_thres(glo.thres, glo.thres_bf16), e.w_l,
                                      e.w_g, e.eps, c);
    *reinterpret_cast<bf16x8*>(e.out + (int64_t)bq * D + 8 * c) = o;
  }
}

// Write one new key/value row per (b, h) at position pos[b] (mod ring if > 0).
template <int D>
__global__ __launch_bounds__(256) void cache_append_kernel(const bf16* kn, const bf16* vn, bf16* kc, bf16* vc,
                                                           const int32_t* pos, int h, int64_t t_cap, int ring,
                                                           int64_t rows) {
  constexpr int CH = D / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t r = idx / CH;  // b * H + head
  const int c = idx % CH;
  if (r >= rows) return;
  const int b = (int)(r / h);
  int p = pos[b];
  if (ring > 0) p %= ring;
  const int64_t dst = (r * t_cap + p) * D + 8 * c;
  *reinterpret_cast<u32x4*>(kc + dst) = *reinterpret_cast<const u32x4*>(kn + r * D + 8 * c);
  *reinterpret_cast<u32x4*>(vc + dst) = *reinterpret_cast<const u32x4*>(vn + r * D + 8 * c);
}

}  // namespace logo

using namespace logo;

static int dec_nsplit(int max_len) { return (max_len + kDecKeysPerWG - 1) / kDecKeysPerWG; }

extern "C" size_t logo_decode_workspace_bytes(int batch, int hq, int d, int max_len) {
  const int ns = dec_nsplit(max_len > 0 ? max_len : 1);
  return (size_t)batch * hq * ns * (d + 2) * sizeof(float);
}

static DecArgs dec_args(const void* q, const void* k_cache, const void* v_cache, const int32_t* lens,
                        const void* gate, const void* thres, int thres_dtype, void* out, void* part, int batch,
                        int hq, int h, int64_t t_cap, int max_len, float scale) {
  DecArgs a{};
  a.q = static_cast<const bf16*>(q);
  a.k = static_cast<const bf16*>(k_cache);
  a.v = static_cast<const bf16*>(v_cache);
  a.lens = lens;
  a.gate = static_cast<const bf16*>(gate);
  a.thres = thres;
  a.thres_bf16 = thres_dtype == LOGO_DTYPE_BF16;
  a.out = static_cast<bf16*>(out);
  a.part = static_cast<float*>(part);
  a.batch = batch;
  a.hq = hq;
  a.h = h;
  a.g = hq / h;
  a.nsplit = dec_nsplit(max_len);
  a.t_cap = t_cap;
  a.scale_log2 = scale * 1.4426950408889634f;
  return a;
}

static int dec_check(int batch, int hq, int h, int d, int dtype, int thres_dtype) {
  LOGO_REQUIRE(batch >= 1 && h >= 1 && hq % h == 0, "bad batch / head counts");
  LOGO_REQUIRE(d == 64 || d == 128, "head dim %d unsupported (64 or 128)", d);
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  LOGO_REQUIRE(thres_dtype == LOGO_DTYPE_BF16 || thres_dtype == LOGO_DTYPE_F32, "thres_dtype must be bf16 or f32");
  return LOGO_OK;
}

extern "C" int logo_decode_attn(const void* q, const void* k_cache, const void* v_cache, const int32_t* lens,
                                const void* gate, const void* thres, int thres_dtype, void* out, void* workspace, int batch,
                                int hq, int h, int d, int64_t t_cap, int max_len, float scale, int dtype,
                                void* stream) {
  const int rc = dec_check(batch, hq, h, d, dtype, thres_dtype);
  if (rc != LOGO_OK) return rc;
  LOGO_REQUIRE(max_len >= 1 && max_len <= t_cap, "max_len must be in [1, t_cap]");
  LOGO_REQUIRE(q && k_cache && v_cache && lens && out && workspace, "null pointer argument");
  LOGO_REQUIRE(gate == nullptr || thres != nullptr, "gate needs thres");
  const DecArgs a = dec_args(q, k_cache, v_cache, lens, gate, thres, thres_dtype, out, workspace, batch, hq, h, t_cap,
                             max_len, scale);
  hipStream_t st = as_stream(stream);
  dim3 grid(a.nsplit, batch * h);  // one workgroup per (split, kv row): the GQA group shares its keys
  const bool gqa = a.g > 1;
  if (d == 128)
    hipLaunchKernelGGL((gqa ? decode_split_kernel<128, true> : decode_split_kernel<128, false>), grid, dim3(256), 0,
                       st, a);
  else
    hipLaunchKernelGGL((gqa ? decode_split_kernel<64, true> : decode_split_kernel<64, false>), grid, dim3(256), 0,
                       st, a);
  LOGO_LAUNCH_CHECK("decode_split_kernel");
  if (a.nsplit > 1) {  // a single split wrote the output already
    if (d == 128)
      hipLaunchKernelGGL(decode_combine_kernel<128>, dim3(batch * hq), dim3(kCombThreads), 0, st, a);
    else
      hipLaunchKernelGGL(decode_combine_kernel<64>, dim3(batch * hq), dim3(kCombThreads), 0, st, a);
    LOGO_LAUNCH_CHECK("decode_combine_kernel");
  }
  return LOGO_OK;
}

// Workspace of logo_decode_attn_fused: the global branch's split partials,
// then the local and the global bf16 rows, each region 256-byte aligned.
static size_t dec_align(size_t x) { return (x + 255) & ~(size_t)255; }

extern "C" size_t logo_decode_fused_workspace_bytes(int batch, int hq, int d, int max_len_global) {
  const size_t rows = (size_t)batch * hq * d * sizeof(bf16);
  return dec_align(logo_decode_workspace_bytes(batch, hq, d, max_len_global)) + 2 * dec_align(rows);
}

extern "C" int logo_decode_attn_fused(const void* q_local, const void* k_local, const void* v_local,
                                      const int32_t* lens_local, int64_t t_cap_local, int max_len_local,
                                      const void* q_global, const void* k_global, const void* v_global,
                                      const int32_t* lens_global, int64_t t_cap_global, int max_len_global,
                                      const void* gate, const void* thres, int thres_dtype, const void* w_local,
                                      const void* w_global, float eps, void* out, void* workspace, int batch, int hq,
                                      int h, int d, float scale, int dtype, void* stream) {
  const int rc = dec_check(batch, hq, h, d, dtype, thres_dtype);
  if (rc != LOGO_OK) return rc;
  LOGO_REQUIRE(max_len_local >= 1 && max_len_local <= t_cap_local && max_len_local <= kDecKeysPerWG,
               "max_len_local must be in [1, min(t_cap_local, %d)]", kDecKeysPerWG);
  LOGO_REQUIRE(max_len_global >= 1 && max_len_global <= t_cap_global, "max_len_global must be in [1, t_cap_global]");
  LOGO_REQUIRE(q_local && k_local && v_local && lens_local && q_global && k_global && v_global && lens_global && gate &&
                   thres && w_local && w_global && out && workspace,
               "null pointer argument");
  char* ws = static_cast<char*>(workspace);
  const size_t part_bytes = dec_align(logo_decode_workspace_bytes(batch, hq, d, max_len_global));
  const size_t row_bytes = dec_align((size_t)batch * hq * d * sizeof(bf16));
  void* lrow = ws + part_bytes;
  void* grow = ws + part_bytes + row_bytes;
  const DecArgs loc = dec_args(q_local, k_local, v_local, lens_local, nullptr, nullptr, thres_dtype, lrow, nullptr,
                               batch, hq, h, t_cap_local, max_len_local, scale);
  const DecArgs glo = dec_args(q_global, k_global, v_global, lens_global, gate, thres, thres_dtype, grow, ws, batch, hq,
                               h, t_cap_global, max_len_global, scale);
  DecEpiArgs e{};
  e.local = static_cast<const bf16*>(lrow);
  e.w_l = static_cast<const bf16*>(w_local);
  e.w_g = static_cast<const bf16*>(w_global);
  e.out = static_cast<bf16*>(out);
  e.eps = eps;
  hipStream_t st = as_stream(stream);
  const dim3 grid(glo.nsplit + 1, batch * h);
  if (d == 128) {
    hipLaunchKernelGGL((glo.g > 1 ? decode_dual_split_kernel<128, true> : decode_dual_split_kernel<128, false>),
                       grid, dim3(256), 0, st, loc, glo);
    LOGO_LAUNCH_CHECK("decode_dual_split_kernel");
    hipLaunchKernelGGL(decode_combine_epi_kernel<128>, dim3(batch * hq), dim3(kCombThreads), 0, st, glo, e);
  } else {
    hipLaunchKernelGGL((glo.g > 1 ? decode_dual_split_kernel<64, true> : decode_dual_split_kernel<64, false>),
                       grid, dim3(256), 0, st, loc, glo);
    LOGO_LAUNCH_CHECK("decode_dual_split_kernel");
    hipLaunchKernelGGL(decode_combine_epi_kernel<64>, dim3(batch * hq), dim3(kCombThreads), 0, st, glo, e);
  }
  LOGO_LAUNCH_CHECK("decode_combine_epi_kernel");
  return LOGO_OK;
}

extern "C" int logo_cache_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                                 const int32_t* pos, int batch, int h, int d, int64_t t_cap, int ring,
                                 int dtype, void* stream) {
  LOGO_REQUIRE(batch >= 1 && h >= 1, "bad batch / head counts");
  LOGO_REQUIRE(d == 64 || d == 128, "head dim %d unsupported (64 or 128)", d);
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16, "only bf16 tensors are supported");
  LOGO_REQUIRE(ring >= 0 && (ring == 0 || ring <= t_cap), "ring must be 0 or <= t_cap");
  LOGO_REQUIRE(k_new && v_new && k_cache && v_cache && pos, "null pointer argument");
  const int64_t rows = (int64_t)batch * h;
  const int64_t total = rows * (d / 8);
  const unsigned nblk = (unsigned)((total + 255) / 256);
  hipStream_t st = as_stream(stream);
  if (d == 128)
    hipLaunchKernelGGL(cache_append_kernel<128>, dim3(nblk), dim3(256), 0, st, static_cast<const bf16*>(k_new),
                       static_cast<const bf16*>(v_new), static_cast<bf16*>(k_cache), static_cast<bf16*>(v_cache),
                       pos, h, t_cap, ring, rows);
  else
    hipLaunchKernelGGL(cache_append_kernel<64>, dim3(nblk), dim3(256), 0, st, static_cast<const bf16*>(k_new),
                       static_cast<const bf16*>(v_new), static_cast<bf16*>(k_cache), static_cast<bf16*>(v_cache),
                       pos, h, t_cap, ring, rows);
  LOGO_LAUNCH_CHECK("cache_append_kernel");
  return LOGO_OK;
}
