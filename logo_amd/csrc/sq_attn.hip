// Query-sparse causal attention, forward and backward, for gfx950.
//
// Semantics follow logo/ops/selected_full_attn.py: selected ("compacted")
// query rows attend causally to every key of their own packed segment up to
// their real position (:33-121); the backward recomputes P from the stored
// log2-domain LSE (:141-228 dq, :231-337 dk/dv) with delta = rowsum(o * dO)
// (:124-138); dk/dv of a GQA group are summed over its query heads (:444-445).
// One difference in rounding: in sparse mode the query rows are pre-scaled
// and rounded once, q' = bf16(-scale log2(e) q) (the forward's registers and
// the backward's q_sel copies), where the reference scales the fp32 product
// (:93).  That adds up to 2^-9 relative error per q element; measured against
// float64 with scores up to +-43 in log2 units, o and the gradients stay
// within 1.0-1.5x of the error of the reference's own rounding chain.
// Differences in structure:
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
#include "sq_attn.hpp"

#include <algorithm>
#include <cstdlib>
#include <mutex>

namespace logo {

// ---------------------------------------------------------------------------
// Backward preprocess: delta = rowsum(o * dO) per compacted row (fp32); in
// sparse mode also the compacted copies q_sel = round(-scale log2(e) q) and
// do_sel = -dO, which let the dq and dk/dv kernels start their S and dP
// accumulators from lse and delta.
// ---------------------------------------------------------------------------
// Each thread takes one 16-byte chunk of kDeltaRows rows (RPB apart), all its
// loads issued before any arithmetic, so a workgroup keeps 2x the bytes in
// flight of a row-per-thread layout (2 rows: 31 us at the T = 32K, r = 0.25
// workload; 4 rows 33 us, 8 rows 35 us, as fewer workgroups share the rows).
constexpr int kDeltaRows = 2;

template <typename EL, int D, bool SPARSE>
__global__ __launch_bounds__(256) void sq_delta_kernel(const AttnArgs a) {
  using E8 = typename Elem<EL>::x8;
  constexpr int LPR = D / 8;          // lanes per row
  constexpr int RPB = 256 / LPR;      // rows per workgroup and step
  constexpr int R = kDeltaRows;
  const int hq = blockIdx.y;
  const int lane_sel = a.lanes > 1 ? hq : 0;
  const int32_t* meta = a.meta + (int64_t)lane_sel * a.meta_stride;
  const int sq = meta[0];
  const int r0 = blockIdx.x * RPB * R + threadIdx.x / LPR;
  const int c = threadIdx.x % LPR;
  if (blockIdx.x * RPB * R >= sq) return;
  int64_t off[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int r = r0 + k * RPB;
    const int64_t t = r < sq ? (SPARSE ? a.q_idx[(int64_t)lane_sel * a.n + r] : (int64_t)r) : 0;
    off[k] = (t * a.hq + hq) * D + 8 * c;
  }
  E8 ov[R], dv[R], qv[R];
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const bool ok = r0 + k * RPB < sq;
    ov[k] = ok ? *reinterpret_cast<const E8*>(a.o + off[k]) : E8{};
    dv[k] = ok ? *reinterpret_cast<const E8*>(a.dout + off[k]) : E8{};
    if (SPARSE) qv[k] = ok ? *reinterpret_cast<const E8*>(a.q + off[k]) : E8{};
  }
#pragma unroll
  for (int k = 0; k < R; ++k) {
    const int r = r0 + k * RPB;
    float acc = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc = fmaf((float)ov[k][e], (float)dv[k][e], acc);
    if (SPARSE && r < sq) {
      // the copies the dq and dk/dv kernels stream: q_sel = round(-c q) with
      // c = scale * log2(e), do_sel = -dO (exact)
      const int64_t soff = ((int64_t)hq * a.n + r) * D + 8 * c;
      E8 dn;
#pragma unroll
      for (int e = 0; e < 8; ++e) dn[e] = -dv[k][e];
      *reinterpret_cast<E8*>(a.do_sel + soff) = dn;
      *reinterpret_cast<E8*>(a.q_sel + soff) = scale8(qv[k], -a.scale_log2);
    }
#pragma unroll
    for (int o = LPR / 2; o > 0; o >>= 1) acc += __shfl_xor(acc, o);
    if (r < sq && c == 0) a.delta[(int64_t)hq * a.n + r] = acc;
  }
}

template <typename EL, int D, bool SPARSE>
static int launch_delta(const AttnArgs& a, hipStream_t st) {
  constexpr int RPB = 256 / (D / 8) * kDeltaRows;
  dim3 grid((unsigned)((a.n + RPB - 1) / RPB), a.hq);
  hipLaunchKernelGGL((sq_delta_kernel<EL, D, SPARSE>), grid, dim3(256), 0, st, a);
  LOGO_LAUNCH_CHECK("sq_delta_kernel");
  return LOGO_OK;
}

int sq_launch_delta(const AttnArgs& a, hipStream_t st, int d, bool sparse, bool half) {
  if (half) return d == 128 ? launch_delta<f16, 128, true>(a, st) : launch_delta<f16, 64, true>(a, st);
  return d == 128 ? (sparse ? launch_delta<bf16, 128, true>(a, st) : launch_delta<bf16, 128, false>(a, st))
                  : (sparse ? launch_delta<bf16, 64, true>(a, st) : launch_delta<bf16, 64, false>(a, st));
}

int device_cus() {
  static std::mutex mu;
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    cache[dev] = cus;
  }
  return cache[dev];
}

static int check_common(int64_t n, int nseq, int hq, int h, int d, int v_dim, int lanes, int dtype,
                        bool sparse, int window) {
  LOGO_REQUIRE(n > 0 && n < ((int64_t)1 << 31), "n_tokens out of range: %lld", (long long)n);
  LOGO_REQUIRE(nseq >= 1, "nseq must be >= 1");
  LOGO_REQUIRE(h >= 1 && hq >= h && hq % h == 0, "HQ (%d) must be a multiple of H (%d)", hq, h);
  LOGO_REQUIRE(d == 64 || d == 128 || d == 256, "head dim %d unsupported (64, 128 or 256)", d);
  // every kernel strides q, k, v, o and the gradients by the one head dim d
  LOGO_REQUIRE(v_dim == d, "value head dim %d must equal the key head dim %d", v_dim, d);
  LOGO_REQUIRE(lanes == 1 || lanes == hq, "lanes must be 1 or HQ");
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16 || dtype == LOGO_DTYPE_F16 || dtype == LOGO_DTYPE_F32,
               "dtype %d unsupported (bf16, fp16 or fp32)", dtype);
  // fp16 and fp32 kernels exist for the query-sparse global branch (no window)
  LOGO_REQUIRE(dtype == LOGO_DTYPE_BF16 || (sparse && window < 0),
               "fp16 and fp32 are supported on the query-sparse path without a window only");
  return LOGO_OK;
}

// Compacted rows a head has in flight in one round of fwd / dq workgroups
// (CUs * 256 / HQ for every form of those kernels), which sets their key walk
// order (QTile::desc); the environment variable LOGO_SQ_DESC=0 keeps every
// walk ascending (A/B timing).
static int walk_round_rows(int hq) {
  const char* env = std::getenv("LOGO_SQ_DESC");
  if (env != nullptr && env[0] == '0') return 0;
  return device_cus() * 256 / hq;
}

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
  a.round_rows = window < 0 ? walk_round_rows(hq) : 0;
  return a;
}

}  // namespace logo

using namespace logo;

extern "C" size_t logo_sq_workspace_bytes(int64_t n_tokens, int nseq, int hq, int d) {
  if (n_tokens <= 0 || nseq < 1 || hq < 1 || (d != 64 && d != 128)) return 0;
  const bool paired = nseq == 1 && n_tokens >= kFwdPairMinTokens;
  const int cap_f = split_cap_for(hq, paired ? 1 : 2), cap_d = split_cap_for(hq, 2);
  const size_t fwd = cap_f >= 2 ? (size_t)hq * 2 * cap_f * fwd_part_floats(d, paired ? 8 : 4) : 0;
  const size_t dq = cap_d >= 2 ? (size_t)hq * 2 * cap_d * dq_part_floats(d) : 0;
  const size_t part = std::max(fwd, dq) * sizeof(float);
  return part == 0 ? 0 : split_cnt_bytes() + part;
}

extern "C" size_t logo_sq_workspace_counter_bytes(void) { return split_cnt_bytes(); }

extern "C" int logo_sq_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                           const int64_t* q_idx, const int32_t* pos, const int32_t* meta,
                           const int32_t* cu, int64_t n_tokens, int nseq, int hq, int h, int d,
                           int v_dim, int lanes, float scale, int window, int dtype, void* workspace,
                           size_t workspace_bytes, void* stream) {
  int rc = check_common(n_tokens, nseq, hq, h, d, v_dim, lanes, dtype, q_idx != nullptr, window);
  if (rc != LOGO_OK) return rc;
  LOGO_REQUIRE(q && k && v && o && lse && meta && cu, "null pointer argument");
  LOGO_REQUIRE((q_idx == nullptr) == (pos == nullptr), "q_idx and pos must both be set or both be null");
  AttnArgs a = make_args(q, k, v, q_idx, pos, meta, cu, n_tokens, nseq, hq, h, lanes, scale, window);
  a.o = static_cast<bf16*>(o);
  a.lse = lse;
  a.ws = workspace;
  a.ws_bytes = workspace ? workspace_bytes : 0;
  const bool sparse = q_idx != nullptr;
  const bool win = window >= 0;
  if (gen_applies(d, dtype)) return gen_launch_fwd(a, as_stream(stream), d, dtype, sparse);
  return sq_launch_fwd(a, as_stream(stream), d, sparse, win, dtype == LOGO_DTYPE_F16);
}

extern "C" int logo_sq_generic(int d, int dtype) { return gen_applies(d, dtype) ? 1 : 0; }

#define LOGO_BWD_PARAMS                                                                        \
  const void *q, const void *k, const void *v, const void *o, const void *dout, const float *lse, \
      float *delta, void *q_sel, void *do_sel, void *dq, void *dk, void *dv, const int64_t *q_idx, \
      const int32_t *pos, const int32_t *meta, const int32_t *cu, int64_t n_tokens, int nseq,      \
      int hq, int h, int d, int v_dim, int lanes, float scale, int window, int dtype, void *workspace, \
      size_t workspace_bytes, void *stream

#define LOGO_BWD_ARGS                                                                             \
  q, k, v, o, dout, lse, delta, q_sel, do_sel, dq, dk, dv, q_idx, pos, meta, cu, n_tokens, nseq, hq, \
      h, d, v_dim, lanes, scale, window, dtype, workspace, workspace_bytes, stream

static int bwd_entry(LOGO_BWD_PARAMS, int phase) {
  int rc = check_common(n_tokens, nseq, hq, h, d, v_dim, lanes, dtype, q_idx != nullptr, window);
  if (rc != LOGO_OK) return rc;
  LOGO_REQUIRE(q && k && v && o && dout && lse && delta && meta && cu, "null pointer argument");
  // each phase needs the outputs it writes: dq (phase 1), dk / dv (phase 2)
  LOGO_REQUIRE((phase == 0 || phase == 2 || dq) && (phase == 0 || phase == 1 || (dk && dv)),
               "null gradient pointer");
  LOGO_REQUIRE((q_idx == nullptr) == (pos == nullptr), "q_idx and pos must both be set or both be null");
  const bool generic = gen_applies(d, dtype);
  LOGO_REQUIRE(q_idx == nullptr || generic || (q_sel && do_sel),
               "sparse backward needs q_sel and do_sel workspaces");
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
  a.ws = workspace;
  a.ws_bytes = workspace ? workspace_bytes : 0;
  const bool sparse = q_idx != nullptr;
  const bool win = window >= 0;
  const bool half = dtype == LOGO_DTYPE_F16;
  hipStream_t st = as_stream(stream);
  if (generic) {  // the generic kernels read q and dO in place (no compacted copies)
    if (phase < 0 || phase == 0) {
      rc = gen_launch_delta(a, st, d, dtype, sparse);
      if (rc != LOGO_OK) return rc;
    }
    if (phase < 0 || phase == 1 || phase == 3) {
      rc = gen_launch_dq(a, st, d, dtype, sparse);
      if (rc != LOGO_OK) return rc;
    }
    if (phase < 0 || phase == 2 || phase == 3) rc = gen_launch_dkv(a, st, d, dtype, sparse);
    return rc;
  }
  if (phase < 0 || phase == 0) {
    rc = sq_launch_delta(a, st, d, sparse, half);
    if (rc != LOGO_OK) return rc;
  }
  // dq, dk and dv together: one pass where the fused window kernel applies
  if ((phase < 0 || phase == 3) && swa_bwd_applies(a, sparse, half)) return swa_launch_bwd(a, st, d);
  if (phase < 0 || phase == 1 || phase == 3) {
    rc = sq_launch_dq(a, st, d, sparse, win, half);
    if (rc != LOGO_OK) return rc;
  }
  if (phase < 0 || phase == 2 || phase == 3) rc = sq_launch_dkv(a, st, d, sparse, win, half);
  return rc;
}

extern "C" int logo_sq_bwd(LOGO_BWD_PARAMS) { return bwd_entry(LOGO_BWD_ARGS, -1); }
extern "C" int logo_sq_bwd_delta(LOGO_BWD_PARAMS) { return bwd_entry(LOGO_BWD_ARGS, 0); }
extern "C" int logo_sq_bwd_dq(LOGO_BWD_PARAMS) { return bwd_entry(LOGO_BWD_ARGS, 1); }
extern "C" int logo_sq_bwd_dkv(LOGO_BWD_PARAMS) { return bwd_entry(LOGO_BWD_ARGS, 2); }
extern "C" int logo_sq_bwd_dqkv(LOGO_BWD_PARAMS) { return bwd_entry(LOGO_BWD_ARGS, 3); }

