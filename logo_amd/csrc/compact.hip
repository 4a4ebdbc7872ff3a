// Row compaction for query-sparse attention (gfx950).
//
// Bit-exact restatement of build_selection (logo/ops/common.py:71-107):
// q_idx = nonzero(selection) in ascending order, pos = q_idx - cu[seg],
// cu_q = exclusive prefix of per-sequence counts; plus the tile prefixes the
// attention kernels use to map a workgroup to (sequence, block), which replace
// prepare_chunk_indices (logo/ops/common.py:110-124) and its host sync.
//
// Short inputs (at most 4096 tokens) and per-head selections of at most 65536
// tokens a lane take one launch with one 1024-thread workgroup per lane
// (compact_small): per-64-token ballots and counts in LDS, the counts'
// exclusive scan, a pass over the kept ballots that writes q_idx / pos, cu_q
// from the group prefixes, then the tile prefixes (one lane of 32768 tokens
// takes it in about 24 us, no faster than the three launches below, which
// spread it over the GPU).
// Everything else takes three launches, none of them synchronising with the
// host:
//   count    : per 4096-token chunk and lane, popcount of wave ballots
//   scatter  : chunk prefix + wave prefix (LDS) + mbcnt rank -> q_idx, pos
//              (and zeros in entries [Sq, N), one per unselected token)
//   finalize : Sq, cu_q by binary search over q_idx, tile prefixes by block scan
#include <mutex>

#include "capi.hpp"
#include "common.hpp"

namespace logo {

constexpr int kChunk = 4096;  // tokens per workgroup: 4 waves x 16 ballots x 64 lanes

__device__ __forceinline__ bool sel_on(const uint8_t* sel, int64_t n, int lanes, int lane, int64_t t) {
  return t < n && sel[t * lanes + lane] != 0;
}

__global__ __launch_bounds__(256) void compact_count(const uint8_t* __restrict__ sel, int64_t n,
                                                     int lanes, int32_t* __restrict__ counts,
                                                     int nchunk) {
  const int lane = blockIdx.y;
  const int64_t base = (int64_t)blockIdx.x * kChunk;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;
  int cnt = 0;
#pragma unroll 4
  for (int s = 0; s < 16; ++s) {
    const int64_t t = base + w * 1024 + s * 64 + l;
    cnt += __popcll(__ballot(sel_on(sel, n, lanes, lane, t)));
  }
  __shared__ int wc[4];
  if (l == 0) wc[w] = cnt;
  __syncthreads();
  if (threadIdx.x == 0) counts[lane * nchunk + blockIdx.x] = wc[0] + wc[1] + wc[2] + wc[3];
}

__device__ __forceinline__ int block_sum(int v, int* red) {
  // 256-thread sum through LDS; red holds 4 ints.
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  const int w = threadIdx.x >> 6;
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

__global__ __launch_bounds__(256) void compact_scatter(const uint8_t* __restrict__ sel, int64_t n,
                                                       int lanes, const int32_t* __restrict__ cu,
                                                       int nseq, const int32_t* __restrict__ counts,
                                                       int nchunk, int64_t* __restrict__ q_idx,
                                                       int32_t* __restrict__ pos) {
  __shared__ int red[4];
  __shared__ int wc[4];
  const int lane = blockIdx.y;
  const int chunk = blockIdx.x;
  const int w = threadIdx.x >> 6, l = threadIdx.x & 63;

  int part = 0, all = 0;
  for (int c = threadIdx.x; c < nchunk; c += 256) {
    const int v = counts[lane * nchunk + c];
    all += v;
    if (c < chunk) part += v;
  }
  const int prefix = block_sum(part, red);
  const int sq = block_sum(all, red);

  const int64_t base = (int64_t)chunk * kChunk + w * 1024;
  uint64_t masks[16];
  int cnt = 0;
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    masks[s] = __ballot(sel_on(sel, n, lanes, lane, base + s * 64 + l));
    cnt += __popcll(masks[s]);
  }
  if (l == 0) wc[w] = cnt;
  __syncthreads();
  int run = prefix;
  for (int i = 0; i < w; ++i) run += wc[i];

  int64_t* qi = q_idx + (int64_t)lane * n;
  int32_t* ps = pos + (int64_t)lane * n;
  const uint64_t below = (l == 0) ? 0ull : (~0ull >> (64 - l));
#pragma unroll
  for (int s = 0; s < 16; ++s) {
    const uint64_t m = masks[s];
    const int rank = run + __popcll(m & below);  // selected tokens before t
    const int64_t t = base + s * 64 + l;
    if ((m >> l) & 1ull) {
      const int sg = seg_of(cu, nseq, t);
      qi[rank] = t;
      ps[rank] = (int32_t)(t - cu[sg]);
    } else if (t < n) {
      // entries [Sq, N) are zero: unselected token t fills entry Sq + (the
      // unselected tokens before it)
      qi[sq + (t - rank)] = 0;
      ps[sq + (t - rank)] = 0;
    }
    run += __popcll(m);
  }
}

// Exclusive scan over NT threads; returns this thread's exclusive prefix and
// writes the block total to *total.  Each wave scans its 64 values with
// shuffles, the wave totals go through LDS (buf[0, NT / 64)), and every
// thread adds those of the waves before its own: three barriers in all (the
// first keeps a previous call's readers of buf ahead of the new writes).
template <int NT = 256>
__device__ __forceinline__ int block_exscan(int v, int* buf, int* total) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int x = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(x, off);
    if (lane >= off) x += y;
  }
  __syncthreads();
  if (lane == 63) buf[w] = x;
  __syncthreads();
  int before = 0, all = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const int t = buf[i];
    before += i < w ? t : 0;
    all += t;
  }
  *total = all;
  __syncthreads();
  return before + x - v;
}

// Tile prefixes per sequence (query tiles of LOGO_BQ compacted rows, key
// tiles of LOGO_BKV tokens) and the header, from cu_q already in meta
// (written by this workgroup before its last barrier).
template <int NT>
__device__ __forceinline__ void meta_tiles(const int32_t* __restrict__ cu, int nseq, int64_t n, int sq,
                                           int32_t* __restrict__ m, int* buf) {
  int32_t* cu_q = m + kMetaHdr;
  int32_t* cu_tq = cu_q + (nseq + 1);
  int32_t* cu_tk = cu_tq + (nseq + 1);
  int carry_q = 0, carry_k = 0;
  for (int s0 = 0; s0 < nseq; s0 += NT) {
    const int s = s0 + threadIdx.x;
    int bq = 0, bk = 0;
    if (s < nseq) {
      const int cq = cu_q[s + 1] - cu_q[s];
      const int ck = cu[s + 1] - cu[s];
      bq = (cq + LOGO_BQ - 1) / LOGO_BQ;
      bk = (ck + LOGO_BKV - 1) / LOGO_BKV;
    }
    int tq, tk;
    const int eq = block_exscan<NT>(bq, buf, &tq);
    const int ek = block_exscan<NT>(bk, buf, &tk);
    if (s < nseq) {
      cu_tq[s] = carry_q + eq;
      cu_tk[s] = carry_k + ek;
    }
    carry_q += tq;
    carry_k += tk;
  }
  if (threadIdx.x == 0) {
    cu_tq[nseq] = carry_q;
    cu_tk[nseq] = carry_k;
    m[0] = sq;
    m[1] = carry_q;
    m[2] = carry_k;
    m[3] = (int)n;
    m[4] = nseq;
    m[5] = m[6] = m[7] = 0;
  }
}

// The whole compaction of one lane of at most kSmallMax tokens in one
// workgroup (same outputs as count + scatter + finalize).
constexpr int kSmallMax = 65536;
constexpr int kSmallThreads = 1024;
__global__ __launch_bounds__(kSmallThreads) void compact_small(const uint8_t* __restrict__ sel, int64_t n,
                                                               int lanes, const int32_t* __restrict__ cu,
                                                               int nseq, int64_t* __restrict__ q_idx,
                                                               int32_t* __restrict__ pos,
                                                               int32_t* __restrict__ meta) {
  constexpr int NW = kSmallThreads / 64;
  __shared__ int gpre[kSmallMax / 64];  // per 64-token group: its count, then its exclusive prefix
  __shared__ uint64_t gmask[kSmallMax / 64];  // per 64-token group: its selection ballot
  __shared__ int buf[NW];
  const int lane = blockIdx.x;
  const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
  const int G = (int)((n + 63) >> 6);
#pragma unroll 8
  for (int gi = w; gi < G; gi += NW) {
    const uint64_t msk = __ballot(sel_on(sel, n, lanes, lane, (int64_t)gi * 64 + l));
    if (l == 0) {
      gpre[gi] = __popcll(msk);
      gmask[gi] = msk;
    }
  }
  __syncthreads();
  int sq;
  {
    // G <= kSmallThreads groups: thread tid scans group tid
    const int v = tid < G ? gpre[tid] : 0;
    const int e = block_exscan<kSmallThreads>(v, buf, &sq);
    if (tid < G) gpre[tid] = e;
  }
  __syncthreads();
  int64_t* qi = q_idx + (int64_t)lane * n;
  int32_t* ps = pos + (int64_t)lane * n;
  const uint64_t below = (l == 0) ? 0ull : (~0ull >> (64 - l));
#pragma unroll 8
  for (int gi = w; gi < G; gi += NW) {
    const int64_t t = (int64_t)gi * 64 + l;
    const uint64_t msk = gmask[gi];
    const int rank = gpre[gi] + __popcll(msk & below);  // selected tokens before t
    if ((msk >> l) & 1ull) {
      const int sg = seg_of(cu, nseq, t);
      qi[rank] = t;
      ps[rank] = (int32_t)(t - cu[sg]);
    } else if (t < n) {
      qi[sq + (t - rank)] = 0;  // entries [Sq, N) are zero, as in compact_scatter
      ps[sq + (t - rank)] = 0;
    }
  }
  // cu_q[s] = selected tokens before token cu[s]: the prefix of its group plus
  // the selected tokens of the group below it
  int32_t* m = meta + (int64_t)lane * LOGO_META_STRIDE(nseq);
  for (int s = w; s <= nseq; s += NW) {
    const int64_t key = cu[s];
    const int gi = (int)(key >> 6);
    int v;
    if (gi >= G) {
      v = sq;
    } else {
      const uint64_t msk = gmask[gi];
      const int r = (int)(key & 63);
      v = gpre[gi] + __popcll(r == 0 ? 0ull : (msk & (~0ull >> (64 - r))));
    }
    if (l == 0) m[kMetaHdr + s] = v;
  }
  __syncthreads();
  meta_tiles<kSmallThreads>(cu, nseq, n, sq, m, buf);
}

// One workgroup per lane.  dense != 0: cu_q = cu and Sq = n (no q_idx).
__global__ __launch_bounds__(256) void compact_finalize(const int32_t* __restrict__ cu, int nseq,
                                                        int64_t n, const int32_t* __restrict__ counts,
                                                        int nchunk, const int64_t* __restrict__ q_idx,
                                                        int32_t* __restrict__ meta, int dense) {
  __shared__ int red[4];
  __shared__ int buf[256];
  const int lane = blockIdx.x;
  const int stride = LOGO_META_STRIDE(nseq);
  int32_t* m = meta + (int64_t)lane * stride;
  int32_t* cu_q = m + kMetaHdr;

  int sq;
  if (dense) {
    sq = (int)n;
  } else {
    int part = 0;
    for (int c = threadIdx.x; c < nchunk; c += 256) part += counts[lane * nchunk + c];
    sq = block_sum(part, red);
  }
  const int64_t* qi = q_idx + (int64_t)lane * n;
  for (int s = threadIdx.x; s <= nseq; s += 256) {
    int v;
    if (dense) {
      v = cu[s];
    } else {
      // cu_q[s] = number of selected rows before token cu[s].
      int lo = 0, hi = sq;
      const int64_t key = cu[s];
      while (lo < hi) {
        int mid = (lo + hi) >> 1;
        if (qi[mid] < key) lo = mid + 1; else hi = mid;
      }
      v = lo;
    }
    cu_q[s] = v;
  }
  __syncthreads();
  meta_tiles<256>(cu, nseq, n, sq, m, buf);
}

// prepare_chunk_indices for an arbitrary chunk size (parity helper).
__global__ __launch_bounds__(256) void chunk_prefix_kernel(const int32_t* __restrict__ cu, int nseq,
                                                           int chunk, int32_t* __restrict__ prefix,
                                                           int32_t* __restrict__ count) {
  __shared__ int buf[256];
  int carry = 0;
  for (int s0 = 0; s0 < nseq; s0 += 256) {
    const int s = s0 + threadIdx.x;
    const int b = s < nseq ? (cu[s + 1] - cu[s] + chunk - 1) / chunk : 0;
    int tot;
    const int e = block_exscan(b, buf, &tot);
    if (s < nseq) prefix[s] = carry + e;
    carry += tot;
  }
  if (threadIdx.x == 0) {
    prefix[nseq] = carry;
    *count = carry;
  }
}

__global__ __launch_bounds__(256) void chunk_list_kernel(const int32_t* __restrict__ prefix, int nseq,
                                                         int32_t* __restrict__ out, int64_t max_tiles) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int nt = prefix[nseq];
  if (t >= nt || t >= max_tiles) return;
  const int s = seg_of(prefix, nseq, t);
  out[2 * t] = s;
  out[2 * t + 1] = (int32_t)(t - prefix[s]);
}

__global__ __launch_bounds__(256) void q_start_kernel(const int32_t* __restrict__ pos,
                                                      const int32_t* __restrict__ cu_q,
                                                      const int32_t* __restrict__ chunks,
                                                      const int32_t* __restrict__ count,
                                                      int64_t max_tiles, int block,
                                                      int32_t* __restrict__ out) {
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (t >= *count || t >= max_tiles) return;
  const int s = chunks[2 * t], j = chunks[2 * t + 1];
  const int lo = cu_q[s], hi = cu_q[s + 1];
  const int first = lower_bound_i32(pos, lo, hi, j * block);
  out[t] = (first - lo) / block;
}

}  // namespace logo

using namespace logo;

extern "C" size_t logo_compact_workspace_bytes(int64_t n_tokens, int lanes) {
  const int64_t nchunk = (n_tokens + kChunk - 1) / kChunk;
  return (size_t)(nchunk > 0 ? nchunk : 1) * (size_t)(lanes > 0 ? lanes : 1) * sizeof(int32_t);
}

static int compact_launch(const uint8_t* selection, int64_t n_tokens, int lanes, const int32_t* cu,
                          int nseq, int64_t* q_idx, int32_t* pos, int32_t* meta, int32_t* counts,
                          hipStream_t st) {
  if (n_tokens <= 4096 || (lanes >= 4 && n_tokens <= kSmallMax)) {
    hipLaunchKernelGGL(compact_small, dim3(lanes), dim3(kSmallThreads), 0, st, selection, n_tokens, lanes, cu, nseq,
                       q_idx, pos, meta);
    LOGO_LAUNCH_CHECK("compact_small");
    return LOGO_OK;
  }
  const int nchunk = (int)((n_tokens + kChunk - 1) / kChunk);
  if (nchunk > 0) {
    dim3 grid(nchunk, lanes);
    hipLaunchKernelGGL(compact_count, grid, dim3(256), 0, st, selection, n_tokens, lanes, counts, nchunk);
    LOGO_LAUNCH_CHECK("compact_count");
    hipLaunchKernelGGL(compact_scatter, grid, dim3(256), 0, st, selection, n_tokens, lanes, cu, nseq,
                       counts, nchunk, q_idx, pos);
    LOGO_LAUNCH_CHECK("compact_scatter");
  }
  hipLaunchKernelGGL(compact_finalize, dim3(lanes), dim3(256), 0, st, cu, nseq, n_tokens, counts,
                     nchunk, q_idx, meta, 0);
  LOGO_LAUNCH_CHECK("compact_finalize");
  return LOGO_OK;
}

#define LOGO_COMPACT_CHECK_ARGS()                                                               \
  LOGO_REQUIRE(n_tokens >= 0 && n_tokens < (int64_t)1 << 31, "n_tokens out of range: %lld",      \
               (long long)n_tokens);                                                            \
  LOGO_REQUIRE(lanes >= 1 && nseq >= 1, "lanes (%d) and nseq (%d) must be >= 1", lanes, nseq);  \
  LOGO_REQUIRE(cu && meta, "null pointer argument");                                            \
  LOGO_REQUIRE(n_tokens == 0 || (selection && q_idx && pos), "null selection/q_idx/pos")

extern "C" int logo_compact(const uint8_t* selection, int64_t n_tokens, int lanes, const int32_t* cu,
                            int nseq, int64_t* q_idx, int32_t* pos, int32_t* meta, void* workspace,
                            void* stream) {
  LOGO_COMPACT_CHECK_ARGS();
  LOGO_REQUIRE(workspace, "null workspace");
  return compact_launch(selection, n_tokens, lanes, cu, nseq, q_idx, pos, meta,
                        static_cast<int32_t*>(workspace), as_stream(stream));
}

// ---------------------------------------------------------------------------
// logo_compact without a workspace argument, for callers that cannot
// allocate.  The per-chunk counts live in a file-scope device array; each
// device holds its own copy at its own address, found once per device with
// hipGetSymbolAddress (the array's name in host code is only a stand-in for
// the symbol).  The counts are written in full by compact_count before any
// kernel reads them, so nothing needs clearing between calls.
// ---------------------------------------------------------------------------
namespace logo {
constexpr int kMaxDevices = 64;
static __device__ __align__(256) int32_t scratch[LOGO_COMPACT_SCRATCH_INTS];
static std::mutex g_scratch_mu;
static int32_t* g_scratch_ptr[kMaxDevices];  // per device, set on the first call there

// The scratch address on the current device (found on first use there).
static int scratch_on_current_device(int32_t** out) {
  int dev = -1;
  LOGO_HIP_CHECK(hipGetDevice(&dev));
  LOGO_REQUIRE(dev >= 0 && dev < kMaxDevices, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    LOGO_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    LOGO_REQUIRE(p != nullptr, "no device address for the compaction scratch");
    g_scratch_ptr[dev] = static_cast<int32_t*>(p);
  }
  *out = g_scratch_ptr[dev];
  return LOGO_OK;
}
}  // namespace logo

extern "C" int logo_compact_noalloc(const uint8_t* selection, int64_t n_tokens, int lanes,
                                    const int32_t* cu, int nseq, int64_t* q_idx, int32_t* pos,
                                    int32_t* meta, void* stream) {
  LOGO_COMPACT_CHECK_ARGS();
  const int64_t need = (int64_t)lanes * ((n_tokens + kChunk - 1) / kChunk);
  LOGO_REQUIRE(need <= LOGO_COMPACT_SCRATCH_INTS,
               "logo_compact_noalloc: %lld tokens x %d lanes need %lld scratch counts, above its fixed %d "
               "(use logo_compact with a workspace)",
               (long long)n_tokens, lanes, (long long)need, LOGO_COMPACT_SCRATCH_INTS);
  int32_t* counts = nullptr;
  const int rc = scratch_on_current_device(&counts);
  if (rc != LOGO_OK) return rc;
  return compact_launch(selection, n_tokens, lanes, cu, nseq, q_idx, pos, meta, counts, as_stream(stream));
}

extern "C" int logo_dense_meta(const int32_t* cu, int nseq, int64_t n_tokens, int32_t* meta,
                               void* stream) {
  LOGO_REQUIRE(n_tokens >= 0 && n_tokens < (int64_t)1 << 31, "n_tokens out of range");
  LOGO_REQUIRE(nseq >= 1 && cu && meta, "bad arguments");
  hipLaunchKernelGGL(compact_finalize, dim3(1), dim3(256), 0, as_stream(stream), cu, nseq, n_tokens,
                     (const int32_t*)nullptr, 0, (const int64_t*)nullptr, meta, 1);
  LOGO_LAUNCH_CHECK("compact_finalize(dense)");
  return LOGO_OK;
}

extern "C" int logo_chunk_indices(const int32_t* cu, int nseq, int chunk, int32_t* out,
                                  int64_t max_tiles, int32_t* count, int32_t* workspace,
                                  void* stream) {
  LOGO_REQUIRE(nseq >= 1 && chunk >= 1 && cu && out && count && workspace, "bad arguments");
  hipStream_t st = as_stream(stream);
  hipLaunchKernelGGL(chunk_prefix_kernel, dim3(1), dim3(256), 0, st, cu, nseq, chunk, workspace, count);
  LOGO_LAUNCH_CHECK("chunk_prefix_kernel");
  if (max_tiles > 0) {
    const int64_t nb = (max_tiles + 255) / 256;
    hipLaunchKernelGGL(chunk_list_kernel, dim3((unsigned)nb), dim3(256), 0, st, workspace, nseq, out,
                       max_tiles);
    LOGO_LAUNCH_CHECK("chunk_list_kernel");
  }
  return LOGO_OK;
}

extern "C" int logo_q_start_blk(const int32_t* pos, const int32_t* cu_q, const int32_t* chunks,
                                const int32_t* count, int64_t max_tiles, int block, int32_t* out,
                                void* stream) {
  LOGO_REQUIRE(block >= 1 && cu_q && chunks && count && out, "bad arguments");
  if (max_tiles <= 0) return LOGO_OK;
  const int64_t nb = (max_tiles + 255) / 256;
  hipLaunchKernelGGL(q_start_kernel, dim3((unsigned)nb), dim3(256), 0, as_stream(stream), pos, cu_q,
                     chunks, count, max_tiles, block, out);
  LOGO_LAUNCH_CHECK("q_start_kernel");
  return LOGO_OK;
}
