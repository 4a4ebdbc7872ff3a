// Shared declarations of the query-sparse attention kernels (gfx950): the
// argument block, the compacted-row views, the per-workgroup query tile and
// the per-phase launch entry points (one translation unit per kernel).
#pragma once

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
  // Key-range split of the fwd / dq tiles (no window): a tile is cut into up
  // to kMaxSplit pieces when its head has few tiles; each piece writes an fp32
  // partial to `part`, and the last piece of a tile to arrive (per-tile counter
  // in `cnt`, zero on entry, left zero) combines them.  split_cap: the pieces
  // per head to aim for (0: no split); the workspace holds 2 split_cap per
  // head.
  float* part;
  int* cnt;
  int split_cap;
  // the caller's workspace (host side only: the launchers carve part / cnt
  // from it when it is large enough for their kernel's split_cap)
  void* ws;
  size_t ws_bytes;
  // Key walk order of the fwd / dq tiles (no window): compacted rows a head
  // has in flight at once (one round of its workgroups, the same for the
  // 8-wave and 4-wave forward and for dq: CUs * 256 / HQ); 0 keeps every tile
  // ascending.  See QTile::desc.
  int round_rows;
};

constexpr int kMaxSplit = 4;

// Single long sequences take 8-wave forward workgroups of two query tiles,
// which share each K / V tile copy between 256 rows (half the copy traffic
// and issue per row); packed or short inputs keep 4-wave single-tile
// workgroups, which give more workgroups where rows are few.
constexpr int64_t kFwdPairMinTokens = 16384;

// Compute units of the current device (cached per device).
int device_cus();

// Pieces per head a split kernel aims for: two rounds of the workgroups the
// device holds at once (wgs_per_cu per CU), shared by the heads.
inline int split_cap_for(int hq, int wgs_per_cu) { return 2 * device_cus() * wgs_per_cu / hq; }

// Pieces per tile for a head with nt tiles: none while its tiles alone fill
// more than three quarters of the target (LPT order balances those), else
// enough to reach the target, at most kMaxSplit.  nt * nper < 1.75 cap.
__host__ __device__ inline int split_pieces(int nt, int cap) {
  if (cap <= 0 || nt <= 0 || 4 * nt > 3 * cap) return 1;
  const int n = (cap + nt - 1) / nt;
  return n < kMaxSplit ? n : kMaxSplit;
}

// Bytes of the arrival counters at the start of the workspace (2 split_cap
// per head: at most 2 workgroups per CU x 2 rounds x 2), 256-byte aligned.
inline size_t split_cnt_bytes() { return ((size_t)8 * device_cus() * sizeof(int) + 255) & ~(size_t)255; }

// fp32 partial floats per piece: forward (NW waves: O [DT][16][64] plus m / l
// [64] per wave), dq (2 waves x 2 row blocks x DT x 16 x 64).
inline size_t fwd_part_floats(int d, int nw) { return (size_t)nw * ((size_t)(d / 32) * 16 * 64 + 64); }
inline size_t dq_part_floats(int d) { return (size_t)2 * 2 * (d / 32) * 16 * 64; }

// Enables the split in `a` when its workspace holds the counters and
// 2 split_cap pieces per head of `floats` each; otherwise split_cap = 0.
inline void split_setup(AttnArgs& a, int wgs_per_cu, size_t floats) {
  const int cap = split_cap_for(a.hq, wgs_per_cu);
  const size_t need = split_cnt_bytes() + (size_t)a.hq * 2 * cap * floats * sizeof(float);
  if (cap >= 2 && a.ws != nullptr && a.ws_bytes >= need) {
    a.cnt = static_cast<int*>(a.ws);
    a.part = reinterpret_cast<float*>(static_cast<char*>(a.ws) + split_cnt_bytes());
    a.split_cap = cap;
  } else {
    a.split_cap = 0;
  }
}

// Cross-workgroup exchange of the split partials.  The L2s of the XCDs are
// not coherent with each other, so partials are stored and loaded with
// agent-scope atomics (sc1: through to the coherent level, no L2 flush or
// invalidate), and the stores are complete (vmcnt(0)) before the counter
// increment that publishes them.
//
// Why this is ordered on gfx950 without release / acquire fences (an
// agent-scope release or acquire compiles to a write-back or invalidate of
// the whole XCD L2 here, which is what the sc1 accesses avoid):
//  1. Each partial store is an agent-scope atomic store, so it writes
//     through the XCD's L2 to the memory-side coherence point.  On gfx9
//     parts vmcnt counts stores as well as loads, and a store is counted
//     until the coherence point acknowledges it: after wait_stores()
//     (s_waitcnt vmcnt(0)) this wave's partials are visible to any
//     agent-scope load.
//  2. __syncthreads() after that wait means every wave of the piece has
//     completed its stores before thread 0 issues the counter add, and the
//     add is itself an agent-scope atomic performed at the coherence point.
//     So when a piece's add returns npieces - 1, every other piece's
//     partials were complete before their adds.
//  3. The last piece's loads of the partials cannot issue early: they are
//     control-dependent on the add's returned value, which reaches the
//     other waves only through the LDS flag after a second __syncthreads();
//     and they are agent-scope atomic loads, which read at the coherence
//     point rather than from a possibly stale L2 line.
// What the compiler must keep: the "memory" clobber of wait_stores() and the
// barriers (both stop it from moving the stores below, or the loads above,
// these points), and the agent scope on every store and load of `part`.
// Plain loads or stores of the partials, or loads moved above the flag
// test, would break the exchange silently.
__device__ __forceinline__ void st_agent(float* p, float v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_agent(const float* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void wait_stores() { asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); }

// Arrival of one piece at its tile's counter (after its partial is stored and
// complete on every wave).  Returns true in the last piece to arrive, which
// also resets the counter; flag: 4 bytes of LDS no longer in use.
__device__ __forceinline__ bool split_arrive(int* cnt, int npieces, int* flag) {
  wait_stores();
  __syncthreads();
  if (threadIdx.x == 0) {
    const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const bool last = old == npieces - 1;
    if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    *flag = last;
  }
  __syncthreads();
  return *flag != 0;
}

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
  // the lane's rows in all segments (cu_q[nseq]) and its tiles (paired
  // tiles counted once); set before init can return false
  int q_end, ntile;
  bool wave_active, valid;
  int64_t t;
  RowView<SPARSE> rv;
  // key-range split: rank = trank * nper + piece; nsplit pieces of this tile
  // exist (nsplit <= nper; 1: no split)
  int rank, trank, piece, nper, nsplit;
  // Walk the key tiles from the last to the first.  The tiles of a head run
  // heaviest first; those of the first round start together at key 0 and
  // walk in step, so each K / V tile is fetched into the XCD's L2 once for
  // all of them.  Tiles of later rounds start one by one, as earlier tiles of
  // different lengths finish: walking up from key 0 each would fetch its
  // keys alone.  Walking down instead, a tile that starts later starts lower,
  // where the tiles that started before it have just arrived, so the tiles of
  // a round converge and share their K / V again.  Rounds alternate: odd
  // rounds walk down.  Rounds are counted in pairs of 128-row tiles (the
  // 8-wave forward's tiles), so the 4-wave forward and dq tiles of the same
  // rows walk the same way (the forms stay bit-identical).
  bool desc;

  // rpw: compacted rows per wave (32 or 64); r / t / p / valid describe the
  // lane's row in the wave's first 32-row block (row_at gives the others).
  // paired: the workgroup takes two consecutive kBQ-row tiles (a single
  // segment only, nseq == 1, so both tiles share one key range).
  // splittable: the tile's keys [kv_lo, kv_hi) may be cut into pieces (a
  // split_cap > 0, no window); the piece's own range replaces them.
  __device__ __forceinline__ bool init(const AttnArgs& a, int wave, int i, bool window, int rpw = 32,
                                       bool paired = false, bool splittable = false) {
    xcd_remap(blockIdx.x, a.hq, rank, hq);
    lane_sel = a.lanes > 1 ? hq : 0;
    const int32_t* meta = a.meta + (int64_t)lane_sel * a.meta_stride;
    const int nt = paired ? (meta[1] + 1) >> 1 : meta[1];
    const int32_t* cu_q = meta + kMetaHdr;
    const int32_t* cu_tq = cu_q + (a.nseq + 1);
    q_end = cu_q[a.nseq];
    ntile = nt;
    nper = splittable ? split_pieces(nt, a.split_cap) : 1;
    if (rank >= nt * nper) return false;
    trank = rank / nper;
    piece = rank - trank * nper;
    {
      // rank of the tile's pair of 128-row tiles, heaviest first
      const int pr = paired ? trank : ((nt + 1) >> 1) - 1 - ((nt - 1 - trank) >> 1);
      const int pairs_per_round = a.round_rows >> 8;
      desc = !window && pairs_per_round > 0 && ((pr / pairs_per_round) & 1);
    }
    const int tile = nt - 1 - trank;  // heaviest (latest) blocks first
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
    nsplit = 1;
    if (nper > 1) {
      // 64-key-aligned chunks; nsplit <= nper pieces, none empty
      const int span = kv_hi - kv_lo;
      const int chunk = (((span + nper - 1) / nper) + 63) & ~63;
      nsplit = (span + chunk - 1) / chunk;
      if (piece >= nsplit) return false;
      kv_lo += piece * chunk;
      kv_hi = min(kv_hi, kv_lo + chunk);
    }
    return true;
  }
};

// Sparse mode: the rows of tokens that no compacted row writes are zero in
// the outputs o and dq ([N, HQ, D]), written by the fwd and dq kernels
// themselves instead of a separate fill of the whole tensor.  The lane's rows
// ascend by token over all its segments (t_0 < t_1 < ... < t_{q_end-1}), so
// the tokens to zero are the gaps (t_{r-1}, t_r) for 0 < r < q_end, the
// leading range [0, t_0) and the trailing range (t_{q_end-1}, N).  Gap r goes
// to the tile that holds row r (the tiles partition [0, q_end)); the leading
// and trailing ranges are cut into one slice per tile, so that a long
// unselected span is spread over the grid instead of one workgroup.  A lane
// without rows has no tiles: then every workgroup of the head's grid zeroes
// one slice of [0, N).  Only piece 0 of a split tile zeroes.  The forward
// also zeroes the head's lse rows [q_end, N), the same way.
// 16 bytes a lane, CHR = D / 8 lanes a row; tokens fit in int (N < 2^31).
template <int D>
__device__ __forceinline__ void zero_row(bf16* out, int tok, int hq_n, int hq, int c16) {
  // non-temporal: no kernel of the op reads the zero rows back (repeated forward
  // calls at T = 32K -1.5%; the fwd + bwd step unchanged within the noise)
  st_nt(reinterpret_cast<u32x4*>(out + ((int64_t)tok * hq_n + hq) * D + 8 * c16), u32x4{0u, 0u, 0u, 0u});
}

// Slice k of nslice of [lo, hi): ceil((hi - lo) / nslice) items a slice.
__device__ __forceinline__ void slice_of(int lo, int hi, int k, int nslice, int& s0, int& s1) {
  const int span = hi - lo;
  const int chunk = (span + nslice - 1) / nslice;
  s0 = lo + (int)min((int64_t)chunk * k, (int64_t)span);
  s1 = lo + (int)min((int64_t)chunk * (k + 1), (int64_t)span);
}

// Slice k of nslice of the tokens [lo, hi), by the workgroup's nthreads.
template <int D>
__device__ __forceinline__ void zero_slice(bf16* out, int hq_n, int hq, int lo, int hi, int k, int nslice,
                                           int nthreads) {
  constexpr int CHR = D / 8;
  const int grp = threadIdx.x / CHR, ngrp = nthreads / CHR, c16 = threadIdx.x % CHR;
  int s0, s1;
  slice_of(lo, hi, k, nslice, s0, s1);
  for (int u = s0 + grp; u < s1; u += ngrp) zero_row<D>(out, u, hq_n, hq, c16);
}

// Gaps of the tile's rows [r0, r_end): wave w takes rows r0 + 64 w + lane,
// stepping 64 nw; each gap found (ballot) is zeroed by the wave's 64 / CHR
// row groups in turn.
template <int D>
__device__ __forceinline__ void zero_gaps(bf16* out, int hq_n, int hq, const RowView<true>& rv, int r0, int r_end,
                                          int nthreads) {
  constexpr int CHR = D / 8, GPW = 64 / CHR;
  const int l = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = nthreads >> 6;
  const int grp = l / CHR, c16 = l % CHR;
  for (int rb = r0 + 64 * wave; rb < r_end; rb += 64 * nw) {
    const int r = rb + l;
    int lo = 0, hi = 0;
    if (r > 0 && r < r_end) {
      lo = (int)rv.token(r - 1) + 1;
      hi = (int)rv.token(r);
    }
    unsigned long long m = __ballot(hi > lo);
    while (m != 0) {
      const int j = __builtin_ctzll(m);
      m &= m - 1;
      const int a0 = __shfl(lo, j), a1 = __shfl(hi, j);
      for (int u = a0 + grp; u < a1; u += GPW) zero_row<D>(out, u, hq_n, hq, c16);
    }
  }
}

// Slice k of nslice of the floats [lo, hi) of p (the forward's lse rows past
// the lane's q_end, which no tile writes, are zero too).
__device__ __forceinline__ void zero_slice_f32(float* p, int lo, int hi, int k, int nslice, int nthreads) {
  int s0, s1;
  slice_of(lo, hi, k, nslice, s0, s1);
  for (int u = s0 + threadIdx.x; u < s1; u += nthreads) p[u] = 0.f;
}

// Everything a tile's workgroup (piece 0) zeroes: its rows' gaps and its
// slices (tile rank k of ntile) of the leading and trailing ranges; lse
// (forward only, else nullptr): its slice of the head's rows [q_end, N).
template <int D>
__device__ __forceinline__ void zero_unselected(const AttnArgs& a, bf16* out, float* lse, const QTile<true>& qt,
                                                int nthreads) {
  const int n = (int)a.n;
  zero_gaps<D>(out, a.hq, qt.hq, qt.rv, qt.r0, qt.r_end, nthreads);
  const int first = (int)qt.rv.token(0), last = (int)qt.rv.token(qt.q_end - 1);
  zero_slice<D>(out, a.hq, qt.hq, 0, first, qt.trank, qt.ntile, nthreads);
  zero_slice<D>(out, a.hq, qt.hq, last + 1, n, qt.trank, qt.ntile, nthreads);
  if (lse != nullptr) zero_slice_f32(lse + (int64_t)qt.hq * n, qt.q_end, n, qt.trank, qt.ntile, nthreads);
}

// A workgroup for which init returned false: in a lane without rows, its
// slice (grid rank of the head's gridDim.x / HQ) of every token (and of the
// head's lse rows).
template <int D>
__device__ __forceinline__ void zero_empty_lane(const AttnArgs& a, bf16* out, float* lse, const QTile<true>& qt,
                                                int nthreads) {
  if (qt.q_end != 0) return;
  const int n = (int)a.n, nslice = (int)(gridDim.x / a.hq);
  zero_slice<D>(out, a.hq, qt.hq, 0, n, qt.rank, nslice, nthreads);
  if (lse != nullptr) zero_slice_f32(lse + (int64_t)qt.hq * n, 0, n, qt.rank, nslice, nthreads);
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <int B>
using BufTag = std::integral_constant<int, B>;

template <typename K>
static inline hipError_t allow_smem(K kernel, size_t bytes) {
  return hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
}

// Per-phase launchers (d = 64 or 128; sparse: compacted rows; window: a
// sliding window is set; half: fp16 elements, sparse without a window only,
// else bf16).  Each returns LOGO_OK or an error code.
int sq_launch_fwd(const AttnArgs& a, hipStream_t st, int d, bool sparse, bool window, bool half);
int sq_launch_delta(const AttnArgs& a, hipStream_t st, int d, bool sparse, bool half);
int sq_launch_dq(const AttnArgs& a, hipStream_t st, int d, bool sparse, bool window, bool half);
int sq_launch_dkv(const AttnArgs& a, hipStream_t st, int d, bool sparse, bool window, bool half);

// The dedicated sliding-window forward (dense rows, window <= 128, bf16):
// whether it serves a call, and its launcher.
bool swa_fwd_applies(const AttnArgs& a, bool sparse, bool half);
int swa_launch_fwd(const AttnArgs& a, hipStream_t st, int d);
// The fused sliding-window backward (dq, dk and dv in one pass; dense rows,
// window <= 128, HQ == H, bf16; delta computed beforehand).
bool swa_bwd_applies(const AttnArgs& a, bool sparse, bool half);
int swa_launch_bwd(const AttnArgs& a, hipStream_t st, int d);

// The generic kernels (gen_attn.hip): head dim 256 (bf16, and fp16 in sparse
// mode) and fp32 in sparse mode (d = 64, 128, 256).  gen_applies: whether a
// call with head dim d and element type dtype runs on them (the entry points
// route such calls there before any tuned kernel).
bool gen_applies(int d, int dtype);
int gen_launch_fwd(const AttnArgs& a, hipStream_t st, int d, int dtype, bool sparse);
int gen_launch_delta(const AttnArgs& a, hipStream_t st, int d, int dtype, bool sparse);
int gen_launch_dq(const AttnArgs& a, hipStream_t st, int d, int dtype, bool sparse);
int gen_launch_dkv(const AttnArgs& a, hipStream_t st, int d, int dtype, bool sparse);

// Calls FN<D, SPARSE, WINDOW>(a, st) for the runtime (d, sparse, window).
#define LOGO_DISPATCH(FN, a, st, d, sparse, window)                                                  \
  ((d) == 128 ? ((sparse) ? ((window) ? FN<128, true, true>(a, st) : FN<128, true, false>(a, st))   \
                          : ((window) ? FN<128, false, true>(a, st) : FN<128, false, false>(a, st))) \
              : ((sparse) ? ((window) ? FN<64, true, true>(a, st) : FN<64, true, false>(a, st))     \
                          : ((window) ? FN<64, false, true>(a, st) : FN<64, false, false>(a, st))))

}  // namespace logo
