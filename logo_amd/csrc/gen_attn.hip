// Generic query-sparse / dense causal attention, forward and backward, for
// the calls the tuned kernels do not cover:
//   * head dims in (128, 256] (run at D = 256, K and V zero-padded by the
//     caller): the reference takes any K <= 256 in one block
//     (logo/ops/selected_full_attn.py:344, logo/ops/common.py:127-168);
//   * fp32 q, k, v on the query-sparse path, computed in fp32 throughout:
//     the reference's dots run in the input dtype, P kept in fp32 for PV
//     (logo/ops/selected_full_attn.py:93-99) and the output in v's dtype
//     (:349).
// Semantics are those of the tuned kernels (sq_fwd.hip, sq_dq.hip,
// sq_dkv.hip): selected (compacted) rows attend causally within their packed
// segment, optionally within a sliding window (keys [p - w, p]); the
// backward recomputes P from the log2-domain lse with delta = rowsum(o * dO)
// (:124-138); dk / dv of a GQA group are summed over its query heads
// (:444-445); rows of unselected tokens are zero in o and dq.
//
// Unlike the tuned kernels these compute the scores the reference's way:
// S = q.k accumulated in fp32 from the unscaled inputs, then scaled by
// scale * log2(e) in fp32 (:93); P and dS are rounded to the input type
// before their products (:99, :206-207), which for fp32 means no rounding.
//
// Structure (simple, one LDS buffer, no software pipelining):
//   16x16 MFMA tiles with a 16-deep k step for every element type:
//   v_mfma_f32_16x16x16_bf16 / _f16 (one per k step) and
//   v_mfma_f32_16x16x4_f32 (four per k step).  Lane l = 16 G + i holds
//   elements 4G .. 4G+3 of the k step for row / column i of an operand, and
//   accumulator items j = 0..3 of row 4G + j, column i, so an accumulator
//   read row-major is directly the B operand of the next product (its rows
//   are the k index).
//   fwd, dq : 4 waves x 16 compacted rows = 64 rows per workgroup (half of a
//             128-row tile of the compaction's tile list); q (and dO) in
//             registers; 32-key K / V tiles through LDS; S^T = K Q^T, so each
//             lane's query is its column i and row statistics reduce over
//             the four lanes i, i+16, i+32, i+48.
//   dk/dv   : 4 waves x 16 keys = 64 keys per workgroup (half of a 128-key
//             tile); K, V and the dK^T / dV^T accumulators in registers; the
//             query heads of the GQA group looped inside; 16-row steps of
//             q, dO, lse, delta and positions through LDS.
// Tiles in LDS are row-major with 16-byte chunks XOR-swizzled by row, so the
// row reads of 16 consecutive rows fall in distinct banks.
#include "sq_attn.hpp"

namespace logo {
namespace gen {

// ---------------------------------------------------------------------------
// MFMA per element type: 16x16 output tiles, a k step of KSTEP, NE = KSTEP / 4
// elements per lane (lane group G holds elements NE G .. NE G + NE - 1 of the
// step for both A and B, so they pair up whatever order the unit sums in)
// ---------------------------------------------------------------------------
template <typename T>
struct Mma;
template <>
struct Mma<bf16> {
  static constexpr int KSTEP = 32, NE = 8;
  using Op = bf16x8;
  using V4 = bf16x4;
  __device__ __forceinline__ static f32x4 mma(Op a, Op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mma<f16> {
  static constexpr int KSTEP = 32, NE = 8;
  using Op = f16x8;
  using V4 = f16x4;
  __device__ __forceinline__ static f32x4 mma(Op a, Op b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Mma<float> {
  static constexpr int KSTEP = 16, NE = 4;
  using Op = f32x4;
  using V4 = f32x4;
  // k slot G of instruction s is element s of lane group G: k = 4 G + s
  __device__ __forceinline__ static f32x4 mma(Op a, Op b, f32x4 c) {
#pragma unroll
    for (int s = 0; s < 4; ++s) c = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], b[s], c, 0, 0, 0);
    return c;
  }
};

// The k-step operand made of accumulators: items of the 16-row accumulator
// tiles acc[0 .. KSTEP / 16), as the input type (the reference's
// `.to(q.dtype)` before a product; exact for fp32).  Element e of lane group
// G is row 16 (e / 4) + 4 G + e % 4 of the step, the order GTile::trk reads
// the matching operand in.
template <typename T>
__device__ __forceinline__ typename Mma<T>::Op to_opk(const f32x4* acc) {
  typename Mma<T>::Op r;
#pragma unroll
  for (int e = 0; e < Mma<T>::NE; ++e) r[e] = (T)acc[e >> 2][e & 3];
  return r;
}

// ---------------------------------------------------------------------------
// LDS tiles: rows of D elements of T, 16-byte chunks XOR-swizzled by row
// ---------------------------------------------------------------------------
template <typename T, int D>
struct GTile {
  using M = Mma<T>;
  using Op = typename M::Op;
  static constexpr int RB = D * (int)sizeof(T);  // bytes per row (>= 128)
  static constexpr int CH = RB / 16;             // 16-byte chunks per row
  static constexpr int SW = CH < 16 ? CH - 1 : 15;
  __device__ __forceinline__ static int off(int r, int ch) { return r * RB + 16 * (ch ^ (r & SW)); }
  // byte offset of element (r, c); 16 bytes from c a multiple of 16 / sizeof(T) stay in one chunk
  __device__ __forceinline__ static int eoff(int r, int c) {
    const int b = c * (int)sizeof(T);
    return off(r, b >> 4) + (b & 15);
  }
  // Row operand: lane (i, G) gets elements KSTEP ks + NE G .. + NE - 1 of row
  // r (one 16-byte chunk).  (LDS reads go through the restrict wrappers of
  // common.hpp, so the compiler does not make them wait for the next tile's
  // copy in flight.)
  __device__ __forceinline__ static Op row(const char* t, int r, int ks, int G) {
    return lds_load(reinterpret_cast<const Op*>(t + eoff(r, M::KSTEP * ks + M::NE * G)));
  }
  // Transposed operand of the k step whose rows start at rb: lane l = 16 G + i
  // gets column c0 + i of rows rb + 16 (e / 4) + 4 G + e % 4 (c0 a multiple
  // of 16), the order to_opk builds the other operand in.
  __device__ __forceinline__ static Op trk(const char* t, int rb, int c0, int l) {
    const int G = l >> 4, i = l & 15;
    if constexpr (sizeof(T) == 2) {
      // ds_read_b64_tr_b16: lane 16G + 4a + b receives element b of the
      // 8-byte chunks addressed by lanes 16G + a + 4e (e = 0..3) as its
      // elements e.  Lane 16G + j addresses row r0 + 4G + j/4 at columns
      // c0 + 4(j%4) .. + 3, so lane 16G + i receives rows r0 + 4G + e of
      // column c0 + i; two reads cover the step's two 16-row blocks.
      using L4 = std::conditional_t<Elem<T>::kHalf, lds_hf16x4, lds_bf16x4>;
      const int r = rb + 4 * G + (i >> 2), c = c0 + 4 * (i & 3);
      const auto lo = ds_read_tr((const L4*)(t + eoff(r, c)));
      const auto hi = ds_read_tr((const L4*)(t + eoff(r + 16, c)));
      return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    } else {
      Op v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = lds_load(reinterpret_cast<const T*>(t + eoff(rb + 4 * G + e, c0 + i)));
      return v;
    }
  }
  // Rows [0, R) global -> LDS by NT threads with buffer_load ... lds (no
  // registers): row r is read from row0 + min(r, last) * stride (elements);
  // each wave instruction fills 1 KB of the tile, lane j the 16 bytes at
  // offset 16 j, which belong to physical chunk pc of row r and so to
  // logical chunk pc ^ swz(r).  The buffer's extent ends at row `last`, so
  // no lane reads past it.  The caller waits (vmcnt) and barriers before
  // the tile is read.
  template <int R, int NT>
  __device__ __forceinline__ static void dma(char* t, const T* row0, int stride, int last) {
    static_assert(R * RB % 1024 == 0, "tiles are whole 1 KB blocks");
    constexpr int LOADS = R * RB / 1024, NWV = NT / 64;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), j = threadIdx.x & 63;
    const int extent = (last * stride) * (int)sizeof(T) + RB;
    const auto rsrc = __builtin_amdgcn_make_buffer_rsrc(const_cast<T*>(row0), (short)0, extent, kBufRsrcWord3);
#pragma unroll
    for (int k = 0; k < (LOADS + NWV - 1) / NWV; ++k) {
      const int b = wave + NWV * k;
      if (LOADS % NWV == 0 || b < LOADS) {
        const int o = 1024 * b + 16 * j;
        const int r = o / RB, pc = (o % RB) >> 4;
        const uint32_t voff = (uint32_t)(min(r, last) * stride * (int)sizeof(T) + 16 * (pc ^ (r & SW)));
        buf_load_lds16(rsrc, reinterpret_cast<bf16*>(t + 1024 * b), voff);
      }
    }
  }
  // Register staging of gathered rows (the dk/dv kernel's q and dO rows):
  // thread tid holds chunks tid, tid + NT, ... of rows [0, R).
  template <int R, int NT>
  struct Staged {
    static constexpr int N = (R * CH + NT - 1) / NT;
    u32x4 v[N];
    template <typename F>
    __device__ __forceinline__ void fetch(F rowptr) {
#pragma unroll
      for (int k = 0; k < N; ++k) {
        const int c = threadIdx.x + NT * k;
        if (R * CH % NT == 0 || c < R * CH)
          v[k] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(rowptr(c / CH)) + 16 * (c % CH));
      }
    }
    __device__ __forceinline__ void stash(char* t) const {
#pragma unroll
      for (int k = 0; k < N; ++k) {
        const int c = threadIdx.x + NT * k;
        if (R * CH % NT == 0 || c < R * CH) *reinterpret_cast<u32x4*>(t + off(c / CH, c % CH)) = v[k];
      }
    }
  };
};

// Sum / max over the four lanes of a query column (i, i+16, i+32, i+48).
__device__ __forceinline__ float col_sum(float x) {
  x += __shfl_xor(x, 16);
  return x + __shfl_xor(x, 32);
}
__device__ __forceinline__ float col_max(float x) {
  x = fmaxf(x, __shfl_xor(x, 16));
  return fmaxf(x, __shfl_xor(x, 32));
}

constexpr int kRowsWG = 64;  // compacted rows per fwd / dq workgroup (half a kBQ tile)
constexpr int kKT = 32;      // keys per K / V tile (fwd, dq)
constexpr int kKeysWG = 64;  // keys per dk/dv workgroup (half a kBKV tile)

// The rows of a fwd / dq workgroup: half (sub) of a kBQ-row tile of the
// compaction's tile list.  qt describes the whole tile for the zero-row
// helpers shared with the tuned kernels (rank: the workgroup's rank in its
// head's grid; trank / ntile: the tile's).
template <bool SPARSE>
struct GenRows {
  QTile<SPARSE> qt;
  int r0, r_end, sub;

  __device__ __forceinline__ bool init(const AttnArgs& a) {
    int rank, hq;
    xcd_remap(blockIdx.x, a.hq, rank, hq);
    qt.rank = rank;
    qt.hq = hq;
    qt.lane_sel = a.lanes > 1 ? hq : 0;
    const int32_t* meta = a.meta + (int64_t)qt.lane_sel * a.meta_stride;
    const int nt = meta[1];
    const int32_t* cu_q = meta + kMetaHdr;
    const int32_t* cu_tq = cu_q + (a.nseq + 1);
    qt.q_end = cu_q[a.nseq];
    qt.ntile = nt;
    qt.trank = rank >> 1;
    sub = rank & 1;
    if (qt.trank >= nt) return false;
    const int tile = nt - 1 - qt.trank;  // latest (heaviest) tiles first
    qt.s = seg_of(cu_tq, a.nseq, tile);
    qt.r0 = cu_q[qt.s] + (tile - cu_tq[qt.s]) * kBQ;
    qt.r_end = min(qt.r0 + kBQ, cu_q[qt.s + 1]);
    qt.bos = a.cu[qt.s];
    qt.seqlen = a.cu[qt.s + 1] - qt.bos;
    qt.h = hq / a.g;
    qt.rv = row_view<SPARSE>(a, qt.lane_sel, qt.bos);
    r0 = qt.r0 + kRowsWG * sub;
    r_end = min(r0 + kRowsWG, qt.r_end);
    return true;
  }
};

// Zero rows of unselected tokens (sparse mode), by the first half of each
// tile, and the whole-lane slices of a lane without rows.  Rows are DB
// bf16-sized units long (D * sizeof(T) / 2).
template <typename T, int D, bool SPARSE>
__device__ __forceinline__ void gen_zero(const AttnArgs& a, void* out, float* lse, const GenRows<SPARSE>& gr,
                                         bool have_rows) {
  if constexpr (SPARSE) {
    constexpr int DB = D * (int)sizeof(T) / 2;
    bf16* o = static_cast<bf16*>(out);
    if (!have_rows) zero_empty_lane<DB>(a, o, lse, gr.qt, 256);
    else if (gr.sub == 0) zero_unselected<DB>(a, o, lse, gr.qt, 256);
  }
}

// ---------------------------------------------------------------------------
// Forward
// ---------------------------------------------------------------------------
template <typename T, int D, bool SPARSE>
__global__ __launch_bounds__(256) void gen_fwd_kernel(const AttnArgs a) {
  using M = Mma<T>;
  using Op = typename M::Op;
  using TL = GTile<T, D>;
  constexpr int KS = D / M::KSTEP;      // k steps over the head dim
  constexpr int DT = D / 16;            // 16-column blocks of O
  constexpr int KK = kKT / M::KSTEP;    // k steps over a tile's keys
  // two stages of [K tile][V tile], 32 keys each
  auto tK = [](int b) { return logo_smem + b * 2 * kKT * TL::RB; };
  auto tV = [](int b) { return logo_smem + (b * 2 + 1) * kKT * TL::RB; };
  const T* q = reinterpret_cast<const T*>(a.q);
  T* o = reinterpret_cast<T*>(a.o);

  GenRows<SPARSE> gr;
  if (!gr.init(a)) {
    gen_zero<T, D, SPARSE>(a, a.o, a.lse, gr, false);
    return;
  }
  gen_zero<T, D, SPARSE>(a, a.o, a.lse, gr, true);
  if (gr.r0 >= gr.r_end) return;  // the second half of a short tile
  const QTile<SPARSE>& qt = gr.qt;
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, i = l & 15, G = l >> 4;
  const int hq = qt.hq, h = qt.h, W = a.window;
  const bool win = W >= 0;
  const int rw0 = gr.r0 + 16 * wave;
  const bool wave_active = rw0 < gr.r_end;
  const int r = rw0 + i;
  const bool valid = r < gr.r_end;
  const int64_t t = valid ? qt.rv.token(r) : 0;
  const int p = valid ? qt.rv.posn(r) : -1;
  const int pw_lo = wave_active ? qt.rv.posn(rw0) : 0;
  const int pw_hi = wave_active ? qt.rv.posn(min(rw0 + 15, gr.r_end - 1)) : -1;
  const int kv_lo = win ? (max(0, qt.rv.posn(gr.r0) - W) & ~(kKT - 1)) : 0;
  const int kv_hi = qt.rv.posn(gr.r_end - 1) + 1;
  const float c = a.scale_log2;
  const int stride = a.h * D;
  const T* k0 = reinterpret_cast<const T*>(a.k) + ((int64_t)qt.bos * a.h + h) * D;
  const T* v0 = reinterpret_cast<const T*>(a.v) + ((int64_t)qt.bos * a.h + h) * D;
  const int last_key = qt.seqlen - 1;
  auto issue = [&](int kt, int b) {  // keys past the segment read its last key (masked)
    const int last = min(kKT - 1, last_key - kt);
    TL::template dma<kKT, 256>(tK(b), k0 + (int64_t)kt * stride, stride, last);
    TL::template dma<kKT, 256>(tV(b), v0 + (int64_t)kt * stride, stride, last);
  };
  const int ntl = (kv_hi - kv_lo + kKT - 1) / kKT;
  issue(kv_lo, 0);

  Op qreg[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks)
    qreg[ks] = valid ? *reinterpret_cast<const Op*>(q + (t * a.hq + hq) * D + M::KSTEP * ks + M::NE * G) : Op{};
  f32x4 oacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) oacc[dt] = f32x4{};
  float m_run = -INFINITY, l_run = 0.f;

  for (int it = 0; it < ntl; ++it) {
    const int kt = kv_lo + kKT * it, b = it & 1;
    wait_vmem();
    __syncthreads();  // tile it has landed; every wave is done with stage b ^ 1
    if (it + 1 < ntl) issue(kt + kKT, b ^ 1);
    if (!wave_active || kt > pw_hi || (win && kt + kKT - 1 < pw_lo - W)) continue;
    const char* kb = tK(b);
    const char* vb = tV(b);
    f32x4 sacc[kKT / 16];
#pragma unroll
    for (int kb16 = 0; kb16 < kKT / 16; ++kb16) {
      sacc[kb16] = f32x4{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) sacc[kb16] = M::mma(TL::row(kb, 16 * kb16 + i, ks, G), qreg[ks], sacc[kb16]);
    }
    // scores in the log2 domain; item j of block kb16 is key kt + 16 kb16 + 4 G + j
    float mx = -INFINITY;
#pragma unroll
    for (int kb16 = 0; kb16 < kKT / 16; ++kb16)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = kt + 16 * kb16 + 4 * G + j;
        const bool vis = key <= p && (!win || key >= p - W);
        sacc[kb16][j] = vis ? sacc[kb16][j] * c : -INFINITY;
        mx = fmaxf(mx, sacc[kb16][j]);
      }
    mx = col_max(mx);
    const float m_new = fmaxf(m_run, mx);
    // A query with no visible key so far keeps m = -inf: its P, O and l stay
    // zero through base 0 (arithmetic, no branch: the MFMAs below run on
    // every lane of the wave).
    const float base = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = exp2f(m_run - base);
    float ls = 0.f;
#pragma unroll
    for (int kb16 = 0; kb16 < kKT / 16; ++kb16)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sacc[kb16][j] = exp2f(sacc[kb16][j] - base);
        ls += sacc[kb16][j];
      }
    l_run = l_run * alpha + col_sum(ls);
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) oacc[dt] *= alpha;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const Op pb = to_opk<T>(&sacc[kk * (M::KSTEP / 16)]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) oacc[dt] = M::mma(TL::trk(vb, M::KSTEP * kk, 16 * dt, l), pb, oacc[dt]);
    }
  }
  if (!valid) return;
  const float inv = 1.f / l_run;
  if (G == 0) a.lse[(int64_t)hq * a.n + r] = m_run + log2f(l_run);
  T* orow = o + (t * a.hq + hq) * D + 4 * G;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    typename M::V4 ov;
#pragma unroll
    for (int j = 0; j < 4; ++j) ov[j] = (T)(oacc[dt][j] * inv);
    *reinterpret_cast<typename M::V4*>(orow + 16 * dt) = ov;
  }
}

// ---------------------------------------------------------------------------
// delta = rowsum(o * dO) per compacted row, fp32 (:124-138)
// ---------------------------------------------------------------------------
template <typename T, int D, bool SPARSE>
__global__ __launch_bounds__(256) void gen_delta_kernel(const AttnArgs a) {
  const int hq = blockIdx.y;
  const int lane_sel = a.lanes > 1 ? hq : 0;
  const int32_t* meta = a.meta + (int64_t)lane_sel * a.meta_stride;
  const int sq = meta[0];
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  const int l = threadIdx.x & 63;
  if (r >= sq) return;
  const int64_t t = SPARSE ? a.q_idx[(int64_t)lane_sel * a.n + r] : (int64_t)r;
  const T* o = reinterpret_cast<const T*>(a.o) + (t * a.hq + hq) * D;
  const T* dout = reinterpret_cast<const T*>(a.dout) + (t * a.hq + hq) * D;
  float acc = 0.f;
#pragma unroll
  for (int e = l; e < D; e += 64) acc = fmaf((float)o[e], (float)dout[e], acc);
#pragma unroll
  for (int s = 32; s > 0; s >>= 1) acc += __shfl_xor(acc, s);
  if (l == 0) a.delta[(int64_t)hq * a.n + r] = acc;
}

// ---------------------------------------------------------------------------
// dq: dS^T = P^T (dP^T - delta), dQ^T += K^T dS^T (:141-228)
// ---------------------------------------------------------------------------
template <typename T, int D, bool SPARSE>
__global__ __launch_bounds__(256) void gen_dq_kernel(const AttnArgs a) {
  using M = Mma<T>;
  using Op = typename M::Op;
  using TL = GTile<T, D>;
  constexpr int KS = D / M::KSTEP, DT = D / 16, KB = kKT / 16, KK = kKT / M::KSTEP;
  auto tK = [](int b) { return logo_smem + b * 2 * kKT * TL::RB; };
  auto tV = [](int b) { return logo_smem + (b * 2 + 1) * kKT * TL::RB; };
  const T* q = reinterpret_cast<const T*>(a.q);
  const T* dout = reinterpret_cast<const T*>(a.dout);
  T* dq = reinterpret_cast<T*>(a.dq);

  GenRows<SPARSE> gr;
  if (!gr.init(a)) {
    gen_zero<T, D, SPARSE>(a, a.dq, nullptr, gr, false);
    return;
  }
  gen_zero<T, D, SPARSE>(a, a.dq, nullptr, gr, true);
  if (gr.r0 >= gr.r_end) return;
  const QTile<SPARSE>& qt = gr.qt;
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, i = l & 15, G = l >> 4;
  const int hq = qt.hq, h = qt.h, W = a.window;
  const bool win = W >= 0;
  const int rw0 = gr.r0 + 16 * wave;
  const bool wave_active = rw0 < gr.r_end;
  const int r = rw0 + i;
  const bool valid = r < gr.r_end;
  const int64_t t = valid ? qt.rv.token(r) : 0;
  const int p = valid ? qt.rv.posn(r) : -1;
  const int pw_lo = wave_active ? qt.rv.posn(rw0) : 0;
  const int pw_hi = wave_active ? qt.rv.posn(min(rw0 + 15, gr.r_end - 1)) : -1;
  const int kv_lo = win ? (max(0, qt.rv.posn(gr.r0) - W) & ~(kKT - 1)) : 0;
  const int kv_hi = qt.rv.posn(gr.r_end - 1) + 1;
  const float c = a.scale_log2;
  const int stride = a.h * D;
  const T* k0 = reinterpret_cast<const T*>(a.k) + ((int64_t)qt.bos * a.h + h) * D;
  const T* v0 = reinterpret_cast<const T*>(a.v) + ((int64_t)qt.bos * a.h + h) * D;
  const int last_key = qt.seqlen - 1;
  auto issue = [&](int kt, int b) {
    const int last = min(kKT - 1, last_key - kt);
    TL::template dma<kKT, 256>(tK(b), k0 + (int64_t)kt * stride, stride, last);
    TL::template dma<kKT, 256>(tV(b), v0 + (int64_t)kt * stride, stride, last);
  };
  const int ntl = (kv_hi - kv_lo + kKT - 1) / kKT;
  issue(kv_lo, 0);

  const float lse = valid ? a.lse[(int64_t)hq * a.n + r] : 0.f;
  const float dlt = valid ? a.delta[(int64_t)hq * a.n + r] : 0.f;
  Op qreg[KS], dreg[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int64_t off = (t * a.hq + hq) * D + M::KSTEP * ks + M::NE * G;
    qreg[ks] = valid ? *reinterpret_cast<const Op*>(q + off) : Op{};
    dreg[ks] = valid ? *reinterpret_cast<const Op*>(dout + off) : Op{};
  }
  f32x4 dqacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) dqacc[dt] = f32x4{};

  for (int it = 0; it < ntl; ++it) {
    const int kt = kv_lo + kKT * it, b = it & 1;
    wait_vmem();
    __syncthreads();
    if (it + 1 < ntl) issue(kt + kKT, b ^ 1);
    if (!wave_active || kt > pw_hi || (win && kt + kKT - 1 < pw_lo - W)) continue;
    const char* kb = tK(b);
    const char* vb = tV(b);
    f32x4 ds[KB];
#pragma unroll
    for (int kb16 = 0; kb16 < KB; ++kb16) {
      f32x4 s = f32x4{}, dp = f32x4{};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        s = M::mma(TL::row(kb, 16 * kb16 + i, ks, G), qreg[ks], s);
        dp = M::mma(TL::row(vb, 16 * kb16 + i, ks, G), dreg[ks], dp);
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int key = kt + 16 * kb16 + 4 * G + j;
        const bool vis = key <= p && (!win || key >= p - W);
        const float pr = vis ? exp2f(s[j] * c - lse) : 0.f;
        ds[kb16][j] = pr * (dp[j] - dlt);
      }
    }
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      const Op db = to_opk<T>(&ds[kk * (M::KSTEP / 16)]);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) dqacc[dt] = M::mma(TL::trk(kb, M::KSTEP * kk, 16 * dt, l), db, dqacc[dt]);
    }
  }
  if (!valid) return;
  T* drow = dq + (t * a.hq + hq) * D + 4 * G;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    typename M::V4 dv;
#pragma unroll
    for (int j = 0; j < 4; ++j) dv[j] = (T)(dqacc[dt][j] * a.scale);
    *reinterpret_cast<typename M::V4*>(drow + 16 * dt) = dv;
  }
}

// ---------------------------------------------------------------------------
// dk / dv: S = Q K^T, P, dP = dO V^T, dS; dV^T += dO^T P, dK^T += Q^T dS,
// summed over the query heads of the GQA group (:231-337, :444-445)
// ---------------------------------------------------------------------------
// Query rows per dk/dv step: one k step of the dV / dK products (whose k
// index is the query row), 32 for 16-bit types and 16 for fp32.
// LDS: two stages of [Q rows][dO rows][lse][delta][pos], that many rows each.
template <typename T>
constexpr int gen_qs() { return Mma<T>::KSTEP; }
template <typename T, int D>
constexpr size_t gen_dkv_stage() {
  return (size_t)2 * gen_qs<T>() * GTile<T, D>::RB + 3 * gen_qs<T>() * sizeof(float);
}

template <typename T, int D, bool SPARSE>
__global__ __launch_bounds__(256) void gen_dkv_kernel(const AttnArgs a) {
  using M = Mma<T>;
  using Op = typename M::Op;
  using TL = GTile<T, D>;
  constexpr int KS = D / M::KSTEP, DT = D / 16;
  constexpr int kQS = gen_qs<T>(), QB = kQS / 16;  // rows per step, 16-row blocks per step
  auto tQ = [](int b) { return logo_smem + b * gen_dkv_stage<T, D>(); };
  auto tO = [](int b) { return logo_smem + b * gen_dkv_stage<T, D>() + kQS * TL::RB; };
  auto sF = [](int b) { return reinterpret_cast<float*>(logo_smem + b * gen_dkv_stage<T, D>() + 2 * kQS * TL::RB); };
  const T* q = reinterpret_cast<const T*>(a.q);
  const T* k = reinterpret_cast<const T*>(a.k);
  const T* v = reinterpret_cast<const T*>(a.v);
  const T* dout = reinterpret_cast<const T*>(a.dout);

  int rank, h;
  xcd_remap(blockIdx.x, a.h, rank, h);
  const int32_t* meta0 = a.meta;
  const int ntk = meta0[2];
  const int tile = rank >> 1, sub = rank & 1;
  if (tile >= ntk) return;
  const int32_t* cu_tk = meta0 + kMetaHdr + 2 * (a.nseq + 1);
  const int s = seg_of(cu_tk, a.nseq, tile);
  const int bos = a.cu[s];
  const int seqlen = a.cu[s + 1] - bos;
  const int k0 = (tile - cu_tk[s]) * kBKV + kKeysWG * sub;
  if (k0 >= seqlen) return;
  const int k_last = min(k0 + kKeysWG, seqlen) - 1;

  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, i = l & 15, G = l >> 4;
  const int key = k0 + 16 * wave + i;
  const bool valid_k = key < seqlen;
  const bool wave_keys = 16 * wave + k0 <= k_last;  // this wave has keys in the segment
  const int W = a.window;
  const bool win = W >= 0;
  const float c = a.scale_log2;

  Op kreg[KS], vreg[KS];
  {
    const int64_t off = ((int64_t)(bos + key) * a.h + h) * D + M::NE * G;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      kreg[ks] = valid_k ? *reinterpret_cast<const Op*>(k + off + M::KSTEP * ks) : Op{};
      vreg[ks] = valid_k ? *reinterpret_cast<const Op*>(v + off + M::KSTEP * ks) : Op{};
    }
  }
  f32x4 dkacc[DT], dvacc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    dkacc[dt] = f32x4{};
    dvacc[dt] = f32x4{};
  }

  typename TL::template Staged<kQS, 256> sq, so;
  float st_lse = 0.f, st_delta = 0.f;
  int st_pos = -1;
  for (int gg = 0; gg < a.g; ++gg) {
    const int hq = h * a.g + gg;
    const int lane_sel = a.lanes > 1 ? hq : 0;
    const int32_t* cu_q = a.meta + (int64_t)lane_sel * a.meta_stride + kMetaHdr;
    const RowView<SPARSE> rv = row_view<SPARSE>(a, lane_sel, bos);
    const int q_lo = cu_q[s], q_hi = cu_q[s + 1];
    // rows ascend by position within the segment (dense rows: position = row - bos)
    auto lb_pos = [&](int lo, int hi, int x) {
      return SPARSE ? wave_lower_bound(rv.ps, lo, hi, x) : min(max(q_lo + x, lo), hi);
    };
    const int rq0 = lb_pos(q_lo, q_hi, k0);
    const int rq_end = win ? lb_pos(rq0, q_hi, k_last + W + 1) : q_hi;
    if (rq0 >= rq_end) continue;  // (uniform) no row of this head sees these keys
    const float* lse_h = a.lse + (int64_t)hq * a.n;
    const float* delta_h = a.delta + (int64_t)hq * a.n;
    const int last = rq_end - 1;
    // q / dO rows of a step through registers (gathered rows); rows past the
    // end read the last row and get position -1 (they see no key)
    auto fetch = [&](int rs) {
      sq.fetch([&](int rr) { return q + (rv.token(min(rs + rr, last)) * a.hq + hq) * D; });
      so.fetch([&](int rr) { return dout + (rv.token(min(rs + rr, last)) * a.hq + hq) * D; });
      if (tid < kQS) {
        const int rr = rs + tid, rc = min(rr, last);
        st_lse = lse_h[rc];
        st_delta = delta_h[rc];
        st_pos = rr < rq_end ? rv.posn(rr) : -1;
      }
    };
    auto stash = [&](int b) {
      sq.stash(tQ(b));
      so.stash(tO(b));
      if (tid < kQS) {
        sF(b)[tid] = st_lse;
        sF(b)[kQS + tid] = st_delta;
        reinterpret_cast<int*>(sF(b))[2 * kQS + tid] = st_pos;
      }
    };
    __syncthreads();  // the previous head's last step is done with both stages
    fetch(rq0);
    stash(0);
    __syncthreads();
    int b = 0;
    for (int rs = rq0; rs < rq_end; rs += kQS, b ^= 1) {
      const bool more = rs + kQS < rq_end;
      if (more) fetch(rs + kQS);  // in flight during this step's products
      if (wave_keys) {
        const char* qb = tQ(b);
        const char* ob = tO(b);
        const float* sLse = sF(b);
        const float* sDelta = sLse + kQS;
        const int* sPos = reinterpret_cast<const int*>(sLse + 2 * kQS);
        f32x4 pr[QB], ds[QB];
#pragma unroll
        for (int qb16 = 0; qb16 < QB; ++qb16) {
          f32x4 sacc = f32x4{}, dpacc = f32x4{};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            sacc = M::mma(TL::row(qb, 16 * qb16 + i, ks, G), kreg[ks], sacc);
            dpacc = M::mma(TL::row(ob, 16 * qb16 + i, ks, G), vreg[ks], dpacc);
          }
          // item j: query row rs + 16 qb16 + 4 G + j, key `key`
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int rj = 16 * qb16 + 4 * G + j;
            const int pq = sPos[rj];
            const bool vis = valid_k && key <= pq && (!win || key >= pq - W);
            pr[qb16][j] = vis ? exp2f(sacc[j] * c - sLse[rj]) : 0.f;
            ds[qb16][j] = pr[qb16][j] * (dpacc[j] - sDelta[rj]);
          }
        }
        const Op pb = to_opk<T>(pr), db = to_opk<T>(ds);
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          dvacc[dt] = M::mma(TL::trk(ob, 0, 16 * dt, l), pb, dvacc[dt]);
          dkacc[dt] = M::mma(TL::trk(qb, 0, 16 * dt, l), db, dkacc[dt]);
        }
      }
      if (more) stash(b ^ 1);  // stage b ^ 1 was last read in the previous step
      __syncthreads();
    }
  }
  if (!valid_k) return;
  // lane (i, G) holds columns 16 dt + 4 G .. + 3 of key `key`
  const int64_t off = ((int64_t)(bos + key) * a.h + h) * D + 4 * G;
  T* dk = reinterpret_cast<T*>(a.dk) + off;
  T* dv = reinterpret_cast<T*>(a.dv) + off;
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    typename M::V4 kv, vv;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      kv[j] = (T)(dkacc[dt][j] * a.scale);
      vv[j] = (T)dvacc[dt][j];
    }
    *reinterpret_cast<typename M::V4*>(dk + 16 * dt) = kv;
    *reinterpret_cast<typename M::V4*>(dv + 16 * dt) = vv;
  }
}

// ---------------------------------------------------------------------------
// Launchers
// ---------------------------------------------------------------------------
// fwd / dq: two stages of a K and a V tile of kKT keys
template <typename T, int D>
constexpr size_t gen_kv_smem() { return (size_t)4 * kKT * GTile<T, D>::RB; }

// fwd / dq grid: two workgroups per 128-row tile (worst case over the lanes),
// per query head.
inline int64_t gen_row_grid(const AttnArgs& a) { return 2 * ((a.n + kBQ - 1) / kBQ + a.nseq) * a.hq; }

template <typename T, int D, bool SPARSE>
int launch_fwd(const AttnArgs& a, hipStream_t st) {
  const int64_t nblk = gen_row_grid(a);
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "grid too large");
  auto kern = gen_fwd_kernel<T, D, SPARSE>;
  const size_t smem = gen_kv_smem<T, D>();
  LOGO_HIP_CHECK(allow_smem(kern, smem));
  hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(256), smem, st, a);
  LOGO_LAUNCH_CHECK("gen_fwd_kernel");
  return LOGO_OK;
}

template <typename T, int D, bool SPARSE>
int launch_delta(const AttnArgs& a, hipStream_t st) {
  dim3 grid((unsigned)((a.n + 3) / 4), a.hq);
  hipLaunchKernelGGL((gen_delta_kernel<T, D, SPARSE>), grid, dim3(256), 0, st, a);
  LOGO_LAUNCH_CHECK("gen_delta_kernel");
  return LOGO_OK;
}

template <typename T, int D, bool SPARSE>
int launch_dq(const AttnArgs& a, hipStream_t st) {
  const int64_t nblk = gen_row_grid(a);
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "grid too large");
  auto kern = gen_dq_kernel<T, D, SPARSE>;
  const size_t smem = gen_kv_smem<T, D>();
  LOGO_HIP_CHECK(allow_smem(kern, smem));
  hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(256), smem, st, a);
  LOGO_LAUNCH_CHECK("gen_dq_kernel");
  return LOGO_OK;
}

template <typename T, int D, bool SPARSE>
int launch_dkv(const AttnArgs& a, hipStream_t st) {
  // two workgroups per 128-key tile (worst case), per kv head
  const int64_t nblk = 2 * ((a.n + kBKV - 1) / kBKV + a.nseq) * a.h;
  LOGO_REQUIRE(nblk < ((int64_t)1 << 31), "grid too large");
  auto kern = gen_dkv_kernel<T, D, SPARSE>;
  const size_t smem = 2 * gen_dkv_stage<T, D>();
  LOGO_HIP_CHECK(allow_smem(kern, smem));
  hipLaunchKernelGGL(kern, dim3((unsigned)nblk), dim3(256), smem, st, a);
  LOGO_LAUNCH_CHECK("gen_dkv_kernel");
  return LOGO_OK;
}

// The instantiations that exist: sparse bf16 / fp16 at D = 256, sparse fp32
// at D = 64, 128, 256, dense (with or without a window) bf16 at D = 256.
#define LOGO_GEN_DISPATCH(FN, a, st, d, dtype, sparse)                                                  \
  do {                                                                                                  \
    if (dtype == LOGO_DTYPE_F32 && sparse)                                                              \
      return d == 64 ? FN<float, 64, true>(a, st) : d == 128 ? FN<float, 128, true>(a, st)              \
                                                             : FN<float, 256, true>(a, st);             \
    if (d == 256 && dtype == LOGO_DTYPE_F16 && sparse) return FN<f16, 256, true>(a, st);               \
    if (d == 256 && dtype == LOGO_DTYPE_BF16) return sparse ? FN<bf16, 256, true>(a, st)                \
                                                            : FN<bf16, 256, false>(a, st);              \
    LOGO_REQUIRE(false, "no generic attention kernel for d=%d dtype=%d sparse=%d", d, dtype, (int)sparse); \
  } while (0)

}  // namespace gen

bool gen_applies(int d, int dtype) { return d == 256 || dtype == LOGO_DTYPE_F32; }

int gen_launch_fwd(const AttnArgs& a, hipStream_t st, int d, int dtype, bool sparse) {
  LOGO_GEN_DISPATCH(gen::launch_fwd, a, st, d, dtype, sparse);
}
int gen_launch_delta(const AttnArgs& a, hipStream_t st, int d, int dtype, bool sparse) {
  LOGO_GEN_DISPATCH(gen::launch_delta, a, st, d, dtype, sparse);
}
int gen_launch_dq(const AttnArgs& a, hipStream_t st, int d, int dtype, bool sparse) {
  LOGO_GEN_DISPATCH(gen::launch_dq, a, st, d, dtype, sparse);
}
int gen_launch_dkv(const AttnArgs& a, hipStream_t st, int d, int dtype, bool sparse) {
  LOGO_GEN_DISPATCH(gen::launch_dkv, a, st, d, dtype, sparse);
}

}  // namespace logo
