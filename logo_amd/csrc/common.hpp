// Shared device helpers for the LoGo attention kernels (gfx950 / CDNA4).
//
// Matrix products run on v_mfma_f32_32x32x16_bf16.  Lane l of a wave64 holds
// (i = l % 32, g = l / 32):
//   A operand  A[m = i][k in Kset(g)]     8 bf16
//   B operand  B[k in Kset(g)][n = i]     8 bf16
//   D/C        D[m = rowmap(g, j)][n = i] 16 fp32, rowmap(g, j) = 8*(j/4) + 4*g + j%4
// The hardware's k ordering inside Kset(g) only has to agree between A and B,
// so operands built from an accumulator (P, dS) use the accumulator's own row
// order as their k order and the matching operand is read from LDS in that
// order (see read_tr_op).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace logo {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Library-wide tile constants (must match include/logo_hip.h).
constexpr int kBQ = 128;   // compacted query rows per workgroup (fwd, dq)
constexpr int kBKV = 128;  // keys per workgroup (dkv)
constexpr int kMetaHdr = 8;

__device__ __forceinline__ int rowmap(int g, int j) { return 8 * (j >> 2) + 4 * g + (j & 3); }

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Eight accumulator items (8h .. 8h+7 of a 32x32 tile) as a bf16 operand.
__device__ __forceinline__ bf16x8 acc_to_bf16(const f32x16& a, int h) {
  bf16x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (bf16)a[8 * h + e];
  return r;
}

// A 64-row x D-column bf16 tile moved global -> registers -> LDS (row-major,
// row stride RS elements) by 256 threads.  Thread tid owns the 16-byte column
// chunk c = tid % CH of rows rg*RPT .. rg*RPT+RPT-1 (rg = tid / CH), so every
// group of CH lanes reads one contiguous row.
template <int D, int RS>
struct Tile64 {
  static constexpr int CH = D / 8;
  static constexpr int RPT = (64 * CH) / 256;  // rows per thread: D/32
  static_assert(RPT == 2 || RPT == 4, "head dim must be 64 or 128");
  u32x4 r[RPT];

  __device__ __forceinline__ static int chunk(int tid) { return tid % CH; }
  __device__ __forceinline__ static int row0(int tid) { return (tid / CH) * RPT; }

  // rowptr(row) returns the row's base pointer or nullptr for a zero row.
  template <typename F>
  __device__ __forceinline__ void load(int tid, F rowptr) {
    const int c = chunk(tid), r0 = row0(tid);
#pragma unroll
    for (int i = 0; i < RPT; ++i) {
      const bf16* p = rowptr(r0 + i);
      r[i] = p ? *reinterpret_cast<const u32x4*>(p + 8 * c) : u32x4{0u, 0u, 0u, 0u};
    }
  }

  __device__ __forceinline__ void store(bf16* lds, int tid) const {
    const int c = chunk(tid), r0 = row0(tid);
#pragma unroll
    for (int i = 0; i < RPT; ++i) *reinterpret_cast<u32x4*>(lds + (r0 + i) * RS + 8 * c) = r[i];
  }
};

// LDS row strides (elements).  Tiles read only with ds_read_b128 along rows
// use D + 8 (row starts 4 banks apart: conflict-free for 16 lanes reading 16
// rows); tiles also read with the transposing ds_read_b64_tr_b16 use D + 16
// (row starts 8 banks apart: the 4 rows x 4 chunks of a 16-lane group hit 32
// distinct banks).
template <int D> constexpr int kRowStride = D + 8;
template <int D> constexpr int kTrStride = D + 16;

// Row-major operand: 8 consecutive columns 16*ks + 8*g of row `row`.
template <int RS>
__device__ __forceinline__ bf16x8 read_row_op(const bf16* lds, int row, int ks, int g) {
  return *reinterpret_cast<const bf16x8*>(lds + row * RS + 16 * ks + 8 * g);
}

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;

// Transposed operand from a row-major tile T (row stride RS): lane (i, g)
// receives T[r0 + 4g + e][c0 + i] for e = 0..3 followed by
// T[r0 + 8 + 4g + e][c0 + i], the k order acc_to_bf16(acc, ks & 1) produces
// for r0 = 16*ks.  ds_read_b64_tr_b16 gives lane 16G + 4a + b element b of the
// 8-byte chunks addressed by lanes 16G + a + 4e (e = 0..3), so lane 16G + j
// addresses row r0 + 4g + j/4, column c0 + 16(G & 1) + 4(j & 3).
template <int RS>
__device__ __forceinline__ bf16x8 read_tr_op(const bf16* lds, int r0, int c0) {
  const int l = threadIdx.x & 63;
  const int G = l >> 4, j = l & 15;
  const bf16* p = lds + (r0 + 4 * (G >> 1) + (j >> 2)) * RS + c0 + 16 * (G & 1) + 4 * (j & 3);
  const bf16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p));
  const bf16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4bf16((lds_bf16x4*)(p + 8 * RS));
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Largest s in [0, n) with arr[s] <= x (arr ascending, arr[0] <= x).
__device__ __forceinline__ int seg_of(const int32_t* arr, int n, int64_t x) {
  int lo = 0, hi = n;  // invariant: arr[lo] <= x, answer < hi
  while (hi - lo > 1) {
    int mid = (lo + hi) >> 1;
    if ((int64_t)arr[mid] <= x) lo = mid; else hi = mid;
  }
  return lo;
}

// First index r in [lo, hi) with arr[r] >= x (arr ascending), hi if none.
__device__ __forceinline__ int lower_bound_i32(const int32_t* arr, int lo, int hi, int x) {
  while (lo < hi) {
    int mid = (lo + hi) >> 1;
    if (arr[mid] < x) lo = mid + 1; else hi = mid;
  }
  return lo;
}

// Workgroup id -> (rank, head) so that the workgroups of one head land on one
// XCD (workgroups are dispatched round-robin over the 8 XCDs), keeping that
// head's K/V in one L2.  Ranks are visited in launch order.
__device__ __forceinline__ void xcd_remap(int L, int heads, int& rank, int& head) {
  if ((heads & 7) == 0) {
    const int hpx = heads >> 3;
    const int xcd = L & 7, k = L >> 3;
    head = xcd * hpx + (k % hpx);
    rank = k / hpx;
  } else {
    head = L % heads;
    rank = L / heads;
  }
}

}  // namespace logo
