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
// order (see read_perm_k).
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
constexpr int kBK = 64;    // keys per LDS tile (fwd, dq) / query rows per LDS tile (dkv)
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

// Pack two bf16 from two dwords: lo halves (even element) or hi halves (odd).
__device__ __forceinline__ uint32_t pack_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t pack_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

// A 64-row x D-column bf16 tile moved global -> registers -> LDS by 256
// threads.  Thread tid owns the 16-byte column chunk c = tid % CH of rows
// rg*RPT .. rg*RPT+RPT-1 (rg = tid / CH), so every group of CH lanes reads
// one contiguous row.
template <int D>
struct Tile64 {
  static constexpr int CH = D / 8;
  static constexpr int RPT = (64 * CH) / 256;  // rows per thread: D/32
  static constexpr int RS = D + 8;             // row-major LDS stride (elements)
  static constexpr int TS = 64 + 4;            // transposed LDS stride (elements)
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

  // Row-major store: lds[row * RS + col].
  __device__ __forceinline__ void store_rows(bf16* lds, int tid) const {
    const int c = chunk(tid), r0 = row0(tid);
#pragma unroll
    for (int i = 0; i < RPT; ++i) *reinterpret_cast<u32x4*>(lds + (r0 + i) * RS + 8 * c) = r[i];
  }

  // Transposed store: lds[col * TS + row].
  __device__ __forceinline__ void store_cols(bf16* lds, int tid) const {
    const int c = chunk(tid), r0 = row0(tid);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int w = e >> 1;
      bf16* dst = lds + (8 * c + e) * TS + r0;
      if constexpr (RPT == 4) {
        u32x2 v;
        v[0] = (e & 1) ? pack_hi(r[0][w], r[1][w]) : pack_lo(r[0][w], r[1][w]);
        v[1] = (e & 1) ? pack_hi(r[2][w], r[3][w]) : pack_lo(r[2][w], r[3][w]);
        *reinterpret_cast<u32x2*>(dst) = v;
      } else {
        *reinterpret_cast<uint32_t*>(dst) = (e & 1) ? pack_hi(r[0][w], r[1][w]) : pack_lo(r[0][w], r[1][w]);
      }
    }
  }
};

// Row-major operand: 8 consecutive columns 16*ks + 8*g of row `row`.
template <int RS>
__device__ __forceinline__ bf16x8 read_row_op(const bf16* lds, int row, int ks, int g) {
  return *reinterpret_cast<const bf16x8*>(lds + row * RS + 16 * ks + 8 * g);
}

// Transposed operand whose k order matches acc_to_bf16(acc, ks & 1) of the
// 32-row accumulator tile ks >> 1: columns 16*ks + {4g..4g+3, 8+4g..8+4g+3}.
template <int TS>
__device__ __forceinline__ bf16x8 read_perm_k(const bf16* lds, int row, int ks, int g) {
  const bf16* p = lds + row * TS + 16 * ks + 4 * g;
  u32x2 lo = *reinterpret_cast<const u32x2*>(p);
  u32x2 hi = *reinterpret_cast<const u32x2*>(p + 8);
  u32x4 v{lo[0], lo[1], hi[0], hi[1]};
  return as_bf16x8(v);
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
