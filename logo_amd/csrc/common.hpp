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

#include <type_traits>
#include <utility>

namespace logo {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16;
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef __fp16 hf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Library-wide tile constants (must match include/logo_hip.h).
constexpr int kBQ = 128;   // compacted query rows per workgroup (fwd, dq)
constexpr int kBKV = 128;  // keys per workgroup (dkv)
constexpr int kMetaHdr = 8;

typedef __attribute__((address_space(3))) bf16x4 lds_bf16x4;
typedef __attribute__((address_space(3))) hf16x4 lds_hf16x4;

// The 16-bit element types the attention kernels compute in: bf16, and fp16
// for fp16 callers (the reference's dots run in the input dtype,
// logo/ops/selected_full_attn.py:95-99).  Storage is 16 bits either way, so
// pointers stay bf16* and only values, MFMAs and conversions change.
template <typename E>
struct Elem;
template <>
struct Elem<bf16> {
  using x8 = bf16x8;
  using x4 = bf16x4;
  static constexpr bool kHalf = false;
  __device__ __forceinline__ static f32x16 mfma(x8 a, x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
  }
};
template <>
struct Elem<f16> {
  using x8 = f16x8;
  using x4 = f16x4;
  static constexpr bool kHalf = true;
  __device__ __forceinline__ static f32x16 mfma(x8 a, x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
  }
};

// D += A * B (v_mfma_f32_32x32x16_bf16) with D held in AGPRs, for
// accumulators that only MFMAs touch inside the loop (the other MFMAs of a
// kernel built with VGPR-form results keep theirs in VGPRs).  The compiler
// does not see inside the asm, so it supplies its own wait states: the
// leading s_nop covers a VALU write of A, B or D just before it, and
// agpr_acc_drain() must run before any other instruction reads D.  That
// includes copies the register allocator itself inserts: a kernel whose
// loop ends up with v_accvgpr_mov of such an accumulator (seen when a
// branch around the MFMA phase became scalar) reads it before the MFMA has
// written it, so the ISA of these kernels is checked for in-loop copies.
__device__ __forceinline__ void mfma32_agpr(f32x16& d, const bf16x8& a, const bf16x8& b) {
  asm volatile("s_nop 2\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma32_agpr(f32x16& d, const f16x8& a, const f16x8& b) {
  asm volatile("s_nop 2\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
}
// mfma32_agpr without the leading wait states, for schedules in which no VALU
// instruction writes A or B within the three instructions before the MFMA
// (the operands are LDS reads, or packed several MFMA slots earlier).  The
// leading s_nop costs three issue cycles per MFMA, which one wave per SIMD
// pays in full (dk/dv: 4% of the kernel).  The ISA test checks the operand
// distance in every kernel that uses it.
__device__ __forceinline__ void mfma32_agpr_ready(f32x16& d, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma32_agpr_ready(f32x16& d, const f16x8& a, const f16x8& b) {
  asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(d) : "v"(a), "v"(b));
}
// Wait states between the last mfma32_agpr and a VALU read of its result
// (an 8-pass MFMA needs fewer than 32).  The compiler may place its own
// copies out of the AGPRs ahead of this operand-less asm, so kernels also run
// it at the end of every iteration of their MFMA loop: the epilogue's reads,
// which cannot move into the loop, then always follow wait states.
__device__ __forceinline__ void agpr_acc_drain() { asm volatile("s_nop 15\n\ts_nop 15"); }

// Reductions over the lane pair (l, l ^ 32): v_permlane32_swap hands every
// lane both values of its pair.
__device__ __forceinline__ float pair_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float pair_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// max(a, b, c) as one v_max3_f32, kept at its place in the instruction
// stream.  (fmaxf on values that come out of an asm anchor would first be
// canonicalised, one extra v_max per operand.)  NaN handling is not needed:
// the attention scores it reduces are finite or -inf.
__device__ __forceinline__ float max3_f32(float a, float b, float c) {
  float r;
  asm volatile("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// min(a, b, c) as one v_min3_f32 (see max3_f32).
__device__ __forceinline__ float min3_f32(float a, float b, float c) {
  float r;
  asm volatile("v_min3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

__device__ __forceinline__ float pair_min(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fminf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// Eight bf16 values times s, each rounded back to bf16 (the pre-scaled query
// rows of the sparse path: the forward's registers and the backward's
// compacted copies are made by this same rounding).
template <typename V>
__device__ __forceinline__ V scale8(const V v, float s) {
  using T = std::remove_cv_t<std::remove_reference_t<decltype(v[0])>>;
  V r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (T)((float)v[e] * s);
  return r;
}
__device__ __forceinline__ bf16x8 scale_bf16x8(const bf16x8 v, float s) { return scale8(v, s); }

// Anchors a value at this point of the instruction stream (an empty asm
// statement that reads and rewrites it): arithmetic on it cannot be hoisted
// above, nor its producer sunk below, this point.  Used with scheduling
// fences to lay out MFMA / VALU / LDS slots explicitly.
template <typename T>
__device__ __forceinline__ void pin(T& x) { asm volatile("" : "+v"(x)); }

// Streaming 16-byte global accesses: non-temporal loads and stores, for data
// a kernel reads or writes once and no kernel re-reads soon (they stream
// faster than ordinary accesses on this part: a 1 GiB copy 5.9-6.1 against
// 5.5 TB/s, a read 7.1 against 6.3 TB/s).  Used where they measured faster:
// the decode cache reads, RoPE, the epilogue's backward and the sparse
// backward's outputs (dq, dk, dv and the zero rows); not where the next
// kernel reads the data again (a store the next kernel reads, such as the
// delta phase's copies or the epilogue's output, measured slower).
template <typename V>
__device__ __forceinline__ V ld_nt(const V* p) { return __builtin_nontemporal_load(p); }
template <typename V>
__device__ __forceinline__ void st_nt(V* p, V v) { __builtin_nontemporal_store(v, p); }

// Calls f(std::integral_constant<int, I>{}) for I = 0 .. N-1 (compile-time
// indices, so per-slot register arrays stay in registers).
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

__device__ __forceinline__ int rowmap(int g, int j) { return 8 * (j >> 2) + 4 * g + (j & 3); }

__device__ __forceinline__ f32x16 mfma32(bf16x8 a, bf16x8 b, f32x16 c) { return Elem<bf16>::mfma(a, b, c); }
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) { return Elem<f16>::mfma(a, b, c); }

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// Eight accumulator items (8h .. 8h+7 of a 32x32 tile) as a 16-bit operand.
template <typename E = bf16>
__device__ __forceinline__ typename Elem<E>::x8 acc_to(const f32x16& a, int h) {
  typename Elem<E>::x8 r;
#pragma unroll
  for (int e = 0; e < 8; ++e) r[e] = (E)a[8 * h + e];
  return r;
}
__device__ __forceinline__ bf16x8 acc_to_bf16(const f32x16& a, int h) { return acc_to<bf16>(a, h); }

// LDS tile layouts.  gfx950's LDS serves 64 four-byte banks per cycle:
// ds_read_b128 16 lanes per cycle, ds_read_b64_tr_b16 32 lanes per cycle.
//   kRow : rows padded to D + 8 elements (start 4 banks apart): 16 lanes
//          reading one 16-byte chunk of 16 consecutive rows hit 64 distinct
//          banks.  For tiles read only along rows.
//   kTr  : rows padded to D + 32 (start 16 banks apart): a transposing read
//          covers rows 4m..4m+3 x 32 consecutive columns, again 64 distinct
//          banks.  For tiles read only through ds_read_b64_tr_b16.
//   kSwz : no padding; the 16-byte chunk ch of row r is stored at chunk
//          ch ^ swz(r), swz(r) = 4*(r & 3) | ((r >> 2) & 3): conflict-free
//          for both read kinds (swz takes all 16 values on 16 aligned rows;
//          on rows 4m..4m+3 times chunks C..C+3, (C | dc) ^ (4e + x) is
//          distinct).  For tiles read both ways.
// Row stores (16 lanes write the 16 chunks of one row) are conflict-free in
// every layout.  D = 64 uses the low three swizzle bits (correct; the
// conflict analysis above is for D = 128).
enum TileKind { kRow = 0, kTr = 1, kSwz = 2 };

template <int D, int KIND>
struct TileGeom {
  static constexpr int RS = KIND == kRow ? D + 8 : KIND == kTr ? D + 32 : D;  // row stride (elements)
  static constexpr int ELEMS = 64 * RS;
  __device__ __forceinline__ static int swz(int r) {
    return KIND == kSwz ? ((((r & 3) << 2) | ((r >> 2) & 3)) & (D / 8 - 1)) : 0;
  }
  // element offset of (row r, logical 16-byte chunk ch)
  __device__ __forceinline__ static int off(int r, int ch) { return r * RS + ((ch ^ swz(r)) << 3); }
};

// A 64-row x D-column bf16 tile moved global -> registers -> LDS by 256
// threads.  Thread tid owns the 16-byte column chunk c = tid % CH of rows
// rg*RPT .. rg*RPT+RPT-1 (rg = tid / CH), so every group of CH lanes reads one
// contiguous row.
template <int D>
struct Tile64 {
  static constexpr int CH = D / 8;
  static constexpr int RPT = (64 * CH) / 256;  // rows per thread: D/32
  static_assert(RPT == 2 || RPT == 4, "head dim must be 64 or 128");
  u32x4 r[RPT];

  __device__ __forceinline__ static int chunk(int tid) { return tid % CH; }
  __device__ __forceinline__ static int row0(int tid) { return (tid / CH) * RPT; }

  // rowptr(row) returns a valid row pointer for every tile row: callers
  // clamp rows past the end of their range to a real row, whose (finite)
  // values the attention mask then ignores, so the loads are unconditional.
  template <typename F>
  __device__ __forceinline__ void load(int tid, F rowptr) {
    const int c = chunk(tid), r0 = row0(tid);
#pragma unroll
    for (int i = 0; i < RPT; ++i) r[i] = *reinterpret_cast<const u32x4*>(rowptr(r0 + i) + 8 * c);
  }

  template <int KIND>
  __device__ __forceinline__ void store(bf16* lds, int tid) const {
    const int c = chunk(tid), r0 = row0(tid);
#pragma unroll
    for (int i = 0; i < RPT; ++i) *reinterpret_cast<u32x4*>(lds + TileGeom<D, KIND>::off(r0 + i, c)) = r[i];
  }
};

// Global -> LDS copy of a 64-row x D-column bf16 tile into the kSwz layout
// with buffer_load_dwordx4 ... lds (no register staging, no LDS store
// instructions).  Each such load writes 64 lanes x 16 bytes = 1 KB contiguous
// at a wave-uniform LDS address, i.e. RPB = 64 / CH whole rows; lane j fills
// physical chunk j % CH of row (block row + j / CH), so it loads that row's
// logical chunk (j % CH) ^ swz(row).  With NW waves, wave w copies rows
// (64 / NW) w .. (64 / NW)(w + 1) - 1.  The caller waits for the loads
// (s_waitcnt vmcnt) before the barrier that publishes the tile.
//
// The loads use a scalar buffer descriptor based at the tile's first row and
// one 32-bit lane offset per 1 KB block (loop-invariant for full tiles).  The
// descriptor's extent is the 64 rows of the tile, so the hardware returns
// zeros for any read past them instead of touching memory outside the tile.
// (The FLAT-encoded global_load_lds form is avoided: while one is in flight
// the compiler treats the LDS counter as out of order and turns every LDS
// operand wait into a full lgkmcnt(0) drain.)
constexpr int kBufRsrcWord3 = 0x00020000;  // raw, untyped 32-bit buffer (gfx9 family)

// One buffer_load_dwordx4 ... lds: 64 lanes x 16 bytes to LDS at `lds`
// (wave-uniform).  A non-template wrapper: clang's host pass drops the host
// stubs of later kernel instantiations when this builtin sits directly in a
// template.
__device__ __forceinline__ void buf_load_lds16(__amdgpu_buffer_rsrc_t r, bf16* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, 0, 0, 0);
}

template <int D, int NW = 4>
struct TileBufDma {
  static constexpr int CH = D / 8;
  static constexpr int RPB = 64 / CH;
  static constexpr int RPW = 64 / NW;
  static constexpr int BLOCKS = RPW / RPB;
  using Geo = TileGeom<D, kSwz>;
  uint32_t o[BLOCKS];  // byte offsets from the tile's first row (all 64 rows valid)
  int row_stride;      // elements

  __device__ __forceinline__ void init(int row_stride_elems) {
    row_stride = row_stride_elems;
    const int wave = threadIdx.x >> 6, j = threadIdx.x & 63;
#pragma unroll
    for (int b = 0; b < BLOCKS; ++b) {
      const int row = RPW * wave + RPB * b + j / CH;
      const int ch = (j % CH) ^ Geo::swz(row);
      o[b] = (uint32_t)(row * row_stride + 8 * ch) * (uint32_t)sizeof(bf16);
    }
  }

  __device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const bf16* row0) const {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<bf16*>(row0), (short)0,
                                             64 * row_stride * (int)sizeof(bf16), kBufRsrcWord3);
  }

  // The wave index as a scalar: the LDS destination of each copy (M0) is then
  // scalar arithmetic instead of a per-copy readfirstlane of a vector value.
  __device__ __forceinline__ static int wave_s() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

  // Rows row0 .. row0 + 63, all valid.
  __device__ __forceinline__ void issue(bf16* tile, const bf16* row0) const {
    const auto r = rsrc(row0);
    const int wave = wave_s();
#pragma unroll
    for (int b = 0; b < BLOCKS; ++b) {
      const int rb = RPW * wave + RPB * b;
      buf_load_lds16(r, tile + rb * D, o[b]);
    }
  }

  // Rows past last_row (< 63) are clamped to it.
  __device__ __forceinline__ void issue_clamped(bf16* tile, const bf16* row0, int last_row) const {
    const auto r = rsrc(row0);
    const int wave = wave_s(), j = threadIdx.x & 63;
#pragma unroll
    for (int b = 0; b < BLOCKS; ++b) {
      const int rb = RPW * wave + RPB * b;
      const int row = rb + j / CH;
      const int ch = (j % CH) ^ Geo::swz(row);
      const uint32_t off = (uint32_t)(min(row, last_row) * row_stride + 8 * ch) * (uint32_t)sizeof(bf16);
      buf_load_lds16(r, tile + rb * D, off);
    }
  }
};

// Wait for this wave's outstanding vector-memory operations (the tile copies
// above) to land.
__device__ __forceinline__ void wait_vmem() { __builtin_amdgcn_s_waitcnt(0); }

// LDS reads through a restrict pointer: inlining gives the read
// alias-scope metadata, without which the compiler's wait-count insertion
// treats it as possibly reading LDS that an in-flight global->LDS copy (the
// next tile, into the other buffer) writes, and stalls it on that copy.
// The kernels order those copies against reads with explicit waits and
// barriers.
template <typename T>
__device__ __attribute__((always_inline)) inline T lds_load(const T* __restrict__ p) {
  return *p;
}
__device__ __attribute__((always_inline)) inline bf16x4 ds_read_tr(const lds_bf16x4* __restrict__ p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16(const_cast<lds_bf16x4*>(p));
}
__device__ __attribute__((always_inline)) inline f16x4 ds_read_tr(const lds_hf16x4* __restrict__ p) {
  return __builtin_bit_cast(f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4f16(const_cast<lds_hf16x4*>(p)));
}

// MFMA operand reads from a tile, with every lane-dependent part of the
// address computed once (init) so that in the unrolled loops each read is a
// lane register plus an immediate.
//   row(tile, rbase, ks): lane (i, g) gets the 8 columns 16*ks + 8*g of row
//     rbase + i (rbase a multiple of 16) -- the A/B operand whose m/n index
//     is the tile row.
//   tr(tile, r0, dt): lane (i, g) gets T[r0 + 4g + e][32*dt + i] for e = 0..3
//     then T[r0 + 8 + 4g + e][32*dt + i] (r0 a multiple of 16), the k order
//     acc_to_bf16(acc, ks & 1) produces for r0 = 16*ks.  ds_read_b64_tr_b16
//     gives lane 16G + 4a + b element b of the 8-byte chunks addressed by
//     lanes 16G + a + 4e (e = 0..3), so lane 16G + j addresses row
//     r0 + 4g + j/4 (+ 8), column 32*dt + 16(G & 1) + 4(j & 3).
template <int D, int KIND>
struct TileReader {
  using Geo = TileGeom<D, KIND>;
  static constexpr int DS = D / 16, DT = D / 32;
  static constexpr bool SWZ = KIND == kSwz;
  int row_off[SWZ ? DS : 1];
  int tr_off[SWZ ? 2 * DT : 1];

  __device__ __forceinline__ void init() {
    const int l = threadIdx.x & 63, i = l & 31, g = l >> 5;
    const int G = l >> 4, j = l & 15;
    if constexpr (SWZ) {
#pragma unroll
      for (int ks = 0; ks < DS; ++ks) row_off[ks] = Geo::off(i, 2 * ks + g);
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int row = 4 * g + (j >> 2) + 8 * h;
          const int col = 32 * dt + 16 * (G & 1) + 4 * (j & 3);
          tr_off[2 * dt + h] = Geo::off(row, col >> 3) + (col & 7);
        }
    } else {
      row_off[0] = i * Geo::RS + 8 * g;
      tr_off[0] = (4 * g + (j >> 2)) * Geo::RS + 16 * (G & 1) + 4 * (j & 3);
    }
  }

  // E: the element type the tile holds (its storage is addressed as bf16)
  template <typename E = bf16>
  __device__ __forceinline__ typename Elem<E>::x8 row(const bf16* tile, int rbase, int ks) const {
    const int o = SWZ ? rbase * Geo::RS + row_off[ks] : rbase * Geo::RS + 16 * ks + row_off[0];
    return lds_load(reinterpret_cast<const typename Elem<E>::x8*>(tile + o));
  }

  template <typename E = bf16>
  __device__ __forceinline__ typename Elem<E>::x8 tr(const bf16* tile, int r0, int dt) const {
    using L4 = std::conditional_t<Elem<E>::kHalf, lds_hf16x4, lds_bf16x4>;
    const int o0 = SWZ ? r0 * Geo::RS + tr_off[2 * dt] : r0 * Geo::RS + 32 * dt + tr_off[0];
    const int o1 = SWZ ? r0 * Geo::RS + tr_off[2 * dt + 1] : o0 + 8 * Geo::RS;
    const auto lo = ds_read_tr((const L4*)(tile + o0));
    const auto hi = ds_read_tr((const L4*)(tile + o1));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
};

// A threshold held on the device as bf16 or fp32 (the model's buffer, read in
// place).
__device__ __forceinline__ float load_thres(const void* p, bool bf16_value) {
  return bf16_value ? (float)*static_cast<const bf16*>(p) : *static_cast<const float*>(p);
}

// Sum over the LPR lanes of a row group (butterfly, fixed order).
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int off = LPR / 2; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

__device__ __forceinline__ float bfr(float x) { return (float)(bf16)x; }

// Fused attention epilogue of one (token, head) row of D elements, held by D/8
// consecutive lanes (lane c owns elements 8c..8c+7), with the eager bf16
// rounding points of the reference (logo/modules/layernorm.py:17-22,
// logo/layers/logo.py:180-181, :225-226, :256-258):
//   Ln  = bf16(w_l * bf16(L * rsqrt(mean(L^2) + eps)))      (same for G)
//   g'  = gate < thres ? 0 : gate
//   out = bf16(bf16(bf16(1 - g') * Ln) + bf16(g' * Gn))
// Every lane of the group must call it (the sums are lane shuffles); the
// result is this lane's 8 elements.
template <int D>
__device__ __forceinline__ bf16x8 epi_fwd_chunk(const bf16x8 lv, const bf16x8 gv, float gate, float thres,
                                                const bf16* w_l, const bf16* w_g, float eps, int c) {
  // Every eager bf16 op of the reference rounds its result; without this the
  // compiler contracts bf16(om * ln) + b into one fma and skips a rounding.
#pragma clang fp contract(off)
  constexpr int LPR = D / 8;
  float ssl = 0.f, ssg = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    ssl = fmaf((float)lv[e], (float)lv[e], ssl);
    ssg = fmaf((float)gv[e], (float)gv[e], ssg);
  }
  ssl = group_sum<LPR>(ssl);
  ssg = group_sum<LPR>(ssg);
  const float rl = rsqrtf(ssl / (float)D + eps);
  const float rg = rsqrtf(ssg / (float)D + eps);
  const float gp = gate < thres ? 0.f : gate;
  const float om = bfr(1.f - gp);
  const bf16x8 wl = *reinterpret_cast<const bf16x8*>(w_l + 8 * c);
  const bf16x8 wg = *reinterpret_cast<const bf16x8*>(w_g + 8 * c);
  bf16x8 o;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float ln = bfr((float)wl[e] * bfr((float)lv[e] * rl));
    const float gn = bfr((float)wg[e] * bfr((float)gv[e] * rg));
    o[e] = (bf16)(bfr(om * ln) + bfr(gp * gn));
  }
  return o;
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

// lower_bound_i32 by a whole wave, 64 probes per round (about log64 of the
// range in dependent loads instead of log2): every lane must call it with the
// same arguments, and every lane gets the result.
__device__ __forceinline__ int wave_lower_bound(const int32_t* arr, int lo, int hi, int x) {
  const int lane = threadIdx.x & 63;
  while (hi - lo > 64) {
    const int stride = (hi - lo + 63) >> 6;
    const int idx = lo + stride * (lane + 1) - 1;  // the last element of chunk `lane`
    const bool ge = idx >= hi || arr[idx] >= x;
    const unsigned long long m = __ballot(ge);
    if (m == 0) return hi;
    const int j0 = __builtin_ctzll(m);  // the first chunk whose last element is >= x
    lo += stride * j0;
    hi = min(hi, lo + stride);
  }
  const bool ge = lo + lane < hi && arr[lo + lane] >= x;
  const unsigned long long m = __ballot(ge);
  return m == 0 ? hi : lo + __builtin_ctzll(m);
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
