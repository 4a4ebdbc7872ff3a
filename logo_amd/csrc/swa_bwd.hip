// Sliding-window causal attention backward for gfx950: dq, dk and dv of the
// local branch (flash-attn window_size=(w, w), causal=True over every row, as
// called by logo/layers/utils.py:144-147, :166-178) in one pass, for windows
// of at most 128 keys, dense rows, HQ == H.
//
// Row p sees keys [p - w, p] of its segment, so a block of 128 keys is seen
// by rows [128 j, 128 j + 127 + w]: four 64-row steps, two of which the next
// block sees again.  The generic dq and dk/dv kernels each start one
// workgroup per tile with its own prologue, epilogue and exposed load
// latency, read q, dO, K and V twice between them and compute S and dP twice.
// Here one persistent workgroup per CU walks a contiguous run of key blocks:
//   * each wave owns 32 keys of the block: V in registers, K in the block's
//     LDS tile (also dQ's operand), dK and dV in AGPRs, stored once when the
//     walk leaves the block; the next block's K (global -> LDS) and V
//     (global -> registers) are loaded during this one;
//   * the 64-row steps stream through two LDS stages (q, dO, lse, delta),
//     the next step's copy in flight while this one computes (step r of a
//     block uses stage r % 2, so every LDS address is a lane register plus
//     a constant);
//   * each wave computes S, P, dP and dS for its keys and the step's visible
//     32-row halves, accumulates dV and dK, and writes dS^T (bf16) to LDS;
//     after a barrier every wave computes one 32-column slice of dQ = dS K
//     from dS^T and the block's K tile (both read transposed);
//   * a step's dQ is finished by the two blocks that see it: the first
//     leaves its part in AGPRs, the next adds its own and stores.  A
//     workgroup whose run starts inside a sequence first recomputes the
//     previous block's part of its first two steps (S, dP, dS and dQ only),
//     and leaves the last two steps of its run's last block to the workgroup
//     after it, so every dQ row is stored by exactly one workgroup and no
//     partial crosses workgroups.
// Results follow the generic kernels: P = exp2(S c - lse) with the forward's
// log2-domain lse, dS = P (dP - delta), dV = P^T dO, dK = scale dS^T Q,
// dQ = scale dS K, fp32 accumulation, bf16 stores.  delta comes from the
// delta kernel.
#include "sq_attn.hpp"

namespace logo {

constexpr int kSwbMaxWindow = 128;

// LDS, bytes: q tiles of the two stages, then their dO tiles (all four within
// the 64 KB reach of the DS instruction offset at D = 128), lse / delta of the
// stages, two K buffers of 128 keys (64-row kSwz tiles), and dS^T
// [128 keys][64 rows] (128-byte rows, swizzled as below).
template <int D>
struct SwbLayout {
  static constexpr int TILE = 64 * D * 2;
  static constexpr int q(int b) { return b * TILE; }
  static constexpr int dout(int b) { return (2 + b) * TILE; }
  static constexpr int lse(int b) { return 4 * TILE + b * 512; }
  static constexpr int delta(int b) { return lse(b) + 256; }
  static constexpr int kbuf(int b) { return 4 * TILE + 1024 + b * 2 * TILE; }
  static constexpr int ds() { return 8 * TILE + 1024; }
  static constexpr int BYTES = ds() + 128 * 64 * 2;
};

// dS^T swizzle: the 8-byte chunk c of row r is stored at chunk c ^ swb_dsw(r).
// Writes (a wave's 32 rows, one chunk each, 32 lanes a cycle): the 16 rows of
// one parity take 16 distinct chunks, so the 32 lanes hit 64 distinct banks.
// Transposed reads (rows 4a .. 4a+3, 8 consecutive chunks each): the two
// rows of each parity land in opposite 8-chunk halves, again 64 banks.
__device__ __forceinline__ int swb_dsw(int r) { return ((r >> 2) & 7) | (((r >> 1) & 1) << 3); }

// dQ k-steps (16 keys) of step r's half q that a 128-key window can reach:
// keys [64 r + 32 q - 128, 64 r + 32 q + 31] within the block.
constexpr int swb_klo(int r, int q) {
  return (64 * r + 32 * q - kSwbMaxWindow > 0 ? 64 * r + 32 * q - kSwbMaxWindow : 0) >> 4;
}
constexpr int swb_khi(int r, int q) { return (64 * r + 32 * q + 31 < 127 ? 64 * r + 32 * q + 31 : 127) >> 4; }

// A key block of the walk: head, block index in its segment and the
// segment's block count, start and length (all workgroup-uniform).
struct SwbBlock {
  int h, j, nt, bos, seqlen;
};

__device__ __forceinline__ SwbBlock swb_block(const AttnArgs& a, const int32_t* cu_tk, int ntk, int u) {
  SwbBlock b;
  b.h = u / ntk;
  const int tile = u - b.h * ntk;
  const int s = seg_of(cu_tk, a.nseq, tile);
  b.j = tile - cu_tk[s];
  b.nt = cu_tk[s + 1] - cu_tk[s];
  b.bos = a.cu[s];
  b.seqlen = a.cu[s + 1] - b.bos;
  return b;
}

// The block after b (unit u + 1): the next block of the segment needs no
// memory reads; only a new segment or head searches the tile prefixes.
__device__ __forceinline__ SwbBlock swb_next(const AttnArgs& a, const int32_t* cu_tk, int ntk, int u,
                                             const SwbBlock& b) {
  if (b.j + 1 < b.nt) {
    SwbBlock n = b;
    n.j += 1;
    return n;
  }
  return swb_block(a, cu_tk, ntk, u + 1);
}

// 64 lanes x 4 bytes global -> LDS (buffer_load_dword ... lds), as
// buf_load_lds16 in common.hpp.
__device__ __forceinline__ void buf_load_lds4(__amdgpu_buffer_rsrc_t r, void* lds, uint32_t voff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 4, voff, 0, 0, 0);
}

// Keeps memory accesses on their side of this point (the vmcnt accounting
// below relies on the issue order of the copies, loads and stores).
__device__ __forceinline__ void mem_fence_compiler() { asm volatile("" ::: "memory"); }

// Step r (rows 128 j + 64 r ..) of block b exists and sees some key of the
// block; a warm-up block runs its last two steps only.  The steps present
// in a block are consecutive.
__device__ __forceinline__ bool swb_present(const SwbBlock& b, int r, bool warm, int w) {
  return !(warm && r < 2) && 128 * b.j + 64 * r < b.seqlen && 64 * r <= 127 + w;
}

// Transposed operand reads (ds_read_b64_tr_b16) of one 32-column group dt,
// chosen at run time, of 64-row tiles with NC columns in layout KIND: lane
// (i, g) gets T[r0 + 4g + e][32 dt + i], then T[r0 + 8 + 4g + e][32 dt + i]
// (the k order of TileReader::tr).
template <int NC, int KIND>
struct TrCol {
  using Geo = TileGeom<NC, KIND>;
  int o0, o1;  // byte offsets for r0 = 0
  __device__ __forceinline__ void init(int dt) {
    const int l = threadIdx.x & 63, g = l >> 5, G = l >> 4, j = l & 15;
    const int col = 32 * dt + 16 * (G & 1) + 4 * (j & 3);
    const int row = 4 * g + (j >> 2);
    o0 = 2 * (Geo::off(row, col >> 3) + (col & 7));
    o1 = 2 * (Geo::off(row + 8, col >> 3) + (col & 7));
  }
  // tile: byte address of the tile; r0 a multiple of 16
  __device__ __forceinline__ bf16x8 tr(uint32_t tile, int r0) const {
    using P = const lds_bf16x4*;
    const auto lo = ds_read_tr((P)(uintptr_t)(tile + 2 * r0 * Geo::RS + o0));
    const auto hi = ds_read_tr((P)(uintptr_t)(tile + 2 * r0 * Geo::RS + o1));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
};

// Sets an AGPR accumulator to zero with an MFMA of zero operands (C = 0):
// clearing it by register writes would have the compiler keep a 16-register
// zero vector alive to copy from.  Ordered with the asm MFMAs like one of them.
__device__ __forceinline__ void zero_acc(f32x16& d, const bf16x8& z) {
  asm volatile("s_nop 2\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %1, 0" : "=a"(d) : "v"(z));
}

// Transposed reads (ds_read_b64_tr_b16) of column group dt (32 rows of the
// step) of the dS^T tile: lane (i, g) gets T[r0 + 4g + e][32 dt + i], then
// T[r0 + 8 + 4g + e][32 dt + i] (the k order of TileReader::tr).  With r0 a
// multiple of 16, swb_dsw(r0 + x) = swb_dsw(x) ^ 4 (r0 / 16 & 1), which flips
// bit 5 of the lane's byte offset for odd r0 / 16.
struct SwbDsCol {
  int o0, o1;  // byte offsets for r0 = 0
  __device__ __forceinline__ void init(int dt) {
    const int l = threadIdx.x & 63, g = l >> 5, G = l >> 4, j = l & 15;
    const int c = 8 * dt + 4 * (G & 1) + (j & 3);
    const int r = 4 * g + (j >> 2);
    o0 = 128 * r + 8 * (c ^ swb_dsw(r));
    o1 = 128 * (r + 8) + 8 * (c ^ swb_dsw(r + 8));
  }
  template <int R0>
  __device__ __forceinline__ bf16x8 tr(uint32_t tile) const {
    constexpr int F = (R0 / 16 & 1) ? 32 : 0;
    using P = const lds_bf16x4*;
    const auto lo = ds_read_tr((P)(uintptr_t)(tile + 128 * R0 + (o0 ^ F)));
    const auto hi = ds_read_tr((P)(uintptr_t)(tile + 128 * R0 + (o1 ^ F)));
    return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  }
};

// Wait states after the last MFMA into these accumulators, tied to them so
// that every read of theirs follows (the reads cannot be scheduled above it).
__device__ __forceinline__ void drain_acc(f32x16& x, f32x16& y) {
  asm volatile("s_nop 15\n\ts_nop 15" : "+a"(x), "+a"(y));
}
__device__ __forceinline__ void drain_acc(f32x16& x) { asm volatile("s_nop 15\n\ts_nop 15" : "+a"(x)); }

// This wave's vector memory operations and LDS accesses complete, then the
// workgroup barrier (__syncthreads() would add a release fence: the same
// waits, plus an L2 write-back on this multi-L2 part).
__device__ __forceinline__ void swb_barrier() { asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory"); }
// The same with up to N vector-memory operations (the youngest) still in flight.
template <int N>
__device__ __forceinline__ void swb_barrier_vm() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}
__device__ __forceinline__ void swb_lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

template <int D>
__global__ __launch_bounds__(256) LOGO_OCC_DKV void swa_bwd_kernel(const AttnArgs a) {
  using L = SwbLayout<D>;
  constexpr int DS = D / 16, DT = D / 32;
  constexpr int QT = DT / 2;  // dQ tiles per wave and step: 2 halves x DT over 4 waves
  char* const sm = logo_smem;
  auto ptr = [&](int off) { return reinterpret_cast<bf16*>(sm + off); };
  const uint32_t sm_addr = (uint32_t)(uintptr_t)sm;

  // the wave index as a scalar: the per-wave visibility tests are then
  // uniform branches (a divergent one makes the compiler copy the asm
  // accumulators through VGPRs at its joins)
  const int tid = threadIdx.x, wave = __builtin_amdgcn_readfirstlane(tid >> 6), l = tid & 63, i = l & 31, g = l >> 5;
  const int W = a.window;
  const float c = a.scale_log2;
  const int32_t* cu_tk = a.meta + kMetaHdr + 2 * (a.nseq + 1);
  const int ntk = a.meta[2];
  const int nunits = ntk * a.h;
  const int u0 = (int)((int64_t)blockIdx.x * nunits / gridDim.x);
  const int u1 = (int)((int64_t)(blockIdx.x + 1) * nunits / gridDim.x);
  if (u0 >= u1) return;

  TileReader<D, kSwz> rd;
  rd.init();
  // dQ tile t of this wave: rows of half qq_of(t), columns 32 dt_w ..
  const int dt_w = D == 128 ? wave : (wave & 1);
  auto qq_of = [&](int t) { return D == 128 ? t : (wave >> 1); };
  TrCol<D, kSwz> kcol;  // K^T reads, column group dt_w
  kcol.init(dt_w);
  SwbDsCol scol[QT];  // dS^T reads: the rows of each dQ tile are its columns
#pragma unroll
  for (int t = 0; t < QT; ++t) scol[t].init(qq_of(t));
  // this wave's 32 keys in a K buffer (byte offset); its dS^T row (key
  // 32 wave + i) and the lane's part of the swizzled chunk index
  const int kw_off = 2 * ((wave >> 1) * 64 * D + 32 * (wave & 1) * D);
  const int ds_row = 128 * (32 * wave + i);
  const int ds_x = g ^ swb_dsw(32 * wave + i);
  TileBufDma<D> dma;
  dma.init(a.hq * D);

  const bf16x8 zero8 = {};
  f32x16 dka[DT], dva[DT], dqa[2][QT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) {
    zero_acc(dka[dt], zero8);
    zero_acc(dva[dt], zero8);
  }
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int t = 0; t < QT; ++t) zero_acc(dqa[s][t], zero8);
  bf16x8 vreg[DS], vnext[DS];

  // Step r of block b into stage B: q and dO rows (two 64-row tiles) and the
  // rows' lse (wave 0) and delta (wave 1), all global -> LDS copies, rows
  // past the segment clamped to its last row (masked).
  auto issue_tile = [&](const SwbBlock& b, int r, auto buf_c) __attribute__((always_inline)) {
    constexpr int B = decltype(buf_c)::value;
    const int row0 = 128 * b.j + 64 * r;
    const int last = min(63, b.seqlen - 1 - row0);
    const int64_t tok = b.bos + row0;
    const bf16* qr = a.q + (tok * a.hq + b.h) * D;
    const bf16* dr = a.dout + (tok * a.hq + b.h) * D;
    if (last == 63) {
      dma.issue(ptr(L::q(B)), qr);
      dma.issue(ptr(L::dout(B)), dr);
    } else {
      dma.issue_clamped(ptr(L::q(B)), qr, last);
      dma.issue_clamped(ptr(L::dout(B)), dr, last);
    }
    if (wave < 2) {
      const float* src = (wave == 0 ? a.lse : a.delta) + (int64_t)b.h * a.n + tok;
      const auto rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(src), (short)0, (last + 1) * 4,
                                                        kBufRsrcWord3);
      buf_load_lds4(rs, sm + (wave == 0 ? L::lse(B) : L::delta(B)), (uint32_t)min(l, last) * 4);
    }
  };
  // K of the block's 128 keys (two 64-row tiles; keys past the segment are
  // clamped to its last key, whose scores the causal mask drops)
  auto issue_k = [&](const SwbBlock& b, int kb) __attribute__((always_inline)) {
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int start = min(128 * b.j + 64 * t, b.seqlen - 1);
      const int last = min(63, b.seqlen - 1 - start);
      const bf16* src = a.k + ((int64_t)(b.bos + start) * a.h + b.h) * D;
      bf16* dst = ptr(L::kbuf(0) + kb * 2 * L::TILE + t * L::TILE);
      if (last == 63) dma.issue(dst, src);
      else dma.issue_clamped(dst, src, last);
    }
  };
  auto load_v = [&](const SwbBlock& b, bf16x8 (&dst)[DS]) __attribute__((always_inline)) {
    const int key = 128 * b.j + 32 * wave + i;
    // keys past the segment read its last key (finite; never visible)
    const bf16* vp = a.v + ((int64_t)(b.bos + min(key, b.seqlen - 1)) * a.h + b.h) * D + 8 * g;
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) dst[ds] = *reinterpret_cast<const bf16x8*>(vp + 16 * ds);
  };

  // One step's S, P, dP, dS for this wave's keys and the step's two 32-row
  // halves h0, h1 (stage B), dV / dK +=, and dS^T to LDS (zeros when the
  // wave sees neither half; a wave that sees one computes both, the other
  // masked to zero, which costs no time: the step's critical path is two
  // halves).  The MFMAs run in eight blocks of DS slots
  //   S(h0) | dP(h0) | S(h1) | dP(h1) | dV(h0) | dK(h0) | dV(h1) | dK(h1)
  // with P = exp2(S c - lse) of h0 under blocks 1-2, dS = P (dP - delta) of
  // h0 under block 3, P of h1 under 4-5 and dS of h1 under 6; each slot's
  // LDS operands are read PF slots ahead, and scheduling fences between the
  // slots keep the VALU work under the MFMAs.  K's rows (the B operand of
  // S) come from the block's LDS tile kt, V's from registers.
  auto compute_step = [&](auto buf_c, const SwbBlock& b, int r, const bf16* kt) __attribute__((always_inline)) {
    constexpr int B = decltype(buf_c)::value;
    constexpr int NSL = 8 * DS, PF = 6;
    constexpr int IPP = 16 / (2 * DS), IPD = 16 / DS;  // P / dS items per slot
    const int R0 = 128 * b.j + 64 * r;
    const int K0 = 128 * b.j + 32 * wave;
    const bool see0 = R0 < b.seqlen && R0 <= K0 + 31 + W && R0 + 31 >= K0;
    const bool see1 = R0 + 32 < b.seqlen && R0 + 32 <= K0 + 31 + W && R0 + 63 >= K0;
    bf16x8 dbf[2][2] = {};  // dS of the halves as bf16 (zeros where not seen)
    if (see0 | see1) {
      const int key = K0 + i;
      // Row p of item (half q, j) is R0 + 32 q + rowmap(g, j) and sees key
      // iff key <= p <= min(key + W, seqlen - 1): with d = p - kb, one
      // unsigned compare (unsigned) d <= lim.  A key past the segment end
      // sees no row: kb then lies far above every row, so d wraps to a huge
      // unsigned value, and lim is 0 (min(W, seqlen - 1 - key) would be
      // negative, a huge unsigned bound).
      const bool kin = key < b.seqlen;
      const int kb = kin ? key : (1 << 30);
      const unsigned lim = kin ? (unsigned)min(W, b.seqlen - 1 - key) : 0u;
      const int d0 = R0 + 4 * g - kb;  // d of item (0, 0)
      const bf16* qb = ptr(L::q(B));
      const bf16* ob = ptr(L::dout(B));
      const f32x4* lb = reinterpret_cast<const f32x4*>(sm + L::lse(B));
      const f32x4* db = reinterpret_cast<const f32x4*>(sm + L::delta(B));
      f32x16 sacc[2], pacc[2];
      bf16x8 pbf[2][2];
      bf16x8 opA[NSL], opB[2 * DS];
      f32x4 l4[2][4], d4[2][4];
      // the LDS operands of slot T
      auto load_slot = [&](auto t_c) __attribute__((always_inline)) {
        constexpr int T = decltype(t_c)::value, BLK = T / DS, K = T % DS;
        if constexpr (BLK == 0 || BLK == 2) {
          opA[T] = rd.row(qb, 16 * BLK, K);
          opB[(BLK / 2) * DS + K] = rd.row(kt, 0, K);
        } else if constexpr (BLK == 1 || BLK == 3) {
          opA[T] = rd.row(ob, 16 * (BLK - 1), K);
        } else {
          constexpr int QQ = (BLK - 4) / 2, HH = K / DT, DTI = K % DT;
          opA[T] = rd.tr((BLK % 2 == 0) ? ob : qb, 32 * QQ + 16 * HH, DTI);
        }
      };
      // An item's inputs are anchored ahead of its slot's MFMA (which then
      // separates the anchor from the VALU op that reads them), its
      // arithmetic follows the MFMA, and pairs are packed to bf16 one slot
      // later: a VALU op right behind an anchor or an exp2 that wrote its
      // input would cost an s_nop.
      auto p_pre = [&](auto q_c, auto j_c) __attribute__((always_inline)) {
        constexpr int QQ = decltype(q_c)::value, JJ = decltype(j_c)::value;
        float sv = sacc[QQ][JJ];
        pin(sv);
        return sv;
      };
      auto p_item = [&](auto q_c, auto j_c, float sv) __attribute__((always_inline)) {
        constexpr int QQ = decltype(q_c)::value, JJ = decltype(j_c)::value;
        const bool vis = (unsigned)(d0 + (32 * QQ + 8 * (JJ / 4) + JJ % 4)) <= lim;
        // masked before the exp2 (exp2(-inf) = 0), so no VALU op reads the
        // exp2 result right behind it
        const float x = fmaf(sv, c, -l4[QQ][JJ / 4][JJ % 4]);
        float pv = fast_exp2(vis ? x : -INFINITY);
        pin(pv);
        sacc[QQ][JJ] = pv;
      };
      auto p_pack = [&](auto q_c, auto j_c) __attribute__((always_inline)) {
        constexpr int QQ = decltype(q_c)::value, JJ = decltype(j_c)::value;
        if constexpr (JJ % 2 == 1) {
          pbf[QQ][JJ / 8][JJ % 8 - 1] = (bf16)sacc[QQ][JJ - 1];
          pbf[QQ][JJ / 8][JJ % 8] = (bf16)sacc[QQ][JJ];
        }
        // a finished group stays here: sunk to its MFMA, the packing would
        // write the operand right before it
        if constexpr (JJ % 8 == 7) pin(pbf[QQ][JJ / 8]);
      };
      auto ds_pre = [&](auto q_c, auto j_c, float& pv, float& dpv) __attribute__((always_inline)) {
        constexpr int QQ = decltype(q_c)::value, JJ = decltype(j_c)::value;
        pv = sacc[QQ][JJ];
        dpv = pacc[QQ][JJ];
        pin(pv);
        pin(dpv);
      };
      auto ds_item = [&](auto q_c, auto j_c, float pv, float dpv) __attribute__((always_inline)) {
        constexpr int QQ = decltype(q_c)::value, JJ = decltype(j_c)::value;
        float dsv = pv * (dpv - d4[QQ][JJ / 4][JJ % 4]);
        pin(dsv);
        pacc[QQ][JJ] = dsv;
      };
      auto ds_pack = [&](auto q_c, auto j_c) __attribute__((always_inline)) {
        constexpr int QQ = decltype(q_c)::value, JJ = decltype(j_c)::value;
        if constexpr (JJ % 2 == 1) {
          dbf[QQ][JJ / 8][JJ % 8 - 1] = (bf16)pacc[QQ][JJ - 1];
          dbf[QQ][JJ / 8][JJ % 8] = (bf16)pacc[QQ][JJ];
        }
        if constexpr (JJ % 8 == 7) pin(dbf[QQ][JJ / 8]);
      };
      static_for<PF>([&](auto t_c) __attribute__((always_inline)) { load_slot(t_c); });
      static_for<NSL>([&](auto s_c) __attribute__((always_inline)) {
        constexpr int S = decltype(s_c)::value, BLK = S / DS, K = S % DS;
        constexpr int HH = K / DT, DTI = K % DT;
        __builtin_amdgcn_sched_barrier(0);
        // the slot's P items (blocks 1, 2, 4, 5) and dS items (blocks 3, 6)
        constexpr bool HASP = BLK == 1 || BLK == 2 || BLK == 4 || BLK == 5, HASD = BLK == 3 || BLK == 6;
        constexpr int QP = BLK >= 4, JP = HASP ? (S - DS * (1 + 3 * QP)) * IPP : 0, QD = BLK == 6, JD = K * IPD;
        float sv[IPP], pv[IPD], dpv[IPD];
        if constexpr (HASP)
          static_for<IPP>([&](auto e_c) __attribute__((always_inline)) {
            constexpr int E = decltype(e_c)::value;
            sv[E] = p_pre(std::integral_constant<int, QP>{}, std::integral_constant<int, JP + E>{});
          });
        if constexpr (HASD)
          static_for<IPD>([&](auto e_c) __attribute__((always_inline)) {
            constexpr int E = decltype(e_c)::value;
            ds_pre(std::integral_constant<int, QD>{}, std::integral_constant<int, JD + E>{}, pv[E], dpv[E]);
          });
        if constexpr (BLK == 0 || BLK == 2) {
          constexpr int QQ = BLK / 2;
          sacc[QQ] = mfma32(opA[S], opB[QQ * DS + K], K == 0 ? f32x16{} : sacc[QQ]);
        } else if constexpr (BLK == 1 || BLK == 3) {
          constexpr int QQ = BLK / 2;
          pacc[QQ] = mfma32(opA[S], vreg[K], K == 0 ? f32x16{} : pacc[QQ]);
        } else {
          // dV / dK: operands from LDS and P / dS packed at least DT slots
          // earlier; D = 128 (DT = 4) needs no leading wait states, D = 64
          // keeps them
          auto acc_mfma = [&](f32x16& acc, const bf16x8& x, const bf16x8& y) __attribute__((always_inline)) {
            if constexpr (DT >= 4) mfma32_agpr_ready(acc, x, y);
            else mfma32_agpr(acc, x, y);
          };
          if constexpr (BLK == 4) acc_mfma(dva[DTI], opA[S], pbf[0][HH]);
          else if constexpr (BLK == 5) acc_mfma(dka[DTI], opA[S], dbf[0][HH]);
          else if constexpr (BLK == 6) acc_mfma(dva[DTI], opA[S], pbf[1][HH]);
          else acc_mfma(dka[DTI], opA[S], dbf[1][HH]);
        }
        if constexpr (S + PF < NSL) load_slot(std::integral_constant<int, S + PF>{});
        // lse / delta of items 4m .. 4m+3 of a half, two slots before the
        // first of them is needed (P of half q from slot DS (1 + 3q), dS from
        // slot DS (3 + 3q))
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            if (S == DS * (1 + 3 * q) + 4 * m / IPP - 2) l4[q][m] = lds_load(lb + 8 * q + 2 * m + g);
            if (S == DS * (3 + 3 * q) + 4 * m / IPD - 2) d4[q][m] = lds_load(db + 8 * q + 2 * m + g);
          }
        if constexpr (HASP)
          static_for<IPP>([&](auto e_c) __attribute__((always_inline)) {
            constexpr int E = decltype(e_c)::value;
            p_item(std::integral_constant<int, QP>{}, std::integral_constant<int, JP + E>{}, sv[E]);
          });
        if constexpr (HASD)
          static_for<IPD>([&](auto e_c) __attribute__((always_inline)) {
            constexpr int E = decltype(e_c)::value;
            ds_item(std::integral_constant<int, QD>{}, std::integral_constant<int, JD + E>{}, pv[E], dpv[E]);
          });
        // the previous slot's items, packed (no item is formed in block 0 or
        // 7, so the packs stay inside the step)
        if constexpr (S >= 1) {
          constexpr int LS = S - 1, LB = LS / DS, LK = LS % DS;
          if constexpr (LB == 1 || LB == 2 || LB == 4 || LB == 5)
            static_for<IPP>([&](auto e_c) __attribute__((always_inline)) {
              constexpr int LQ = LB >= 4;
              p_pack(std::integral_constant<int, LQ>{},
                     std::integral_constant<int, (LS - DS * (1 + 3 * LQ)) * IPP + decltype(e_c)::value>{});
            });
          if constexpr (LB == 3 || LB == 6)
            static_for<IPD>([&](auto e_c) __attribute__((always_inline)) {
              ds_pack(std::integral_constant<int, LB == 6>{}, std::integral_constant<int, LK * IPD + decltype(e_c)::value>{});
            });
        }
      });
      __builtin_amdgcn_sched_barrier(0);
    }
    // dS^T row = key 32 wave + i of the block, columns 32 qq + 8 m + 4 g + e:
    // 8-byte chunk 8 qq + 2 m + g, swizzled (written after the branch: an
    // else branch beside the accumulating one makes the compiler copy the
    // accumulators between registers inside it)
    char* const st = sm + L::ds() + ds_row;
#pragma unroll
    for (int qq = 0; qq < 2; ++qq)
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        const bf16x8 src = dbf[qq][m >> 1];
        *reinterpret_cast<bf16x4*>(st + 8 * ((8 * qq + 2 * m) ^ ds_x)) =
            (m & 1) ? __builtin_shufflevector(src, src, 4, 5, 6, 7) : __builtin_shufflevector(src, src, 0, 1, 2, 3);
      }
  };

  // dQ of step R's rows += dS K.  The k-steps are those a 128-key window can
  // reach (keys [row - 128, row + 31] of the half): exact for w = 128, a
  // superset for smaller windows, whose extra dS^T entries are zeros.
  // Compile-time bounds keep the MFMA sequence free of branches; operands
  // are read two MFMAs ahead.
  auto dq_phase = [&](auto r_c, uint32_t kbuf_addr) __attribute__((always_inline)) {
    constexpr int R = decltype(r_c)::value, SET = R & 1;
    // tile 0: half 0 (D = 128) or the wave's half (D = 64: bounds over both)
    constexpr int LO0 = swb_klo(R, 0), HI0 = swb_khi(R, QT == 2 ? 0 : 1);
    constexpr int LO1 = swb_klo(R, 1), HI1 = swb_khi(R, 1);
    constexpr int N0 = HI0 - LO0 + 1, N1 = QT == 2 ? HI1 - LO1 + 1 : 0;
    constexpr int NM = N0 + N1, PFQ = 2;
    bf16x8 ka[NM], sb[NM];
    auto load = [&](auto m_c) __attribute__((always_inline)) {
      constexpr int M = decltype(m_c)::value, T = M < N0 ? 0 : 1;
      constexpr int KS = M < N0 ? LO0 + M : LO1 + M - N0;
      ka[M] = kcol.tr(kbuf_addr + (KS >> 2) * L::TILE, 16 * (KS & 3));
      sb[M] = scol[T].template tr<16 * (KS & 3)>(sm_addr + L::ds() + (KS >> 2) * 64 * 128);
    };
    static_for<(PFQ < NM ? PFQ : NM)>([&](auto m_c) __attribute__((always_inline)) { load(m_c); });
    static_for<NM>([&](auto m_c) __attribute__((always_inline)) {
      constexpr int M = decltype(m_c)::value, T = M < N0 ? 0 : 1;
      __builtin_amdgcn_sched_barrier(0);
      mfma32_agpr_ready(dqa[SET][T], ka[M], sb[M]);  // operands straight from LDS
      if constexpr (M + PFQ < NM) load(std::integral_constant<int, M + PFQ>{});
    });
    __builtin_amdgcn_sched_barrier(0);
  };
  // store the finished dQ rows of step R, then clear its accumulators
  auto store_dq = [&](auto r_c, const SwbBlock& b) __attribute__((always_inline)) {
    constexpr int R = decltype(r_c)::value, SET = R & 1;
    if constexpr (QT == 2) drain_acc(dqa[SET][0], dqa[SET][1]);
    else drain_acc(dqa[SET][0]);
#pragma unroll
    for (int t = 0; t < QT; ++t) {
      // Lane (i, g) holds columns 32 dt + 8 m + 4 g + e of row i.  For each
      // pair m, m + 1 the two lanes of a row trade one half (permlane32
      // swap), so lane g = 0 stores columns 8 m .. 8 m + 7 and lane g = 1
      // columns 8 m + 8 .. 8 m + 15: 16 bytes a lane, 32 contiguous bytes a
      // row per store.
      const int row = 128 * b.j + 64 * R + 32 * qq_of(t) + i;
      bf16* dst = a.dq + ((int64_t)(b.bos + min(row, b.seqlen - 1)) * a.hq + b.h) * D + 32 * dt_w + 8 * g;
#pragma unroll
      for (int m = 0; m < 4; m += 2) {
        bf16x4 lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = (bf16)(dqa[SET][t][4 * m + e] * a.scale);
          hi[e] = (bf16)(dqa[SET][t][4 * m + 4 + e] * a.scale);
        }
        const u32x2 lo2 = __builtin_bit_cast(u32x2, lo), hi2 = __builtin_bit_cast(u32x2, hi);
        // g = 0 gives its columns 8 m + 8 .. (hi), g = 1 its 8 m + 4 .. (lo)
        u32x2 x = g ? lo2 : hi2, y;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
          const auto r = __builtin_amdgcn_permlane32_swap(x[k], x[k], false, false);
          y[k] = g ? r[0] : r[1];
        }
        const u32x4 v = g ? u32x4{y[0], y[1], hi2[0], hi2[1]} : u32x4{lo2[0], lo2[1], y[0], y[1]};
        if (row < b.seqlen) *reinterpret_cast<u32x4*>(dst + 8 * m) = v;
      }
      zero_acc(dqa[SET][t], zero8);
    }
  };
  // Store dK / dV of the block (keep: not a warm-up block, whose sums are
  // only cleared), then clear them.  The bf16 tiles go through LDS that is
  // free at the block's end (its K buffer: dK; stage 1's q and dO tiles:
  // dV), so that each global store writes 16 contiguous bytes a lane and a
  // whole 256-byte row per 16 lanes; stored straight from the MFMA layout,
  // every store instruction wrote 16-byte pieces of 32 rows.
  auto store_kv = [&](const SwbBlock& b, bool keep, int kbuf) __attribute__((always_inline)) {
    using G = TileGeom<D, kSwz>;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) drain_acc(dka[dt], dva[dt]);
    if (keep) {
      // lane indices anchored here: the offsets below are recomputed per
      // block instead of being hoisted out of the walk (registers held
      // through every step)
      int lane = tid;
      pin(lane);
      const int row = 32 * (wave & 1) + (lane & 31), gl = (lane >> 5) & 1;
      bf16* const kt2 = ptr(L::kbuf(0) + kbuf * 2 * L::TILE + (wave >> 1) * L::TILE);
      bf16* const vt2 = ptr((wave >> 1) == 0 ? L::q(1) : L::dout(1));
#pragma unroll
      for (int dt = 0; dt < DT; ++dt)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          bf16x4 kv, vv;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            kv[e] = (bf16)(dka[dt][4 * m + e] * a.scale);
            vv[e] = (bf16)dva[dt][4 * m + e];
          }
          *reinterpret_cast<bf16x4*>(kt2 + G::off(row, 4 * dt + m) + 4 * gl) = kv;
          *reinterpret_cast<bf16x4*>(vt2 + G::off(row, 4 * dt + m) + 4 * gl) = vv;
          __builtin_amdgcn_sched_barrier(0);
        }
      swb_lds_barrier();
      constexpr int CH = D / 8, RPT = 64 * CH / 256;
      const int c = lane % CH, r0 = lane / CH;
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const bf16* src = t < 2 ? ptr(L::kbuf(0) + kbuf * 2 * L::TILE + t * L::TILE) : ptr(t == 2 ? L::q(1) : L::dout(1));
        bf16* const dst = t < 2 ? a.dk : a.dv;
#pragma unroll
        for (int k = 0; k < RPT; ++k) {
          const int r = r0 + (256 / CH) * k;
          const int key = 128 * b.j + 64 * (t & 1) + r;
          const u32x4 val = lds_load(reinterpret_cast<const u32x4*>(src + G::off(r, c)));
          if (key < b.seqlen)
            *reinterpret_cast<u32x4*>(dst + ((int64_t)(b.bos + key) * a.h + b.h) * D + 8 * c) = val;
        }
        __builtin_amdgcn_sched_barrier(0);  // a tile at a time: few registers live
      }
      swb_lds_barrier();  // the LDS is read: the next block's copies may land there
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      zero_acc(dka[dt], zero8);
      zero_acc(dva[dt], zero8);
    }
  };

  // The walk: a warm-up block (the one before u0: S, dP, dS and dQ of its
  // last two steps) when the run starts inside a sequence and the window
  // reaches back.
  SwbBlock cur = swb_block(a, cu_tk, ntk, u0);
  const bool warm = cur.j > 0 && W >= 1;
  int u = u0;
  if (warm) {
    cur.j -= 1;
    u = u0 - 1;
  }
  issue_k(cur, 0);
  load_v(cur, vnext);
  issue_tile(cur, warm ? 2 : 0, std::integral_constant<int, 0>{});  // step 0 or 2: stage 0
  swb_barrier();
#pragma unroll
  for (int ds = 0; ds < DS; ++ds) vreg[ds] = vnext[ds];
  int kb = 0;
  // vector-memory loads a wave issues for the next block (K copies, V rows)
  constexpr int N_KV = 2 * TileBufDma<D>::BLOCKS + DS;

  for (; u < u1; ++u) {
    const bool wblk = u < u0;
    const bool has_nxt = u + 1 < u1;
    const SwbBlock nxt = has_nxt ? swb_next(a, cu_tk, ntk, u, cur) : cur;
    const uint32_t kbuf_addr = sm_addr + L::kbuf(0) + kb * 2 * L::TILE;
    const bf16* kt = reinterpret_cast<const bf16*>(sm + L::kbuf(0) + kb * 2 * L::TILE + kw_off);
    static_for<4>([&](auto r_c) __attribute__((always_inline)) {
      constexpr int R = decltype(r_c)::value, B = R & 1;
      using Cur = std::integral_constant<int, B>;
      using Nxt = std::integral_constant<int, B ^ 1>;
      if (!swb_present(cur, R, wblk, W)) return;
      // Issue order (vector memory): the previous step's stores (already
      // issued), this step's prefetch, then on the block's first step the
      // next block's K / V.  Loads complete in issue order, so the end of
      // the step waits until only those K / V loads may be outstanding
      // (vmcnt(N_KV)); stores in between do not matter (the younger loads
      // alone keep the count above N_KV while the prefetch is in flight).
      // Prefetch into the other stage: step R + 1 of this block, or step 0
      // (stage 0) of the next block when this is stage 1; after an even last
      // step that copy waits for the end of the step.
      const bool pf_here = R < 3 && swb_present(cur, R + 1, wblk, W);
      const bool pf_next = !pf_here && has_nxt && B == 1;
      mem_fence_compiler();
      if (pf_here) issue_tile(cur, R + 1, Nxt{});
      else if (pf_next) issue_tile(nxt, 0, Nxt{});
      mem_fence_compiler();
      const bool kv = R == (wblk ? 2 : 0) && has_nxt;
      if (kv) {
        issue_k(nxt, kb ^ 1);
        load_v(nxt, vnext);
      }
      mem_fence_compiler();
      // (steps 2, 3 of the run's last block are finished by the next
      // workgroup: what this one sums for them is never stored)
      compute_step(Cur{}, cur, R, kt);
      swb_lds_barrier();  // dS^T complete
      dq_phase(r_c, kbuf_addr);
      // next stage landed; this stage, dS^T and K free.  The block's last
      // step waits for everything (the next block's K is read next).
      if (kv && pf_here) swb_barrier_vm<N_KV>();
      else swb_barrier();
      // rows of steps 0, 1 are finished (the previous block's part came first)
      if (R < 2 && !wblk) store_dq(r_c, cur);
      if (!pf_here && has_nxt && B == 0) {
        mem_fence_compiler();
        issue_tile(nxt, 0, std::integral_constant<int, 0>{});
        swb_barrier();
      }
    });
    // the next block's V: its loads completed at the last step's barrier, so
    // the wait the compiler places on them here is free; after the stores
    // below it would wait for those stores too (anchored here, the copy
    // cannot sink below them)
#pragma unroll
    for (int ds = 0; ds < DS; ++ds) {
      vreg[ds] = vnext[ds];
      pin(vreg[ds]);
    }
    store_kv(cur, !wblk, kb);
    kb ^= 1;
    cur = nxt;
  }
}

template <int D>
static int launch_swa_bwd(const AttnArgs& a, hipStream_t st) {
  const int64_t ntmax = (a.n + kBKV - 1) / kBKV + a.nseq;
  const int cus = device_cus();
  LOGO_REQUIRE(cus > 0, "device query failed");
  const int64_t units = ntmax * a.h;
  const unsigned grid = (unsigned)(units < cus ? units : cus);
  auto kern = swa_bwd_kernel<D>;
  LOGO_HIP_CHECK(allow_smem(kern, (size_t)SwbLayout<D>::BYTES));
  hipLaunchKernelGGL(kern, dim3(grid), dim3(256), (size_t)SwbLayout<D>::BYTES, st, a);
  LOGO_LAUNCH_CHECK("swa_bwd_kernel");
  return LOGO_OK;
}

bool swa_bwd_applies(const AttnArgs& a, bool sparse, bool half) {
  return !sparse && !half && a.g == 1 && a.window >= 0 && a.window <= kSwbMaxWindow;
}

int swa_launch_bwd(const AttnArgs& a, hipStream_t st, int d) {
  return d == 128 ? launch_swa_bwd<128>(a, st) : launch_swa_bwd<64>(a, st);
}

}  // namespace logo
