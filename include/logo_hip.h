/*
 * logo_hip.h -- C ABI of the MI355X (gfx950) LoGo attention hot path.
 *
 * Every entry point takes raw device pointers, element counts and a HIP
 * stream (passed as void*), launches asynchronously on that stream, and
 * returns LOGO_OK or an error code; logo_last_error() gives the message of
 * the calling thread's last failure.  No entry point allocates device memory:
 * the caller passes every output and workspace buffer.
 *
 * Tensor layouts follow the reference's packed varlen convention with the
 * batch axis (B = 1) dropped (logo/ops/selected_full_attn.py:505-514):
 *   q [N, HQ, D], k [N, H, D], v [N, H, D], o [N, HQ, D]  (bf16, contiguous)
 *   selection: uint8 [N] (shared by all heads, the reference API) or
 *              uint8 [N, HQ] (per-(token, head) extension); "lanes" = 1 or HQ.
 *   cu: int32 [nseq + 1], cu[0] = 0, cu[nseq] = N, non-decreasing.
 *
 * Compaction metadata ("meta"), int32, one block of LOGO_META_STRIDE(nseq)
 * per lane:
 *   [0] Sq   selected rows           [1] NTq  query tiles of LOGO_BQ rows
 *   [2] NTk  key tiles of LOGO_BKV   [3] N    [4] nseq   [5..7] reserved
 *   [8 ...]                      cu_q  [nseq+1]  (logo/ops/common.py:94-96)
 *   [8 +   (nseq+1) ...]         prefix of ceil(count_s / LOGO_BQ)
 *   [8 + 2*(nseq+1) ...]         prefix of ceil(len_s / LOGO_BKV)
 * Row lists: q_idx int64 [lanes, N], pos int32 [lanes, N]; entries
 * [0, Sq) of each lane are the rows (logo/ops/common.py:90-93), entries
 * [Sq, N) are written zero.
 * lse / delta: float32 [HQ, N] indexed by compacted row (log2 domain lse,
 * logo/ops/selected_full_attn.py:118-119); the forward writes zero to the lse
 * rows past the lane's rows, delta rows past Sq are left unwritten.
 */
#ifndef LOGO_HIP_H_
#define LOGO_HIP_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define LOGO_OK 0
#define LOGO_EINVAL 1
#define LOGO_EHIP 2

#define LOGO_BQ 128
#define LOGO_BKV 128
#define LOGO_META_HDR 8
#define LOGO_META_STRIDE(nseq) (LOGO_META_HDR + 3 * ((nseq) + 1))

#define LOGO_DTYPE_BF16 0
#define LOGO_DTYPE_F32 1
#define LOGO_DTYPE_F16 2

/* Message of the calling thread's last error ("" if none). */
const char* logo_last_error(void);

/* ABI version of this library (7: logo_read_calibration's nontemporal flag; 6: logo_head_linear_grad_acc;
   5: head dim 256, fp32, logo_sq_generic). */
int logo_abi_version(void);

/*
 * Streaming-read calibration (no counterpart in the reference): reads `bytes`
 * (a multiple of 16) of the 16-byte aligned device buffer `buf` once with a
 * grid of `grid` 256-thread workgroups, for timing the read bandwidth the
 * part delivers in practice (the ceiling the decode kernel's bandwidth is
 * compared with); `nontemporal` != 0 uses non-temporal loads, as the decode
 * kernel's cache reads do.  `sink` is device memory of at least grid * 4
 * bytes, which it leaves unchanged unless a workgroup's XOR of its words hits
 * a sentinel.
 */
int logo_read_calibration(const void* buf, size_t bytes, void* sink, int grid, int nontemporal, void* stream);

/* Bytes of workspace logo_compact needs. */
size_t logo_compact_workspace_bytes(int64_t n_tokens, int lanes);

/*
 * Row compaction (wavefront ballot + prefix sum): selected rows per lane in
 * ascending token order, their positions inside their segment, cu_q, and the
 * tile prefixes in `meta`.  Bit-exact restatement of build_selection,
 * logo/ops/common.py:71-107 (q_idx :90, seg :92, pos_ids :93, cu_q :94-96).
 */
int logo_compact(const uint8_t* selection, int64_t n_tokens, int lanes,
                 const int32_t* cu, int nseq, int64_t* q_idx, int32_t* pos,
                 int32_t* meta, void* workspace, void* stream);

/*
 * logo_compact without the workspace argument: no counterpart in the
 * reference.  For callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving loops).  The per-chunk counts go to a
 * fixed device array of LOGO_COMPACT_SCRATCH_INTS int32 (256 KB, held by each
 * GPU the library runs on until the process ends), so lanes *
 * ceil(n_tokens / 4096) must not exceed it (LOGO_EINVAL otherwise, e.g. up to
 * 16.7M tokens with 16 lanes).  Every call on one GPU shares that array, so
 * only one call per GPU may be in flight at a time: calls that overlap on
 * one GPU (different streams, or threads) race and corrupt each other's
 * q_idx.  Calls queued on one stream run in order and do not overlap.
 * Outputs and their meaning are those of logo_compact.
 */
#define LOGO_COMPACT_SCRATCH_INTS 65536
int logo_compact_noalloc(const uint8_t* selection, int64_t n_tokens, int lanes,
                         const int32_t* cu, int nseq, int64_t* q_idx, int32_t* pos,
                         int32_t* meta, void* stream);

/*
 * Metadata for dense attention over every row (cu_q = cu, Sq = N), used by
 * the sliding-window branch and the all-ones ("flash") global branch
 * (logo/layers/utils.py:107-234, logo/ops/dense_full_attn.py:12-22).
 */
int logo_dense_meta(const int32_t* cu, int nseq, int64_t n_tokens, int32_t* meta,
                    void* stream);

/*
 * (sequence id, block id) tile list for blocks of `chunk` rows over cu, in
 * order; *count receives NT.  Restates prepare_chunk_indices,
 * logo/ops/common.py:110-124.  `out` holds max_tiles pairs; `workspace`
 * holds nseq + 1 int32.
 */
int logo_chunk_indices(const int32_t* cu, int nseq, int chunk, int32_t* out,
                       int64_t max_tiles, int32_t* count, int32_t* workspace,
                       void* stream);

/*
 * First compacted-query block of each key block: for tile t = (s, j) of
 * `chunks`, (lower_bound(pos[cu_q[s]:cu_q[s+1]], j*block) - 0) / block.
 * Restates _compute_q_start_blk, logo/ops/selected_full_attn.py:374-402.
 */
int logo_q_start_blk(const int32_t* pos, const int32_t* cu_q, const int32_t* chunks,
                     const int32_t* count, int64_t max_tiles, int block, int32_t* out,
                     void* stream);

/*
 * Query-sparse causal attention forward on selected rows
 * (sq_full_attn_fwd_kernel + _fwd, logo/ops/selected_full_attn.py:33-121,
 * :340-362, with the q gather :461 and output scatter :469-471 fused).
 * Writes every row of o: o[t] for selected tokens t, zero for the others
 * (the reference's zero-initialised output, :469-470; no fill by the caller),
 * and lse per compacted row.  q_idx/pos == NULL selects dense mode (every row, meta from
 * logo_dense_meta).  window < 0: full causal; window >= 0: keys
 * [p - window, p] (logo/layers/utils.py:144-147).
 * d is the head dim of q and k (64, 128 or 256); v_dim is that of v and o,
 * which the reference keeps separate (V, :341) and which must equal d here:
 * every kernel strides all of them by d.  The Python op zero-pads other
 * K, V <= 256 to 64, 128 or 256 before it calls this (the reference takes
 * K <= 256 in one block, :344).
 * dtype: LOGO_DTYPE_BF16; LOGO_DTYPE_F16 or LOGO_DTYPE_F32 in sparse mode
 * without a window (the reference's dots run in the input dtype, :80 :93-99
 * :108).  Every element tensor of the call (q, k, v, o, and for the backward
 * dout, q_sel, do_sel, dq, dk, dv) holds that type.  d = 256 and fp32 run on
 * generic kernels (logo_sq_generic); the others on the tuned ones.
 * workspace / workspace_bytes (may be NULL / 0): device memory that lets the
 * forward and dq kernels (no window) cut the key range of each query tile
 * into pieces when a head has few tiles, so that a grid which would fill the
 * GPU once is not bound by its heaviest tile (the reference has no
 * counterpart: its grid is one program per chunk, :348 :413).  Its first
 * bytes are arrival counters that must be zero when a call starts; every call
 * leaves them zero, so one zero-fill serves every later call.  Calls that
 * share a workspace must not overlap.  Too small (or NULL): no split.
 */
int logo_sq_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
                const int64_t* q_idx, const int32_t* pos, const int32_t* meta,
                const int32_t* cu, int64_t n_tokens, int nseq, int hq, int h, int d,
                int v_dim, int lanes, float scale, int window, int dtype, void* workspace,
                size_t workspace_bytes, void* stream);

/*
 * Bytes of the workspace logo_sq_fwd and logo_sq_bwd_dq need to split tiles
 * on the current device (0: they never split for this shape), and how many
 * of them, at its start, are the counters that must be zero.
 */
size_t logo_sq_workspace_bytes(int64_t n_tokens, int nseq, int hq, int d);
size_t logo_sq_workspace_counter_bytes(void);

/*
 * 1 when calls with head dim d and element type dtype run on the generic
 * attention kernels (d = 256, or LOGO_DTYPE_F32), 0 for the tuned ones (no
 * counterpart in the reference, whose Triton kernels take every size).  The
 * generic kernels take no split workspace, and their sparse backward reads q
 * and dout in place: q_sel and do_sel may be NULL.
 */
int logo_sq_generic(int d, int dtype);

/*
 * Backward (logo/ops/selected_full_attn.py:124-138 delta, :141-228 dq,
 * :231-337 dk/dv, :444-445 GQA sum).  o and dout are [N, HQ, D]; writes
 * every row of dq (zero for unselected tokens, as the zero-initialised dq of
 * the scatter :487-488, which is fused; no fill by the caller), every row of
 * dk and dv [N, H, D], and the workspaces delta [HQ, N]
 * fp32 and, in sparse mode, q_sel / do_sel [HQ, N, D] bf16: compacted copies
 * of the selected q and dO rows (the reference's q_sel / do_sel, :461 :483),
 * filled by the delta phase, of the call's dtype.  Dense mode ignores q_sel /
 * do_sel.
 */
int logo_sq_bwd(const void* q, const void* k, const void* v, const void* o,
    const void* dout, const float* lse, float* delta, void* q_sel, void* do_sel,
    void* dq, void* dk, void* dv, const int64_t* q_idx, const int32_t* pos,
    const int32_t* meta, const int32_t* cu, int64_t n_tokens, int nseq, int hq,
    int h, int d, int v_dim, int lanes, float scale, int window, int dtype, void* workspace,
    size_t workspace_bytes, void* stream);

/*
 * The three backward phases of logo_sq_bwd as separate launches, same
 * arguments: delta and the q_sel / do_sel copies (:124-138, :365-371), dq
 * (:141-228, :424-432), dk/dv (:231-337, :433-445).  Callers time or overlap
 * them one by one; dq and dk/dv read what the delta phase wrote.  Each phase
 * needs only the outputs it writes (dq, or dk and dv); the others may be NULL.
 */
int logo_sq_bwd_delta(const void* q, const void* k, const void* v, const void* o,
    const void* dout, const float* lse, float* delta, void* q_sel, void* do_sel,
    void* dq, void* dk, void* dv, const int64_t* q_idx, const int32_t* pos,
    const int32_t* meta, const int32_t* cu, int64_t n_tokens, int nseq, int hq,
    int h, int d, int v_dim, int lanes, float scale, int window, int dtype, void* workspace,
    size_t workspace_bytes, void* stream);
int logo_sq_bwd_dq(const void* q, const void* k, const void* v, const void* o,
    const void* dout, const float* lse, float* delta, void* q_sel, void* do_sel,
    void* dq, void* dk, void* dv, const int64_t* q_idx, const int32_t* pos,
    const int32_t* meta, const int32_t* cu, int64_t n_tokens, int nseq, int hq,
    int h, int d, int v_dim, int lanes, float scale, int window, int dtype, void* workspace,
    size_t workspace_bytes, void* stream);
int logo_sq_bwd_dkv(const void* q, const void* k, const void* v, const void* o,
    const void* dout, const float* lse, float* delta, void* q_sel, void* do_sel,
    void* dq, void* dk, void* dv, const int64_t* q_idx, const int32_t* pos,
    const int32_t* meta, const int32_t* cu, int64_t n_tokens, int nseq, int hq,
    int h, int d, int v_dim, int lanes, float scale, int window, int dtype, void* workspace,
    size_t workspace_bytes, void* stream);

/*
 * The dq and dk/dv phases together (after logo_sq_bwd_delta), same arguments,
 * dq, dk and dv all required: the two phases above in turn, except for the
 * local sliding-window branch (dense rows, 0 <= window <= 128, HQ == H, bf16;
 * logo/layers/utils.py:144-147), which runs one fused pass that computes S
 * and dP once for all three gradients.  logo_sq_bwd takes the same route.
 */
int logo_sq_bwd_dqkv(const void* q, const void* k, const void* v, const void* o,
    const void* dout, const float* lse, float* delta, void* q_sel, void* do_sel,
    void* dq, void* dk, void* dv, const int64_t* q_idx, const int32_t* pos,
    const int32_t* meta, const int32_t* cu, int64_t n_tokens, int nseq, int hq,
    int h, int d, int v_dim, int lanes, float scale, int window, int dtype, void* workspace,
    size_t workspace_bytes, void* stream);

/*
 * Fused epilogue forward: gate threshold, the two branch context RMSNorms
 * (one [D] weight each, shared by all heads) and the gated fusion, with the
 * reference's eager bf16 rounding points (logo/modules/layernorm.py:17-22;
 * logo/layers/logo.py:180-181, :225-226, :256-258).  L, G: [N, H, D];
 * gate: [N] (post-sigmoid); thres: one value on the device, of thres_dtype
 * (LOGO_DTYPE_BF16 or LOGO_DTYPE_F32: the threshold buffer as the model holds
 * it, read in place); w_l, w_g: [D]; out: [N, H*D].
 */
int logo_epilogue_fwd(const void* L, const void* G, const void* gate, const void* thres, int thres_dtype,
                      const void* w_l, const void* w_g, void* out, int64_t n_tokens,
                      int heads, int d, float eps, int dtype, void* stream);

/* Bytes of workspace logo_epilogue_bwd needs. */
size_t logo_epilogue_bwd_workspace_bytes(int64_t n_tokens, int heads, int d);

/*
 * Fused epilogue backward (autograd of the same expression): dL, dG [N, H, D],
 * dgate [N] (zero where gate < thres: the masked_fill at logo/layers/logo.py:256
 * blocks it), dw_l, dw_g [D]; reductions are deterministic.
 */
int logo_epilogue_bwd(const void* L, const void* G, const void* gate, const void* thres, int thres_dtype,
                      const void* w_l, const void* w_g, const void* dout, void* dL, void* dG,
                      void* dgate, void* dw_l, void* dw_g, int64_t n_tokens, int heads, int d,
                      float eps, void* workspace, int dtype, void* stream);

/* Bytes of split-K workspace logo_decode_attn needs for rows of <= max_len keys. */
size_t logo_decode_workspace_bytes(int batch, int hq, int d, int max_len);

/*
 * Gate-aware decode attention, one query token per sequence: for row b with
 * gate[b] >= *thres (thres of thres_dtype, as for logo_epilogue_fwd; or every
 * row when gate is NULL), out[b, hq] =
 * softmax(scale * q[b, hq] K[b, h, 0:lens[b]]^T) V[b, h, 0:lens[b]]; rows
 * whose gate fails get zeros and read no cache (the reference runs dense
 * attention for all rows and masks, logo/layers/logo.py:228-249, :256-258).
 * q, out: [B, HQ, D]; k_cache, v_cache: [B, H, t_cap, D] (logo/cache.py
 * layout, preallocated); max_len >= every lens[b] (sizes the grid).
 */
int logo_decode_attn(const void* q, const void* k_cache, const void* v_cache, const int32_t* lens,
                     const void* gate, const void* thres, int thres_dtype, void* out, void* workspace, int batch,
                     int hq, int h, int d, int64_t t_cap, int max_len, float scale, int dtype,
                     void* stream);

/* Bytes of workspace logo_decode_attn_fused needs (global rows of <= max_len_global keys). */
size_t logo_decode_fused_workspace_bytes(int batch, int hq, int d, int max_len_global);

/*
 * One decode step's attention for both LoGo branches and the fused epilogue
 * in two launches: the local branch (q_local over its window cache, every row
 * active, max_len_local <= 256), the gate-aware global branch (as
 * logo_decode_attn with gate / thres), then the context norms, gate mask and
 * fusion of logo_epilogue_fwd (weights w_local, w_global [D], eps) into
 * out [B, HQ, D].  Bit-identical to logo_decode_attn twice followed by
 * logo_epilogue_fwd; replaces logo/layers/logo.py:228-258 at decode.
 */
int logo_decode_attn_fused(const void* q_local, const void* k_local, const void* v_local,
                           const int32_t* lens_local, int64_t t_cap_local, int max_len_local,
                           const void* q_global, const void* k_global, const void* v_global,
                           const int32_t* lens_global, int64_t t_cap_global, int max_len_global,
                           const void* gate, const void* thres, int thres_dtype, const void* w_local,
                           const void* w_global, float eps, void* out, void* workspace, int batch, int hq,
                           int h, int d, float scale, int dtype, void* stream);

/*
 * Append one key/value row per (b, h) at position pos[b] of a preallocated
 * cache [B, H, t_cap, D] (ring > 0: at pos[b] % ring, the local window),
 * replacing the per-step torch.cat of logo/cache.py:97-118.
 */
int logo_cache_append(const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                      const int32_t* pos, int batch, int h, int d, int64_t t_cap, int ring,
                      int dtype, void* stream);

/*
 * Rotary embedding, in place, of up to four [N, H_i, D] bf16 tensors (q, k and
 * the global q, k; a NULL tensor is skipped) with one [N, D] cos / sin pair:
 * x' = x * cos + rotate_half(x) * sin with the eager bf16 rounding of
 * logo/modules/rotary.py:81-106 (apply_rotary_pos_emb, rotate_half), called at
 * logo/layers/logo.py:132-139.
 */
int logo_rope_apply(void* x0, int h0, void* x1, int h1, void* x2, int h2, void* x3, int h3,
                    const void* cos, const void* sin, int64_t n_tokens, int d, int dtype,
                    void* stream);

/*
 * Rotary embedding of up to four [N, H_i, D] bf16 tensors x_i into outputs y_i
 * (y_i == x_i allowed; a NULL x_i is skipped) with one [N, D] cos / sin pair.
 * inverse = 0: the forward rotation of logo_rope_apply (same rounding);
 * inverse = 1: its transpose, the gradient of the rotation: with x = dL/dy,
 * y1 = bf16(bf16(x1 * cos1) + bf16(x2 * sin2)) and
 * y2 = bf16(bf16(x2 * cos2) - bf16(x1 * sin1)), the rounding points of eager
 * autograd through logo/modules/rotary.py:81-106 (mul backward, then the
 * cat / neg backward of rotate_half), so a training step's RoPE forward and
 * backward are one launch each (logo/layers/logo.py:132-139).
 */
int logo_rope(const void* x0, void* y0, int h0, const void* x1, void* y1, int h1, const void* x2,
              void* y2, int h2, const void* x3, void* y3, int h3, const void* cos, const void* sin,
              int64_t n_tokens, int d, int inverse, int dtype, void* stream);

/*
 * Per-head projection of a few tokens, for up to three tensors in one launch
 * (a NULL x_i is skipped): y_i[t, h, :] = x_i[t, h, :] W_i[h] with x_i
 * [n_tokens, h_i, d], W_i [h_i, d, e], y_i [n_tokens, h_i, e], bf16, fp32
 * accumulation.  The LoGo layer's linear_proj global re-parameterisation
 * (logo/layers/logo.py:86-94, the einsum over heads of q, k and v) at decode
 * sizes (n_tokens <= 4096; d <= 256, e <= 128).
 */
int logo_head_proj(const void* x0, const void* w0, void* y0, int h0, const void* x1, const void* w1, void* y1,
                   int h1, const void* x2, const void* w2, void* y2, int h2, int n_tokens, int d, int e, int dtype,
                   void* stream);

/*
 * One decode step's q / k / v transform for a LoGo layer (linear_proj): from
 * each token's stacked projection row qkv[b, :] = [q | k | v] (row stride ldq
 * elements; H, HK, HK heads of d), the per-head global projections with wq
 * [H, d, d], wk / wv [HK, d, d] (as logo_head_proj), RoPE with cos / sin
 * [batch, d] of q, k and the global q, k (as logo_rope_apply), and the cache
 * appends of logo_cache_append: rotated k and v into the local ring
 * [batch, HK, ring, d] at pos[b] % ring, rotated global k and global v into the
 * global cache [batch, HK, t_cap, d] at pos[b].  Writes the rotated q and
 * global q to q_out / gq_out [batch, H, d].  With gate_out non-NULL it also
 * writes the gate sigmoid(qkv[b, gate_col]) of each token to gate_out [batch]
 * (logo/layers/logo.py:130, the gate projection stacked into the same row).
 * Replaces the layer's global projection, gate sigmoid, RoPE and cache update
 * of a decode step (logo/layers/logo.py:86-94, :130-150; logo/cache.py:97-118)
 * with one launch.
 */
int logo_decode_qkv(const void* qkv, int64_t ldq, const void* wq, const void* wk, const void* wv, const void* cos,
                    const void* sin, const int32_t* pos, void* q_out, void* gq_out, void* local_k, void* local_v,
                    void* global_k, void* global_v, int64_t gate_col, void* gate_out, int batch, int h, int hk,
                    int d, int ring, int64_t t_cap, int dtype, void* stream);

/*
 * Per-head linear map on the [N, H, d] layout in place: y[n, h, :] =
 * x[n, h, :] W_h (transpose_w = 0) or x[n, h, :] W_h^T (transpose_w = 1), W
 * [H, d, d]; x row n at x + n * ldx, y row n at y + n * ldy (elements).  The
 * linear_proj global re-parameterisation at training sizes
 * (logo/layers/logo.py:86-94) and its input gradient, without the head-major
 * copies of a batched GEMM.
 */
int logo_head_linear(const void* x, int64_t ldx, const void* w, void* y, int64_t ldy, int64_t n_tokens, int heads,
                     int d, int transpose_w, int dtype, void* stream);

/* Bytes of fp32 workspace logo_head_linear_dw needs. */
size_t logo_head_linear_dw_workspace_bytes(int64_t n_tokens, int heads, int d);

/*
 * Weight gradient of logo_head_linear: dw[h] = sum_n x[n, h, :]^T dy[n, h, :]
 * ([H, d, d], d = 128), reduced over token chunks in a fixed order.
 */
int logo_head_linear_dw(const void* x, int64_t ldx, const void* dy, int64_t ldy, void* dw, void* workspace,
                        int64_t n_tokens, int heads, int d, int dtype, void* stream);

/*
 * Input gradient of logo_head_linear summed with another gradient of the same
 * tensor: dx[n, h, :] = bf16(bf16(dy[n, h, :] W_h^T) + add[n, h, :]), the
 * product rounded as logo_head_linear's and the sum as an eager bf16 add.
 * Rows at dy + n * lddy, add + n * ldadd, dx + n * lddx (elements; dx may be
 * add itself).  No counterpart in the reference: it folds autograd's
 * accumulation of the two gradients of the layer's q, k and v (the local
 * branch through RoPE, the global one through this map,
 * logo/layers/logo.py:86-94, :121-158) into the map's backward.
 */
int logo_head_linear_grad_acc(const void* dy, int64_t lddy, const void* w, const void* add, int64_t ldadd, void* dx,
                              int64_t lddx, int64_t n_tokens, int heads, int d, int dtype, void* stream);

/*
 * Residual add + RMSNorm of the decoder: s_out = r + x (bf16, as the eager
 * add rounds) and y = RMSNorm(s_out) with weight w (as logo_rmsnorm), rows of
 * cols bf16 (a multiple of 8, at most 4096): the residual adds and the
 * post-attention / next input norms of logo/modeling_logo.py:58-66.
 */
int logo_add_rmsnorm(const void* r, const void* x, const void* w, void* s_out, void* y, int64_t rows, int cols,
                     float eps, int dtype, void* stream);

/*
 * SwiGLU activation y[row] = silu(g) * u with g = gu[row, 0:cols] and
 * u = gu[row, cols:2 cols] (row stride ld >= 2 cols, the stacked gate / up
 * projection), each op rounded to bf16 as the eager F.silu and mul
 * (logo/modules/mlp.py:24-27).
 */
int logo_silu_mul(const void* gu, int64_t ld, void* y, int64_t rows, int cols, int dtype, void* stream);

/*
 * RMSNorm of rows [rows, cols] bf16 with weight [cols]: y = w * bf16(x *
 * rsqrt(mean(x^2) + eps)), mean in fp32 (logo/modules/layernorm.py:17-22; the
 * decoder's input / post-attention / final norms, logo/modeling_logo.py:58-59,
 * :152).  cols: a multiple of 8, at most 4096.
 */
int logo_rmsnorm(const void* x, const void* w, void* y, int64_t rows, int cols, float eps,
                 int dtype, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LOGO_HIP_H_ */
