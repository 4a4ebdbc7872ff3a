// TORCH_LIBRARY(logo_hip) registration of the hot-path entry points of
// liblogo_hip.so, so that torch.library / torch.compile see them as operators
// with schemas (their fake kernels are registered from logo_amd/_torch_ops.py).
//
// Host code only: every operator checks its tensors (device, dtype,
// contiguity, shapes), allocates its outputs with the caching allocator on the
// current stream, and calls the C entry point, which launches on that stream.
// The library's own checks stay the last line (a failure raises with
// logo_last_error()).  Operators, the C entry point each wraps, and the
// reference code it replaces:
//   compact       logo_compact        build_selection, logo/ops/common.py:71-107
//   dense_meta    logo_dense_meta     all-rows metadata of the dense / SWA branches
//   sq_fwd        logo_sq_fwd         logo/ops/selected_full_attn.py:33-121, :340-362
//   sq_bwd_delta  logo_sq_bwd_delta   :124-138, :365-371
//   sq_bwd_dq     logo_sq_bwd_dq      :141-228, :424-432
//   sq_bwd_dkv    logo_sq_bwd_dkv     :231-337, :433-445
//   sq_bwd_dqkv   logo_sq_bwd_dqkv    dq and dk/dv together (one fused pass for
//                                     the sliding window, logo/layers/utils.py:144-147)
//   sq_bwd        delta, then dqkv    :124-445 (dq, dk, dv; workspaces internal)
//   epilogue_fwd  logo_epilogue_fwd   logo/layers/logo.py:180-181, :225-226, :256-258
//   epilogue_bwd  logo_epilogue_bwd   the autograd of epilogue_fwd
//   decode_attn   logo_decode_attn    logo/layers/logo.py:228-249
#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstdlib>
#include <mutex>
#include <utility>
#include <vector>

#include "../../include/logo_hip.h"

namespace {

void* sp() { return reinterpret_cast<void*>(c10::hip::getCurrentHIPStream().stream()); }

void ok(int rc, const char* what) { TORCH_CHECK(rc == LOGO_OK, what, " failed: ", logo_last_error()); }

const void* cptr(const at::Tensor& t) { return t.data_ptr(); }
void* mptr(at::Tensor& t) { return t.data_ptr(); }
template <typename T>
const T* opt_ptr(const std::optional<at::Tensor>& t) {
  return t.has_value() ? static_cast<const T*>(t->data_ptr()) : nullptr;
}

void need(const at::Tensor& t, const char* name, at::ScalarType dt) {
  TORCH_CHECK(t.is_cuda(), "logo_hip: ", name, " must be a ROCm GPU tensor");
  TORCH_CHECK(t.scalar_type() == dt, "logo_hip: ", name, " must be ", dt, ", got ", t.scalar_type());
  TORCH_CHECK(t.is_contiguous(), "logo_hip: ", name, " must be contiguous");
}

// compact(selection bool or u8 [N] or [N, lanes], cu i32 [nseq+1])
//   -> (q_idx i64 [lanes, N], pos i32 [lanes, N], meta)
std::tuple<at::Tensor, at::Tensor, at::Tensor> compact(const at::Tensor& sel, const at::Tensor& cu) {
  need(sel, "selection", sel.scalar_type() == at::kBool ? at::kBool : at::kByte);
  need(cu, "cu_seqlens", at::kInt);
  const int64_t n = sel.size(0);
  const int lanes = sel.dim() == 2 ? (int)sel.size(1) : 1;
  const int nseq = (int)cu.numel() - 1;
  auto i32 = cu.options();
  // entries past each lane's Sq: zero, written by the compaction itself
  // (n == 0 keeps one zero entry per lane)
  auto q_idx = n > 0 ? at::empty({lanes, n}, i32.dtype(at::kLong)) : at::zeros({lanes, 1}, i32.dtype(at::kLong));
  auto pos = n > 0 ? at::empty({lanes, n}, i32) : at::zeros({lanes, 1}, i32);
  auto meta = at::empty({lanes * LOGO_META_STRIDE(nseq)}, i32);
  auto ws = at::empty({(int64_t)logo_compact_workspace_bytes(n, lanes)}, i32.dtype(at::kByte));
  ok(logo_compact(static_cast<const uint8_t*>(sel.data_ptr()), n, lanes, cu.data_ptr<int32_t>(), nseq,
                  q_idx.data_ptr<int64_t>(), pos.data_ptr<int32_t>(), meta.data_ptr<int32_t>(), ws.data_ptr(),
                  sp()),
     "logo_compact");
  return {q_idx, pos, meta};
}

at::Tensor dense_meta(const at::Tensor& cu, int64_t n_tokens) {
  need(cu, "cu_seqlens", at::kInt);
  const int nseq = (int)cu.numel() - 1;
  auto meta = at::empty({LOGO_META_STRIDE(nseq)}, cu.options());
  ok(logo_dense_meta(cu.data_ptr<int32_t>(), nseq, n_tokens, meta.data_ptr<int32_t>(), sp()), "logo_dense_meta");
  return meta;
}

// q, k, v of one element type (bf16; fp16 or fp32 for the C library's
// query-sparse kernels, which rejects other fp16 / fp32 calls itself);
// returns its dtype code.
int check_attn(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v) {
  const at::ScalarType qt = q.scalar_type();
  const at::ScalarType dt = qt == at::kHalf || qt == at::kFloat ? qt : at::kBFloat16;
  need(q, "q", dt);
  need(k, "k", dt);
  need(v, "v", dt);
  TORCH_CHECK(q.dim() == 3 && k.dim() == 3 && v.dim() == 3, "logo_hip: q, k, v must be [N, heads, D]");
  TORCH_CHECK(k.size(0) == q.size(0) && v.sizes() == k.sizes() && k.size(2) == q.size(2),
              "logo_hip: q [N, HQ, D], k and v [N, H, D] must agree");
  return dt == at::kHalf ? LOGO_DTYPE_F16 : dt == at::kFloat ? LOGO_DTYPE_F32 : LOGO_DTYPE_BF16;
}

// Whether the call runs on the generic kernels (no compacted copies, no split).
bool generic_path(const at::Tensor& q, int dtype) { return logo_sq_generic((int)q.size(2), dtype) != 0; }

// Split workspace of the fwd / dq kernels for this shape (empty: no split).
// Its size depends only on the device's CU count, HQ and D (the pieces a
// split aims for fill the device twice, whatever N is): at most 136 MB at
// D = 128 on MI355X.
//  * Outside graph capture: one buffer per (device, stream), kept across
//    calls and grown on demand.  The kernels leave its counter prefix zero,
//    so only a new buffer needs the zero fill, and calls on one stream run in
//    order, so they never overlap on it.  At most kMaxCachedStreams buffers
//    are kept; beyond that the oldest entry is dropped (its memory returns to
//    the caching allocator on its own stream, after the work queued there).
//  * Under capture (hipStreamIsCapturing): a fresh buffer per call from the
//    caching allocator, its counters cleared by a fill kernel recorded in the
//    graph.  The graph's memory pool keeps the buffer for the graph's
//    lifetime, so a later eager call that regrows the cached buffer cannot
//    free memory a replay still uses, and a replay never depends on counters
//    that eager calls left behind.
// The environment variable LOGO_SQ_SPLIT=0 turns the split off (A/B timing,
// and tests that compare kernel variants bit for bit).
constexpr size_t kMaxCachedStreams = 16;

at::Tensor split_workspace(const at::Tensor& q, const at::Tensor& cu, int dtype) {
  const char* env = std::getenv("LOGO_SQ_SPLIT");
  const bool off = (env != nullptr && env[0] == '0') || generic_path(q, dtype);
  const size_t bytes =
      off ? 0 : logo_sq_workspace_bytes(q.size(0), (int)cu.numel() - 1, (int)q.size(1), (int)q.size(2));
  if (bytes == 0) return at::empty({0}, q.options().dtype(at::kByte));
  hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
  TORCH_CHECK(hipStreamIsCapturing(static_cast<hipStream_t>(sp()), &status) == hipSuccess,
              "logo_hip: hipStreamIsCapturing failed");
  if (status != hipStreamCaptureStatusNone) {
    auto ws = at::empty({(int64_t)bytes}, q.options().dtype(at::kByte));
    ws.narrow(0, 0, (int64_t)logo_sq_workspace_counter_bytes()).zero_();
    return ws;
  }
  static std::mutex mu;
  static std::vector<std::pair<std::pair<int, void*>, at::Tensor>> cache;  // oldest first
  const auto key = std::make_pair((int)q.get_device(), sp());
  std::lock_guard<std::mutex> lock(mu);
  auto it = std::find_if(cache.begin(), cache.end(), [&](const auto& e) { return e.first == key; });
  if (it == cache.end()) {
    if (cache.size() >= kMaxCachedStreams) cache.erase(cache.begin());
    cache.emplace_back(key, at::Tensor());
    it = cache.end() - 1;
  }
  at::Tensor& ws = it->second;
  if (!ws.defined() || (size_t)ws.numel() < bytes) {
    ws = at::empty({(int64_t)bytes}, q.options().dtype(at::kByte));
    ws.narrow(0, 0, (int64_t)logo_sq_workspace_counter_bytes()).zero_();
  }
  return ws;
}

std::tuple<at::Tensor, at::Tensor> sq_fwd(const at::Tensor& q, const at::Tensor& k, const at::Tensor& v,
                                          const std::optional<at::Tensor>& q_idx,
                                          const std::optional<at::Tensor>& pos, const at::Tensor& meta,
                                          const at::Tensor& cu, int64_t lanes, double scale, int64_t window) {
  const int dtype = check_attn(q, k, v);
  const int64_t n = q.size(0), hq = q.size(1), h = k.size(1), d = q.size(2);
  // Every row of o and lse is written (sparse mode: zero for unselected
  // tokens and for lse rows past each lane's rows, by the kernel).
  auto o = at::empty_like(q);
  auto lse = at::empty({hq, n}, q.options().dtype(at::kFloat));
  auto ws = window < 0 ? split_workspace(q, cu, dtype) : at::empty({0}, q.options().dtype(at::kByte));
  ok(logo_sq_fwd(cptr(q), cptr(k), cptr(v), mptr(o), lse.data_ptr<float>(), opt_ptr<int64_t>(q_idx),
                 opt_ptr<int32_t>(pos), meta.data_ptr<int32_t>(), cu.data_ptr<int32_t>(), n, (int)cu.numel() - 1,
                 (int)hq, (int)h, (int)d, (int)v.size(2), (int)lanes, (float)scale, (int)window, dtype,
                 ws.numel() ? ws.data_ptr() : nullptr, (size_t)ws.numel(), sp()),
     "logo_sq_fwd");
  return {o, lse};
}

// One backward phase (0 delta, 1 dq, 2 dk/dv) through its C entry point.
struct Bwd {
  const at::Tensor &q, &k, &v, &o, &lse, &dout;
  const std::optional<at::Tensor>&q_idx, &pos;
  const at::Tensor &meta, &cu;
  int64_t lanes;
  double scale;
  int64_t window;
  int call(int phase, at::Tensor* delta, at::Tensor* q_sel, at::Tensor* do_sel, at::Tensor* dq, at::Tensor* dk,
           at::Tensor* dv) const {
    const int dtype = check_attn(q, k, v);
    need(o, "o", q.scalar_type());
    need(dout, "dout", q.scalar_type());
    TORCH_CHECK(o.sizes() == q.sizes() && dout.sizes() == q.sizes(), "logo_hip: o and dout must be [N, HQ, D]");
    if (phase > 0) {
      need(*delta, "delta", at::kFloat);
      TORCH_CHECK(delta->numel() == q.size(0) * q.size(1), "logo_hip: delta must be [HQ, N]");
      if (q_idx.has_value() && !generic_path(q, dtype)) {
        need(*q_sel, "q_sel", q.scalar_type());
        need(*do_sel, "do_sel", q.scalar_type());
        TORCH_CHECK(q_sel->numel() == q.numel() && do_sel->numel() == q.numel(),
                    "logo_hip: q_sel and do_sel must be [HQ, N, D]");
      }
    }
    using F = decltype(&logo_sq_bwd);
    F fn = phase == 0 ? &logo_sq_bwd_delta : phase == 1 ? &logo_sq_bwd_dq : phase == 2 ? &logo_sq_bwd_dkv
                                                                                  : &logo_sq_bwd_dqkv;
    auto p = [](at::Tensor* t) -> void* { return t && t->numel() ? t->data_ptr() : nullptr; };
    at::Tensor ws = (phase == 1 || phase == 3) && window < 0 ? split_workspace(q, cu, dtype)
                                                            : at::empty({0}, q.options().dtype(at::kByte));
    return fn(cptr(q), cptr(k), cptr(v), cptr(o), cptr(dout), lse.data_ptr<float>(),
              static_cast<float*>(p(delta)), p(q_sel), p(do_sel), p(dq), p(dk), p(dv), opt_ptr<int64_t>(q_idx),
              opt_ptr<int32_t>(pos), meta.data_ptr<int32_t>(), cu.data_ptr<int32_t>(), q.size(0),
              (int)cu.numel() - 1, (int)q.size(1), (int)k.size(1), (int)q.size(2), (int)v.size(2), (int)lanes,
              (float)scale, (int)window, dtype, p(&ws), (size_t)ws.numel(), sp());
  }
};

#define LOGO_BWD_SCHEMA_ARGS                                                                                 \
  const at::Tensor &q, const at::Tensor &k, const at::Tensor &v, const at::Tensor &o, const at::Tensor &lse, \
      const at::Tensor &dout, const std::optional<at::Tensor>&q_idx, const std::optional<at::Tensor>&pos,    \
      const at::Tensor &meta, const at::Tensor &cu, int64_t lanes, double scale, int64_t window

// delta [HQ, N] fp32 (rows past Sq unwritten) and, in sparse mode on the tuned
// kernels, the compacted copies q_sel / do_sel [HQ, N, D] (empty in dense mode
// and on the generic kernels, which read q and dout in place): workspaces of
// the dq and dk/dv phases, whose rows past each head's Sq are left unwritten.
std::tuple<at::Tensor, at::Tensor, at::Tensor> sq_bwd_delta(LOGO_BWD_SCHEMA_ARGS) {
  const bool sparse = q_idx.has_value() && !generic_path(q, check_attn(q, k, v));
  auto delta = at::empty({q.size(1), q.size(0)}, q.options().dtype(at::kFloat));
  auto q_sel = sparse ? at::empty({q.size(1), q.size(0), q.size(2)}, q.options()) : at::empty({0}, q.options());
  auto do_sel = sparse ? at::empty_like(q_sel) : at::empty({0}, q.options());
  Bwd b{q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window};
  ok(b.call(0, &delta, &q_sel, &do_sel, nullptr, nullptr, nullptr), "logo_sq_bwd_delta");
  return {delta, q_sel, do_sel};
}

at::Tensor sq_bwd_dq(LOGO_BWD_SCHEMA_ARGS, const at::Tensor& delta, const at::Tensor& q_sel,
                     const at::Tensor& do_sel) {
  check_attn(q, k, v);
  auto dq = at::empty_like(q);  // every row written (sparse: unselected rows zero)
  Bwd b{q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window};
  auto dl = delta, qs = q_sel, ds = do_sel;
  ok(b.call(1, &dl, &qs, &ds, &dq, nullptr, nullptr), "logo_sq_bwd_dq");
  return dq;
}

std::tuple<at::Tensor, at::Tensor> sq_bwd_dkv(LOGO_BWD_SCHEMA_ARGS, const at::Tensor& delta,
                                              const at::Tensor& q_sel, const at::Tensor& do_sel) {
  check_attn(q, k, v);
  auto dk = at::empty_like(k);
  auto dv = at::empty_like(v);
  Bwd b{q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window};
  auto dl = delta, qs = q_sel, ds = do_sel;
  ok(b.call(2, &dl, &qs, &ds, nullptr, &dk, &dv), "logo_sq_bwd_dkv");
  return {dk, dv};
}

// dq, dk and dv after the delta phase (one fused pass for the sliding window).
std::tuple<at::Tensor, at::Tensor, at::Tensor> sq_bwd_dqkv(LOGO_BWD_SCHEMA_ARGS, const at::Tensor& delta,
                                                           const at::Tensor& q_sel, const at::Tensor& do_sel) {
  check_attn(q, k, v);
  auto dq = at::empty_like(q);
  auto dk = at::empty_like(k);
  auto dv = at::empty_like(v);
  Bwd b{q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window};
  auto dl = delta, qs = q_sel, ds = do_sel;
  ok(b.call(3, &dl, &qs, &ds, &dq, &dk, &dv), "logo_sq_bwd_dqkv");
  return {dq, dk, dv};
}

// The whole backward: (dq, dk, dv), its workspaces internal.
std::tuple<at::Tensor, at::Tensor, at::Tensor> sq_bwd(LOGO_BWD_SCHEMA_ARGS) {
  auto ws = sq_bwd_delta(q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window);
  return sq_bwd_dqkv(q, k, v, o, lse, dout, q_idx, pos, meta, cu, lanes, scale, window, std::get<0>(ws),
                     std::get<1>(ws), std::get<2>(ws));
}

int thres_code(const at::Tensor& thres) {
  TORCH_CHECK(thres.numel() == 1 && (thres.scalar_type() == at::kBFloat16 || thres.scalar_type() == at::kFloat),
              "logo_hip: the threshold is one bf16 or fp32 value");
  return thres.scalar_type() == at::kBFloat16 ? LOGO_DTYPE_BF16 : LOGO_DTYPE_F32;
}

// L, G [n, H, D] bf16, gate [n] bf16 (post-sigmoid), w_l / w_g [D] -> out [n, H * D]
at::Tensor epilogue_fwd(const at::Tensor& L, const at::Tensor& G, const at::Tensor& gate, const at::Tensor& thres,
                        const at::Tensor& w_l, const at::Tensor& w_g, double eps) {
  need(L, "L", at::kBFloat16);
  need(G, "G", at::kBFloat16);
  need(gate, "gate", at::kBFloat16);
  TORCH_CHECK(L.dim() == 3 && G.sizes() == L.sizes() && gate.numel() == L.size(0), "logo_hip: epilogue shapes");
  auto out = at::empty({L.size(0), L.size(1) * L.size(2)}, L.options());
  ok(logo_epilogue_fwd(cptr(L), cptr(G), cptr(gate), cptr(thres), thres_code(thres), cptr(w_l), cptr(w_g),
                       mptr(out), L.size(0), (int)L.size(1), (int)L.size(2), (float)eps, LOGO_DTYPE_BF16, sp()),
     "logo_epilogue_fwd");
  return out;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor, at::Tensor> epilogue_bwd(
    const at::Tensor& L, const at::Tensor& G, const at::Tensor& gate, const at::Tensor& thres, const at::Tensor& w_l,
    const at::Tensor& w_g, const at::Tensor& dout, double eps) {
  need(L, "L", at::kBFloat16);
  need(dout, "dout", at::kBFloat16);
  const int64_t n = L.size(0), H = L.size(1), D = L.size(2);
  auto dL = at::empty_like(L), dG = at::empty_like(G), dgate = at::empty_like(gate);
  auto dwl = at::empty_like(w_l), dwg = at::empty_like(w_g);
  auto ws = at::empty({(int64_t)logo_epilogue_bwd_workspace_bytes(n, (int)H, (int)D)}, L.options().dtype(at::kByte));
  ok(logo_epilogue_bwd(cptr(L), cptr(G), cptr(gate), cptr(thres), thres_code(thres), cptr(w_l), cptr(w_g),
                       cptr(dout), mptr(dL), mptr(dG), mptr(dgate), mptr(dwl), mptr(dwg), n, (int)H, (int)D,
                       (float)eps, ws.data_ptr(), LOGO_DTYPE_BF16, sp()),
     "logo_epilogue_bwd");
  return {dL, dG, dgate, dwl, dwg};
}

// q [B, HQ, D], caches [B, H, T_cap, D], lens i32 [B]; gate [B] with thres, or neither.
at::Tensor decode_attn(const at::Tensor& q, const at::Tensor& k_cache, const at::Tensor& v_cache,
                       const at::Tensor& lens, const std::optional<at::Tensor>& gate,
                       const std::optional<at::Tensor>& thres, int64_t max_len, double scale) {
  need(q, "q", at::kBFloat16);
  need(lens, "lens", at::kInt);
  TORCH_CHECK(gate.has_value() == thres.has_value(), "logo_hip: gate and thres go together");
  const int64_t B = q.size(0), HQ = q.size(1), D = q.size(2);
  auto out = at::empty_like(q);
  auto ws = at::empty({(int64_t)logo_decode_workspace_bytes((int)B, (int)HQ, (int)D, (int)max_len)},
                      q.options().dtype(at::kByte));
  ok(logo_decode_attn(cptr(q), cptr(k_cache), cptr(v_cache), lens.data_ptr<int32_t>(),
                      gate.has_value() ? cptr(*gate) : nullptr, thres.has_value() ? cptr(*thres) : nullptr,
                      thres.has_value() ? thres_code(*thres) : LOGO_DTYPE_F32, mptr(out), ws.data_ptr(), (int)B,
                      (int)HQ, (int)k_cache.size(1), (int)D, k_cache.size(2), (int)max_len, (float)scale,
                      LOGO_DTYPE_BF16, sp()),
     "logo_decode_attn");
  return out;
}

}  // namespace

TORCH_LIBRARY(logo_hip, m) {
  m.def("compact(Tensor selection, Tensor cu) -> (Tensor, Tensor, Tensor)");
  m.def("dense_meta(Tensor cu, int n_tokens) -> Tensor");
  m.def("sq_fwd(Tensor q, Tensor k, Tensor v, Tensor? q_idx, Tensor? pos, Tensor meta, Tensor cu, int lanes, "
        "float scale, int window) -> (Tensor, Tensor)");
  m.def("sq_bwd_delta(Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse, Tensor dout, Tensor? q_idx, "
        "Tensor? pos, Tensor meta, Tensor cu, int lanes, float scale, int window) -> (Tensor, Tensor, Tensor)");
  m.def("sq_bwd_dq(Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse, Tensor dout, Tensor? q_idx, Tensor? pos, "
        "Tensor meta, Tensor cu, int lanes, float scale, int window, Tensor delta, Tensor q_sel, Tensor do_sel) "
        "-> Tensor");
  m.def("sq_bwd_dkv(Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse, Tensor dout, Tensor? q_idx, "
        "Tensor? pos, Tensor meta, Tensor cu, int lanes, float scale, int window, Tensor delta, Tensor q_sel, "
        "Tensor do_sel) -> (Tensor, Tensor)");
  m.def("sq_bwd_dqkv(Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse, Tensor dout, Tensor? q_idx, "
        "Tensor? pos, Tensor meta, Tensor cu, int lanes, float scale, int window, Tensor delta, Tensor q_sel, "
        "Tensor do_sel) -> (Tensor, Tensor, Tensor)");
  m.def("sq_bwd(Tensor q, Tensor k, Tensor v, Tensor o, Tensor lse, Tensor dout, Tensor? q_idx, Tensor? pos, "
        "Tensor meta, Tensor cu, int lanes, float scale, int window) -> (Tensor, Tensor, Tensor)");
  m.def("epilogue_fwd(Tensor L, Tensor G, Tensor gate, Tensor thres, Tensor w_l, Tensor w_g, float eps) -> Tensor");
  m.def("epilogue_bwd(Tensor L, Tensor G, Tensor gate, Tensor thres, Tensor w_l, Tensor w_g, Tensor dout, "
        "float eps) -> (Tensor, Tensor, Tensor, Tensor, Tensor)");
  m.def("decode_attn(Tensor q, Tensor k_cache, Tensor v_cache, Tensor lens, Tensor? gate, Tensor? thres, "
        "int max_len, float scale) -> Tensor");
}

TORCH_LIBRARY_IMPL(logo_hip, CUDA, m) {
  m.impl("compact", &compact);
  m.impl("dense_meta", &dense_meta);
  m.impl("sq_fwd", &sq_fwd);
  m.impl("sq_bwd_delta", &sq_bwd_delta);
  m.impl("sq_bwd_dq", &sq_bwd_dq);
  m.impl("sq_bwd_dkv", &sq_bwd_dkv);
  m.impl("sq_bwd_dqkv", &sq_bwd_dqkv);
  m.impl("sq_bwd", &sq_bwd);
  m.impl("epilogue_fwd", &epilogue_fwd);
  m.impl("epilogue_bwd", &epilogue_bwd);
  m.impl("decode_attn", &decode_attn);
}
