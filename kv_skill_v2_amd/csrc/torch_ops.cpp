// The per-token operators of the `xenc` namespace, defined and implemented in C++ so that a
// decode call costs one dispatcher hop into the C ABI (include/xenc_hip.h): no Python in the
// call, outputs allocated by torch's caching allocator, torch's current HIP stream of the query's
// device.  Their fake (meta) kernels are registered from Python (kv_skill_v2_amd/torch_ops.py),
// as are the prefill operators.  Host code only: built with the system C++ compiler against
// torch's headers into libxenc_torch.so, next to libxenc_hip.so, whose C ABI it calls.
//
//   xenc::route_topk          LibraryInjector.route (xenc/injector.py:220-229) for few rows
//   xenc::library_read        the read of LibraryInjector._branch (xenc/injector.py:236-265)
//   xenc::route_read          both in one call (the top-k inside the read kernel when it can)
//   xenc::paged_decode_joint  DecodeReader.__call__ (xenc/d23_read_kernels.py:145-160)
#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <string>
#include <tuple>

#include "xenc_hip.h"

namespace {

// Error codes of the C ABI as Python exceptions: argument errors are ValueError, a failed
// launch RuntimeError (the same mapping as kv_skill_v2_amd._lib.check).
void check(int rc, const char* what) {
  if (rc == XENC_OK) return;
  std::string msg = std::string(what) + ": " + xenc_strerror(rc);
  if (rc == XENC_EHIP) msg += " (hipError " + std::to_string(xenc_last_hip_error()) + ")";
  if (rc == XENC_EINVAL || rc == XENC_ENULL || rc == XENC_EALIGN || rc == XENC_EWORKSPACE ||
      rc == XENC_ESCRATCH)
    TORCH_CHECK_VALUE(false, msg);
  TORCH_CHECK(false, msg);
}

void* stream_of(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.device().index()).stream(); }

template <class T>
T* ptr(const at::Tensor& t) {
  return static_cast<T*>(t.data_ptr());
}

int as_int(const c10::SymInt& v) { return static_cast<int>(v.expect_int()); }

at::TensorOptions f32(const at::Tensor& like) { return like.options().dtype(at::kFloat); }
at::TensorOptions i32(const at::Tensor& like) { return like.options().dtype(at::kInt); }

std::tuple<at::Tensor, at::Tensor, at::Tensor> route_topk(const at::Tensor& q, const at::Tensor& S,
                                                          const at::Tensor& chunk_ptr, const at::Tensor& q_group,
                                                          c10::SymInt top_k, double route_temp, c10::SymInt cmax,
                                                          c10::SymInt kk) {
  const c10::DeviceGuard guard(q.device());
  const int64_t M = q.size(0), d = q.size(1);
  const int C = as_int(cmax), K = as_int(kk);
  at::Tensor w = at::empty({M, C}, f32(q)), idx = at::empty({M, K}, i32(q)), wsel = at::empty({M, K}, f32(q));
  if (M)
    check(xenc_route_topk(ptr<const float>(q), q.stride(0), (int)M, (int)d, ptr<const float>(S),
                          ptr<const int>(chunk_ptr), ptr<const int>(q_group), (int)chunk_ptr.numel() - 1,
                          as_int(top_k), (float)route_temp, ptr<float>(w), w.stride(0), ptr<int>(idx),
                          ptr<float>(wsel), K, stream_of(q)),
          "xenc_route_topk");
  return {w, idx, wsel};
}

at::Tensor library_read(const at::Tensor& q, const at::Tensor& pages, const at::Tensor& chunk_page,
                        const at::Tensor& chunk_nvalid, const at::Tensor& chunk_ptr, const at::Tensor& q_group,
                        const at::Tensor& idx, const at::Tensor& w_sel, double read_temp, bool softmax,
                        c10::SymInt nsplit, at::Tensor& workspace, c10::SymInt max_rows) {
  const c10::DeviceGuard guard(q.device());
  const int64_t M = q.size(0), d = pages.size(-1), K = idx.size(1);
  at::Tensor r = at::empty({M, d}, f32(q));
  if (M == 0 || K == 0) return r.zero_();
  check(xenc_library_read_decode(ptr<const float>(q), q.stride(0), (int)M, (int)d, pages.data_ptr(),
                                 (int)pages.size(1), pages.stride(0), ptr<const int>(chunk_page),
                                 ptr<const int>(chunk_nvalid), ptr<const int>(chunk_ptr), ptr<const int>(q_group),
                                 (int)chunk_ptr.numel() - 1, ptr<const int>(idx), ptr<const float>(w_sel), (int)K,
                                 (float)read_temp, softmax ? 1 : 0, as_int(nsplit), ptr<float>(r), r.stride(0),
                                 workspace.data_ptr(), (size_t)workspace.numel(), as_int(max_rows), stream_of(q)),
        "xenc_library_read_decode");
  return r;
}

std::tuple<at::Tensor, at::Tensor, at::Tensor, at::Tensor> route_read(
    const at::Tensor& q, const at::Tensor& S, const at::Tensor& pages, const at::Tensor& chunk_page,
    const at::Tensor& chunk_nvalid, const at::Tensor& chunk_ptr, const at::Tensor& q_group, c10::SymInt top_k,
    double route_temp, c10::SymInt cmax, c10::SymInt kk, double read_temp, bool softmax, c10::SymInt nsplit,
    at::Tensor& workspace, c10::SymInt max_rows) {
  const c10::DeviceGuard guard(q.device());
  const int64_t M = q.size(0), d = q.size(1);
  const int C = as_int(cmax), K = as_int(kk);
  at::Tensor w = at::empty({M, C}, f32(q)), idx = at::empty({M, K}, i32(q)), wsel = at::empty({M, K}, f32(q));
  at::Tensor r = at::empty({M, pages.size(-1)}, f32(q));
  if (M)
    check(xenc_route_read_decode(ptr<const float>(q), q.stride(0), (int)M, (int)d, ptr<const float>(S),
                                 pages.data_ptr(), (int)pages.size(1), pages.stride(0), ptr<const int>(chunk_page),
                                 ptr<const int>(chunk_nvalid), ptr<const int>(chunk_ptr), ptr<const int>(q_group),
                                 (int)chunk_ptr.numel() - 1, as_int(top_k), (float)route_temp, ptr<float>(w),
                                 w.stride(0), ptr<int>(idx), ptr<float>(wsel), K, (float)read_temp,
                                 softmax ? 1 : 0, as_int(nsplit), ptr<float>(r), r.stride(0), workspace.data_ptr(),
                                 (size_t)workspace.numel(), as_int(max_rows), stream_of(q)),
          "xenc_route_read_decode");
  return {w, idx, wsel, r};
}

int joint_dtype(const at::Tensor& k) {
  if (k.scalar_type() == at::kHalf) return 0;
  TORCH_CHECK_VALUE(k.scalar_type() == at::kBFloat16, "paged_decode_joint: pools must be fp16 or bf16");
  return 1;
}

void paged_decode_joint(const at::Tensor& q, const at::Tensor& op_k, const at::Tensor& op_v, const at::Tensor& op_bt,
                        const at::Tensor& op_len, const at::Tensor& own_k, const at::Tensor& own_v,
                        const at::Tensor& own_bt, const at::Tensor& own_len, double scale, c10::SymInt nsplit,
                        c10::SymInt chunk, at::Tensor& workspace, c10::SymInt max_n, at::Tensor& out) {
  const c10::DeviceGuard guard(q.device());
  const int64_t N = q.size(0), hq = q.size(1), d = q.size(2), hkv = op_k.size(2);
  if (N == 0) return;
  check(xenc_paged_decode_joint(joint_dtype(op_k), (int)N, (int)hq, (int)hkv, (int)d, q.data_ptr(), q.stride(0),
                                q.stride(1), op_k.data_ptr(), op_v.data_ptr(), op_k.stride(0), op_k.stride(1),
                                op_k.stride(2), (int)op_k.size(1), ptr<const int>(op_bt), op_bt.stride(0),
                                ptr<const int>(op_len), own_k.data_ptr(), own_v.data_ptr(), own_k.stride(0),
                                own_k.stride(1), own_k.stride(2), (int)own_k.size(1), ptr<const int>(own_bt),
                                own_bt.stride(0), ptr<const int>(own_len), (float)scale, as_int(nsplit),
                                as_int(chunk), ptr<float>(out), out.stride(0), out.stride(1), workspace.data_ptr(),
                                (size_t)workspace.numel(), as_int(max_n), stream_of(q)),
        "xenc_paged_decode_joint");
}

}  // namespace

TORCH_LIBRARY_FRAGMENT(xenc, m) {
  m.def("route_topk(Tensor q, Tensor S, Tensor chunk_ptr, Tensor q_group, SymInt top_k, float route_temp, "
        "SymInt cmax, SymInt kk) -> (Tensor, Tensor, Tensor)");
  m.def("library_read(Tensor q, Tensor pages, Tensor chunk_page, Tensor chunk_nvalid, Tensor chunk_ptr, "
        "Tensor q_group, Tensor idx, Tensor w_sel, float read_temp, bool softmax, SymInt nsplit, "
        "Tensor(a!) workspace, SymInt max_rows) -> Tensor");
  m.def("route_read(Tensor q, Tensor S, Tensor pages, Tensor chunk_page, Tensor chunk_nvalid, Tensor chunk_ptr, "
        "Tensor q_group, SymInt top_k, float route_temp, SymInt cmax, SymInt kk, float read_temp, bool softmax, "
        "SymInt nsplit, Tensor(a!) workspace, SymInt max_rows) -> (Tensor, Tensor, Tensor, Tensor)");
  m.def("paged_decode_joint(Tensor q, Tensor op_k, Tensor op_v, Tensor op_bt, Tensor op_len, Tensor own_k, "
        "Tensor own_v, Tensor own_bt, Tensor own_len, float scale, SymInt nsplit, SymInt chunk, "
        "Tensor(a!) workspace, SymInt max_n, Tensor(b!) out) -> ()");
}

TORCH_LIBRARY_IMPL(xenc, CUDA, m) {
  m.impl("route_topk", &route_topk);
  m.impl("library_read", &library_read);
  m.impl("route_read", &route_read);
  m.impl("paged_decode_joint", &paged_decode_joint);
}
