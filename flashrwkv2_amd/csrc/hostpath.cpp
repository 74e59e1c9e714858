// Native fast path of the per-step calls of the decode / serving loop: the
// graph-form ticket preparation and the fp32-state recurrence with a ticket.
//
// The Python layer (flashrwkv2_amd/_C.py) implements the whole `_C` contract
// of the reference (flashrwkv2._C: csrc/sm120/tmix/wkv7/
// infer_recurrent_fp32io16_forward_varlen.cpp:89-387 and csrc/validation.cpp:
// 27-129), including every error message.  These functions decide the valid
// case of those checks on at::Tensor metadata directly and launch through
// the C ABI; whenever a call is not plainly valid (or needs the sequence
// split, a decay bias, another device) they return None and the caller runs
// the Python path, which either raises the reference's error or performs the
// call.  So the checks' messages have one source, and a call that succeeds
// here is one the Python path would have accepted.

#include <torch/extension.h>

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>

#include "../../include/flashrwkv2_amd.h"

namespace py = pybind11;

namespace {

constexpr int64_t kInt32Max = 2147483647;

int64_t version_of(const at::Tensor& t) { return t.is_inference() ? -1 : t._version(); }

bool cuda_contig_on(const at::Tensor& t, int dev) {
  return t.is_cuda() && t.is_contiguous() && t.get_device() == dev;
}

bool current_device_is(int dev) {
  int cur = -1;
  return hipGetDevice(&cur) == hipSuccess && cur == dev;
}

// The facts of a validated metadata ticket that each consumer re-checks
// (…fp32io16_forward_varlen.cpp:89-225): the identity, storage, version and
// geometry of the two metadata tensors, the sizes the ticket was validated
// for, the stream it is bound to, and the device pointers the kernels read.
struct TicketFacts {
  const c10::TensorImpl* qsl = nullptr;
  const c10::TensorImpl* slots = nullptr;
  const void* qsl_ptr = nullptr;
  const void* slots_ptr = nullptr;
  int64_t qsl_version = -1, slots_version = -1;
  int64_t qsl_numel = 0, slots_numel = 0;
  bool qsl_contig = false, slots_contig = false;
  int64_t total_tokens = 0, pool_size = 0, max_seqlen = 0;
  bool graph = false;
  int64_t stream = 0;
  const int32_t* qsl_snap = nullptr;
  const int32_t* slots_snap = nullptr;
  const int32_t* status = nullptr;

  TicketFacts(const at::Tensor& q, const at::Tensor& s, const at::Tensor& q_snap,
              const at::Tensor& s_snap, const at::Tensor& st, int64_t total, int64_t pool,
              int64_t maxlen, bool graph_mode, int64_t stream_handle)
      : qsl(q.unsafeGetTensorImpl()),
        slots(s.unsafeGetTensorImpl()),
        qsl_ptr(q.data_ptr()),
        slots_ptr(s.data_ptr()),
        qsl_version(version_of(q)),
        slots_version(version_of(s)),
        qsl_numel(q.numel()),
        slots_numel(s.numel()),
        qsl_contig(q.dim() == 1 && q.is_contiguous()),
        slots_contig(s.dim() == 1 && s.is_contiguous()),
        total_tokens(total),
        pool_size(pool),
        max_seqlen(maxlen),
        graph(graph_mode),
        stream(stream_handle),
        qsl_snap(q_snap.data_ptr<int32_t>()),
        slots_snap(s_snap.data_ptr<int32_t>()),
        status(st.data_ptr<int32_t>()) {}

  // RecurrentMetadataTicket::check_compatible's valid case
  bool matches(const at::Tensor& q, const at::Tensor& s, int64_t total, int64_t pool,
               int64_t maxlen, int64_t stream_handle) const {
    if (q.unsafeGetTensorImpl() != qsl || s.unsafeGetTensorImpl() != slots) return false;
    if (q.data_ptr() != qsl_ptr || s.data_ptr() != slots_ptr) return false;
    if (!graph && ((qsl_version >= 0 && version_of(q) != qsl_version) ||
                   (slots_version >= 0 && version_of(s) != slots_version)))
      return false;
    if (!(qsl_contig && slots_contig && q.dim() == 1 && s.dim() == 1 && q.is_contiguous() &&
          s.is_contiguous() && q.numel() == qsl_numel && s.numel() == slots_numel))
      return false;
    return total == total_tokens && pool == pool_size &&
           (maxlen <= 0 || maxlen == max_seqlen) && stream_handle == stream;
  }
};

int dtype_code(at::ScalarType t) {
  return t == at::kBFloat16 ? FR2_DTYPE_BFLOAT16 : t == at::kHalf ? FR2_DTYPE_FLOAT16 : -1;
}

// tmix_wkv7_recurrent_fp32_from_decay_logits with a ticket and no decay bias
// (…fp32io16_forward_varlen.cpp:330-387): the output tensor, an int status
// code when the library rejected the launch, or None for the Python path.
py::object recurrent_fp32(const TicketFacts& f, const at::Tensor& qsl, const at::Tensor& slots,
                          const at::Tensor& state, const at::Tensor& r, const at::Tensor& w,
                          const at::Tensor& k, const at::Tensor& v, const at::Tensor& a,
                          const at::Tensor& b, double scale, int64_t max_seqlen,
                          int64_t stream) {
  if (!state.is_cuda() || !state.is_contiguous() || state.scalar_type() != at::kFloat ||
      state.dim() != 4)
    return py::none();
  const int dev = state.get_device();
  const int64_t H = state.size(1), D = state.size(2);
  if (state.size(0) <= 0 || H <= 0 || H > kInt32Max || state.size(3) != D ||
      (D != 64 && D != 128 && D != 256) || state.size(0) > kInt32Max)
    return py::none();
  if (!cuda_contig_on(qsl, dev) || !cuda_contig_on(slots, dev) ||
      qsl.scalar_type() != at::kInt || slots.scalar_type() != at::kInt)
    return py::none();
  const int64_t n = slots.numel();
  if (n <= 0 || n > 65535 || slots.dim() != 1 || qsl.dim() != 1 || qsl.numel() != n + 1)
    return py::none();
  const int dtype = dtype_code(r.scalar_type());
  if (dtype < 0 || r.dim() != 3 || r.size(0) <= 0 || r.size(0) > kInt32Max || r.size(1) != H ||
      r.size(2) != D || !cuda_contig_on(r, dev))
    return py::none();
  for (const at::Tensor* t : {&w, &k, &v, &a, &b})
    if (t->scalar_type() != r.scalar_type() || t->sizes() != r.sizes() || !cuda_contig_on(*t, dev))
      return py::none();
  // misaligned views (an odd storage offset) take the Python path, which
  // runs them on aligned copies
  for (const at::Tensor* t : {&r, &w, &k, &v, &a, &b})
    if (reinterpret_cast<uintptr_t>(t->data_ptr()) & 15u) return py::none();
  if (!std::isfinite(scale)) return py::none();
  if (!f.matches(qsl, slots, r.size(0), state.size(0), max_seqlen, stream)) return py::none();
  if (!current_device_is(dev)) return py::none();
  // the sequence split (few long sequences) allocates a workspace and uses a
  // second stream: left to the Python path
  int32_t pieces = 1, piece_len = 0, lead_len = 0;
  int64_t ws = 0;
  if (fr2_wkv7_recurrent_fp32_split_plan(static_cast<int32_t>(n), static_cast<int32_t>(H),
                                         static_cast<int32_t>(D),
                                         static_cast<int32_t>(f.max_seqlen), &pieces,
                                         &piece_len, &lead_len, &ws) != FR2_OK ||
      pieces > 1)
    return py::none();
  at::Tensor out = at::empty_like(v);
  const int rc = fr2_wkv7_recurrent_fp32_forward(
      f.qsl_snap, f.slots_snap, f.status, static_cast<int32_t>(n), static_cast<int32_t>(H),
      static_cast<int32_t>(D), r.size(0), static_cast<int32_t>(f.max_seqlen), dtype,
      state.data_ptr<float>(), r.data_ptr(), w.data_ptr(), nullptr, k.data_ptr(), v.data_ptr(),
      a.data_ptr(), b.data_ptr(), out.data_ptr(), static_cast<float>(scale),
      reinterpret_cast<void*>(stream));
  if (rc != FR2_OK) return py::int_(rc);
  return py::cast(out);
}

// prepare_tmix_wkv7_recurrent_graph_metadata's valid case (…cpp:277-326):
// (status, workspace) after the device validation launch, an int status code
// when the library rejected it, or None for the Python path.
py::object prepare_graph(const at::Tensor& qsl, const at::Tensor& slots,
                         const at::Tensor& live_tokens, const at::Tensor& live_seqs,
                         int64_t token_capacity, int64_t sequence_capacity, int64_t pool_size,
                         int64_t max_seqlen_capacity, int64_t stream) {
  if (!qsl.is_cuda()) return py::none();
  const int dev = qsl.get_device();
  for (const at::Tensor* t : {&qsl, &slots, &live_tokens, &live_seqs})
    if (!cuda_contig_on(*t, dev) || t->scalar_type() != at::kInt) return py::none();
  if (!(sequence_capacity > 0 && sequence_capacity <= 65535 && slots.dim() == 1 &&
        slots.numel() == sequence_capacity && qsl.dim() == 1 &&
        qsl.numel() == sequence_capacity + 1 && token_capacity > 0 &&
        token_capacity <= kInt32Max && pool_size > 0 && pool_size <= kInt32Max &&
        max_seqlen_capacity > 0 && max_seqlen_capacity <= token_capacity &&
        live_tokens.numel() == 1 && live_seqs.numel() == 1))
    return py::none();
  if (!current_device_is(dev)) return py::none();
  const auto opts = qsl.options();
  at::Tensor status = at::empty({3}, opts);
  at::Tensor seen = at::empty({pool_size}, opts);
  const int rc = fr2_wkv7_prepare_metadata(
      qsl.data_ptr<int32_t>(), slots.data_ptr<int32_t>(), static_cast<int32_t>(sequence_capacity),
      static_cast<int32_t>(token_capacity), static_cast<int32_t>(pool_size),
      static_cast<int32_t>(max_seqlen_capacity), live_tokens.data_ptr<int32_t>(),
      live_seqs.data_ptr<int32_t>(), status.data_ptr<int32_t>(), seen.data_ptr<int32_t>(),
      nullptr, nullptr, reinterpret_cast<void*>(stream));
  if (rc != FR2_OK) return py::int_(rc);
  return py::make_tuple(status, seen);
}

}  // namespace

PYBIND11_MODULE(_hostpath, m) {
  m.doc() = "native fast path of the per-step ticket and recurrence calls";
  py::class_<TicketFacts>(m, "TicketFacts")
      .def(py::init<const at::Tensor&, const at::Tensor&, const at::Tensor&, const at::Tensor&,
                    const at::Tensor&, int64_t, int64_t, int64_t, bool, int64_t>());
  m.def("recurrent_fp32", &recurrent_fp32);
  m.def("prepare_graph", &prepare_graph);
}
