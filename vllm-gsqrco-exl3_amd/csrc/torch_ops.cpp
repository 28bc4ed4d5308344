// torch.ops._C_gguf: the reference's Route L op surface (plugin/vllm_gguf_plugin/csrc/
// lcpp_shim.cu:973-1008), registered from C++ over the C ABI of libgguf_mi355x.so
// (include/gguf_mi355x.h). Host code only: each op turns its tensors into gguf_view structs,
// allocates the output and the workspace with torch's caching allocator on X's device (so calls
// are safe under graph capture), and calls the library on torch's current stream.
//
// Same namespace (registered as a fragment), op names and schemas as the reference.
// Implementations are registered for CUDA (HIP tensors on ROCm) and, as in the reference
// (lcpp_shim.cu:997-1008), for CPU, where
// the library runs every guard and the call ends with "must be CUDA tensors". A guard that
// fails raises RuntimeError with the library's message (the reference's message fragments, in
// its order). The fake (meta) implementations for torch.compile are registered from Python
// (vllm_gguf_plugin/_C_gguf.py).
#include <ATen/ATen.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <exception>
#include <optional>

#include "../../include/gguf_mi355x.h"

namespace {

int32_t dtype_code(const at::Tensor& t) {
  switch (t.scalar_type()) {
    case at::kFloat: return GGUF_DT_F32;
    case at::kHalf: return GGUF_DT_F16;
    case at::kBFloat16: return GGUF_DT_BF16;
    case at::kByte: return GGUF_DT_U8;
    default: return GGUF_DT_OTHER;
  }
}

gguf_view make_view(const at::Tensor& t) {
  gguf_view v{};
  v.data = t.numel() ? t.data_ptr() : nullptr;
  v.dtype = dtype_code(t);
  v.ndim = (int32_t)t.dim();
  for (int64_t i = 0; i < std::min<int64_t>(2, t.dim()); ++i) {
    v.size[i] = t.size(i);
    v.stride[i] = t.stride(i);
  }
  v.device = t.is_cuda() ? (int32_t)t.get_device() : -1;
  return v;
}

[[noreturn]] void raise_last() { TORCH_CHECK(false, gguf_last_error()); }

void* stream_of(const at::Tensor& t) {
  return t.is_cuda() ? (void*)c10::hip::getCurrentHIPStream(t.get_device()).stream() : nullptr;
}

// The output and workspace tensors of one product, made by the library's allocator callback once
// its guards have passed. A failed allocation (torch raises) is kept and raised after the call.
struct OpAlloc {
  const at::Tensor& X;
  int64_t row;
  at::Tensor y, ws;
  std::exception_ptr err;
};

void* op_alloc(void* ctx, int what, size_t bytes) {
  OpAlloc& a = *static_cast<OpAlloc*>(ctx);
  try {
    if (what == GGUF_ALLOC_OUTPUT) {
      a.y = at::empty({a.X.size(0), a.row}, a.X.options());
      return a.y.numel() ? a.y.data_ptr() : nullptr;
    }
    a.ws = at::empty({(int64_t)bytes}, a.X.options().dtype(at::kByte));
    return a.ws.data_ptr();
  } catch (...) {
    a.err = std::current_exception();
    return nullptr;
  }
}

// One product through gguf_mul_mat_alloc: the guards (host only, once), then the output and the
// workspace from torch's caching allocator, then the launches on the current stream.
at::Tensor mul_mat(int op, const at::Tensor& W, const at::Tensor& X, int64_t type, int64_t row,
                   const std::optional<at::Tensor>& x_q8) {
  const gguf_view wv = make_view(W), xv = make_view(X);
  gguf_view qv{};
  const gguf_view* qp = nullptr;
  if (x_q8) {
    qv = make_view(*x_q8);
    qp = &qv;
  }
  OpAlloc a{X, row, {}, {}, nullptr};
  const int rc = gguf_mul_mat_alloc(op, &wv, &xv, type, row, qp, &op_alloc, &a, stream_of(X));
  if (a.err) std::rethrow_exception(a.err);
  if (rc != GGUF_OK) raise_last();
  return a.y;
}

template <int OP>
at::Tensor op_q8(const at::Tensor& W, const at::Tensor& X, int64_t type, int64_t row,
                 const std::optional<at::Tensor>& x_q8) {
  return mul_mat(OP, W, X, type, row, x_q8);
}

template <int OP>
at::Tensor op_own(const at::Tensor& W, const at::Tensor& X, int64_t type, int64_t row) {
  return mul_mat(OP, W, X, type, row, std::nullopt);
}

// the small dense product (gguf_dense_mul_mat): Y[n, rows] = X @ W.T in X's dtype
at::Tensor dense_mul_mat(const at::Tensor& W, const at::Tensor& X) {
  const gguf_view wv = make_view(W), xv = make_view(X);
  const int64_t n = X.dim() == 2 ? X.size(0) : 0, rows = W.dim() == 2 ? W.size(0) : 0;
  at::Tensor y = at::empty({n, rows}, X.options());
  const int rc = gguf_dense_mul_mat(&wv, &xv, y.numel() ? y.data_ptr() : nullptr,
                                    (size_t)(y.numel() * y.element_size()), stream_of(X));
  if (rc != GGUF_OK) raise_last();
  return y;
}

at::Tensor quantize_q8_1(const at::Tensor& X, int64_t type, bool mmq, bool vendored) {
  const gguf_view xv = make_view(X);
  const int64_t nbytes = X.dim() == 2 ? (int64_t)gguf_q8_1_bytes(X.size(0), X.size(1), mmq) : 0;
  at::Tensor out = at::empty({nbytes}, X.options().dtype(at::kByte));
  const int rc = gguf_lcpp_quantize_q8_1(&xv, type, mmq, vendored, nbytes ? out.data_ptr() : nullptr,
                                         (size_t)nbytes, stream_of(X));
  if (rc != GGUF_OK) raise_last();
  return out;
}

}  // namespace

// A fragment of the namespace, as the reference adds its Route L ops to the _C_gguf library of its
// stock ops (lcpp_shim.cu:973 beside torch_bindings.cpp:22): this registration loads beside any
// other library that defines _C_gguf (the stock extension's ggml_dequantize, for one).
TORCH_LIBRARY_FRAGMENT(_C_gguf, m) {
  m.def("lcpp_mul_mat_vec_q(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor");
  m.def("lcpp_mul_mat_q(Tensor W, Tensor X, int type, SymInt row) -> Tensor");
  m.def("lcpp_mul_mat_vec_iq3(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor");
  m.def("lcpp_mul_mat_vec_iq3_mma(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor");
  m.def("lcpp_mul_mat_vec_own(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor");
  m.def("lcpp_mul_mat_mma_k(Tensor W, Tensor X, int type, SymInt row) -> Tensor");
  m.def("lcpp_mul_mat_vec_iq3_mma_packed(Tensor W, Tensor X, int type, SymInt row, Tensor? x_q8=None) -> Tensor");
  m.def("lcpp_mul_mat_iq3_packed(Tensor W, Tensor X, int type, SymInt row) -> Tensor");
  m.def("lcpp_quantize_q8_1(Tensor X, int type, bool mmq, bool vendored) -> Tensor");
  m.def("dense_mul_mat(Tensor W, Tensor X) -> Tensor");
}

#define GGUF_IMPLS(KEY)                                                                   \
  TORCH_LIBRARY_IMPL(_C_gguf, KEY, m) {                                                    \
    m.impl("lcpp_mul_mat_vec_q", &op_q8<GGUF_OP_MUL_MAT_VEC_Q>);                          \
    m.impl("lcpp_mul_mat_q", &op_own<GGUF_OP_MUL_MAT_Q>);                                 \
    m.impl("lcpp_mul_mat_vec_iq3", &op_q8<GGUF_OP_MUL_MAT_VEC_IQ3>);                      \
    m.impl("lcpp_mul_mat_vec_iq3_mma", &op_q8<GGUF_OP_MUL_MAT_VEC_IQ3_MMA>);              \
    m.impl("lcpp_mul_mat_vec_own", &op_q8<GGUF_OP_MUL_MAT_VEC_OWN>);                      \
    m.impl("lcpp_mul_mat_mma_k", &op_own<GGUF_OP_MUL_MAT_MMA_K>);                         \
    m.impl("lcpp_mul_mat_vec_iq3_mma_packed", &op_q8<GGUF_OP_MUL_MAT_VEC_IQ3_MMA_PACKED>); \
    m.impl("lcpp_mul_mat_iq3_packed", &op_own<GGUF_OP_MUL_MAT_IQ3_PACKED>);               \
    m.impl("lcpp_quantize_q8_1", &quantize_q8_1);                                         \
    m.impl("dense_mul_mat", &dense_mul_mat);                                              \
  }
GGUF_IMPLS(CUDA)
GGUF_IMPLS(CPU)
#undef GGUF_IMPLS
