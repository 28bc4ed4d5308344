// C ABI of libgguf_mi355x.so (declared in include/gguf_mi355x.h): guards, workspace sizing and
// dispatch to the gfx950 kernels. Host code only; nothing here touches the GPU until every
// guard has passed.
//
// The guards restate the reference's run() type checks (lcpp_shim.cu:767-791) and check_inputs
// (lcpp_shim.cu:690-732) in the same order with the same message fragments, so callers (and the
// CPU guard tests) see the same rejections. Types served: the reference's Route L set (Q2_K,
// Q4_K, Q6_K, IQ2_XXS, IQ2_XS, IQ2_S, IQ3_XXS, IQ3_S, IQ4_XS, IQ1_M; lcpp_shim.cu:676-684).
#include <hip/hip_runtime.h>

#include <climits>
#include <cstdarg>
#include <cstdio>
#include <mutex>
#include <string>

#include "../../include/gguf_mi355x.h"
#include "gguf_common.h"
#include "split_k.h"

namespace gguf {
hipError_t launch_quantize(const void* x, int dtype, int64_t n, int64_t k, int64_t s01, int type, bool mmq, void* y,
                           hipStream_t stream);
hipError_t launch_gemv_raw(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                           void* y, int y_dtype, hipStream_t stream);
hipError_t launch_gemm(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                       void* y, int y_dtype, hipStream_t stream);
hipError_t launch_gemv_packed(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* q8, int n,
                              void* y, int y_dtype, hipStream_t stream);
hipError_t launch_quantize_xq(const void* x, int dtype, int64_t n, int64_t k, int64_t s01, int type, bool vec,
                              void* y, hipStream_t stream, uint32_t* zero = nullptr, int zero_words = 0);
hipError_t launch_q8_1_to_xq(const void* q8, int64_t n, int64_t k, int type, void* y, hipStream_t stream,
                             uint32_t* zero = nullptr, int zero_words = 0);
hipError_t launch_gemm_xq(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n,
                          void* y, int y_dtype, bool mmq, void* split_ws, hipStream_t stream);
int raw_split(int type, int64_t nrows, int64_t k, int64_t n);
int tile_split(int64_t nrows, int64_t k, int64_t n);
hipError_t launch_gemv_packed_x(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x, int x_dtype,
                                int64_t s01, int n, void* y, int y_dtype, hipStream_t stream);
bool gemv_rows_supported(int type, int64_t nrows, int64_t row_bytes, int64_t k, int64_t n);
bool gemv_packed_x_supported(int64_t nrows, int64_t k, int64_t n);
hipError_t launch_gemv_rows_x(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x,
                              int x_dtype, int64_t s01, int n, void* y, int y_dtype, hipStream_t stream);
bool gemv_rows_x_supported(int type, int64_t nrows, int64_t row_bytes, int64_t k, int64_t n);
bool gemv_mfma4_supported(int type, int64_t nrows, int64_t row_bytes, int64_t k, int64_t n);
bool gemv_generic_x_supported(int type, int64_t nrows, int64_t row_bytes, int64_t k, int64_t n);
bool gemv_iq3xxs_stream_supported(int64_t nrows, int64_t row_bytes, int64_t k, int64_t n, bool fused);
hipError_t launch_gemv_iq3xxs_stream(const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x,
                                     int x_dtype, int64_t s01, int n, void* y, int y_dtype, hipStream_t stream);
hipError_t launch_gemm_iq3xxs_packed(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n,
                                     void* y, int y_dtype, hipStream_t stream);
hipError_t launch_gemv_generic_x(int type, const uint8_t* W, int64_t row_bytes, int nrows, int k, const void* x,
                                 int x_dtype, int64_t s01, int n, void* y, int y_dtype, hipStream_t stream);
hipError_t launch_gemm_packed_xq(const uint8_t* W, int64_t row_bytes, int nrows, int k, const uint8_t* xq, int n,
                                 void* y, int y_dtype, void* split_ws, hipStream_t stream);
hipError_t launch_quantize_xh(const void* x, int dtype, int64_t n, int64_t k, int64_t s01, int type, void* y,
                              hipStream_t stream);
bool prefill_uses_xh(int type, bool packed);
bool small_h_supported(int type, bool packed);
bool small_h_range(int type, int64_t nrows, int64_t n);
hipError_t launch_gemm_small_h(int type, bool packed, const uint8_t* W, int64_t row_bytes, int nrows, int k,
                               const uint8_t* xh, int n, void* y, int y_dtype, hipStream_t stream);
hipError_t launch_gemm_prefill(int type, bool packed, const uint8_t* W, int64_t row_bytes, int nrows, int k,
                               const uint8_t* xq, int n, void* y, int y_dtype, hipStream_t stream);
hipError_t launch_iq3_pack(int type, uint8_t* w, int64_t rows, int64_t row_bytes, bool unpack, uint8_t* scratch,
                           size_t scratch_bytes, hipStream_t stream);
size_t iq3_pack_scratch_bytes(int64_t rows, int64_t row_bytes);
hipError_t launch_dense(int dtype, const void* W, int64_t ws0, int rows, int k, const void* X, int64_t xs0, int n,
                        void* y, hipStream_t stream);
}  // namespace gguf

namespace {

thread_local std::string g_err;

int fail(const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_err = buf;
  return GGUF_EINVAL;
}

int hip_fail(hipError_t e, const char* op, const char* what) {
  char buf[512];
  snprintf(buf, sizeof(buf), "%s: HIP error in %s: %s", op, what, hipGetErrorString(e));
  g_err = buf;
  return GGUF_EHIP;
}

const char* op_name(int op) {
  switch (op) {
    case GGUF_OP_MUL_MAT_VEC_Q: return "lcpp_mul_mat_vec_q";
    case GGUF_OP_MUL_MAT_Q: return "lcpp_mul_mat_q";
    case GGUF_OP_MUL_MAT_VEC_IQ3: return "lcpp_mul_mat_vec_iq3";
    case GGUF_OP_MUL_MAT_VEC_IQ3_MMA: return "lcpp_mul_mat_vec_iq3_mma";
    case GGUF_OP_MUL_MAT_VEC_OWN: return "lcpp_mul_mat_vec_own";
    case GGUF_OP_MUL_MAT_MMA_K: return "lcpp_mul_mat_mma_k";
    case GGUF_OP_MUL_MAT_VEC_IQ3_MMA_PACKED: return "lcpp_mul_mat_vec_iq3_mma_packed";
    case GGUF_OP_MUL_MAT_IQ3_PACKED: return "lcpp_mul_mat_iq3_packed";
    default: return "gguf_mul_mat";
  }
}

// lcpp_type_supported (lcpp_shim.cu:676-684)
bool type_served(int64_t t) {
  return t == gguf::kQ4_K || t == gguf::kQ6_K || t == gguf::kIQ3_S || t == gguf::kIQ4_XS || t == gguf::kQ2_K ||
         t == gguf::kIQ2_XXS || t == gguf::kIQ2_XS || t == gguf::kIQ2_S || t == gguf::kIQ3_XXS || t == gguf::kIQ1_M;
}

using gguf::kIQ1_M;
using gguf::kIQ2_S;
using gguf::kIQ3_XXS;

// Q2_K, the IQ2 types, IQ3_XXS and IQ1_M run on the generic kernels: the dot4 GEMV for the decode
// ops, the per-slice MFMA GEMM for the product ops; the packed ops on IQ3_XXS read its unit layout
// (the IQ3 stream GEMV, and the generic GEMM staging the layout's fields into GGUF blocks)
bool generic(int64_t t) { return gguf::generic_type((int)t); }

// the generic types whose product ops run on the xq-layout GEMM (D4 scales); Q2_K's D2S6 layout
// stays on the per-slice GEMM over block_q8_1_mmq
bool generic_xq(int64_t t) { return generic(t) && t != gguf::kQ2_K && t != kIQ1_M; }

bool is_float(int32_t dt) { return dt == GGUF_DT_F32 || dt == GGUF_DT_F16 || dt == GGUF_DT_BF16; }

int64_t elem_size(int32_t dt) { return dt == GGUF_DT_F32 ? 4 : dt == GGUF_DT_U8 ? 1 : 2; }

bool op_packed(int op) { return op == GGUF_OP_MUL_MAT_VEC_IQ3_MMA_PACKED || op == GGUF_OP_MUL_MAT_IQ3_PACKED; }
bool op_gemm(int op) {
  return op == GGUF_OP_MUL_MAT_Q || op == GGUF_OP_MUL_MAT_MMA_K || op == GGUF_OP_MUL_MAT_IQ3_PACKED;
}
bool op_iq3(int op) {
  return op == GGUF_OP_MUL_MAT_VEC_IQ3 || op == GGUF_OP_MUL_MAT_VEC_IQ3_MMA || op_packed(op);
}
// activation-row limits of the ops (lcpp_shim.cu:775-777; mma_k_max_cols = 64)
int64_t op_max_rows(int op) {
  if (op == GGUF_OP_MUL_MAT_Q || op == GGUF_OP_MUL_MAT_IQ3_PACKED) return 0;
  if (op == GGUF_OP_MUL_MAT_MMA_K) return 64;
  if (op == GGUF_OP_MUL_MAT_VEC_IQ3_MMA_PACKED) return 32;
  return 8;
}

// check_inputs (lcpp_shim.cu:690-732). Returns K, or -1 with g_err set.
int64_t check_inputs(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row, int64_t max_rows,
                     const char* op) {
  if (!type_served(type)) return fail("%s: unsupported ggml type %lld", op, (long long)type), -1;
  if (W->ndim != 2 || X->ndim != 2) return fail("%s: W and X must be 2-D", op), -1;
  if (W->dtype != GGUF_DT_U8) return fail("%s: W must be uint8", op), -1;
  if (!is_float(X->dtype)) return fail("%s: X must be fp32, fp16 or bf16", op), -1;
  const int64_t ts = gguf::block_bytes((int)type);
  const int64_t row_bytes = W->size[1];
  if (!(row_bytes > 0 && row_bytes % ts == 0))
    return fail("%s: W row bytes %lld not a multiple of the block size %lld", op, (long long)row_bytes,
                (long long)ts), -1;
  const int64_t k = row_bytes / ts * gguf::kQK;
  if (k % 512 != 0)
    return fail("%s: K=%lld must be a multiple of 512 (no weight tail padding)", op, (long long)k), -1;
  if (!(k <= INT_MAX && W->size[0] <= INT_MAX)) return fail("%s: W too large", op), -1;
  if (!(row > 0 && row <= W->size[0]))
    return fail("%s: row=%lld out of range (W has %lld rows)", op, (long long)row, (long long)W->size[0]), -1;
  if (W->stride[1] != 1) return fail("%s: W inner stride must be 1", op), -1;
  if (!(W->size[0] == 1 || W->stride[0] == row_bytes))
    return fail("%s: W rows must be contiguous (row stride %lld, row bytes %lld)", op, (long long)W->stride[0],
                (long long)row_bytes), -1;
  if (reinterpret_cast<uintptr_t>(W->data) % 16 != 0) return fail("%s: W data must be 16-byte aligned", op), -1;
  if (X->size[1] != k)
    return fail("%s: X has %lld columns, W rows hold K=%lld", op, (long long)X->size[1], (long long)k), -1;
  if (!(X->stride[1] == 1 && (X->size[0] <= 1 || X->stride[0] >= k))) return fail("%s: X inner stride must be 1", op), -1;
  if (max_rows > 0 && X->size[0] > max_rows)
    return fail("%s: at most %lld rows, got %lld", op, (long long)max_rows, (long long)X->size[0]), -1;
  if (X->size[0] > INT_MAX) return fail("%s: X too large", op), -1;
  // device checks last, so host views exercise every guard above and are then rejected
  if (W->device < 0 || X->device < 0) return fail("%s: W and X must be CUDA tensors", op), -1;
  if (W->device != X->device) return fail("%s: W and X must be on the same device", op), -1;
  return k;
}

// run()'s checks (lcpp_shim.cu:767-791) then check_inputs; returns K or -1.
int64_t check_op(int op, const gguf_view* W, const gguf_view* X, int64_t type, int64_t row, const gguf_view* x_q8) {
  if (op < 0 || op >= GGUF_OP_COUNT) return fail("gguf_mul_mat: unknown op %d", op), -1;
  const char* name = op_name(op);
  if (!W || !X) return fail("%s: W and X must be given", name), -1;
  if (op_iq3(op) && !(type == gguf::kIQ3_S || type == kIQ3_XXS))
    return fail("%s: IQ3_S or IQ3_XXS only, got type %lld", name, (long long)type), -1;
  if (op == GGUF_OP_MUL_MAT_VEC_OWN && !(type == gguf::kQ4_K || type == kIQ2_S))
    return fail("%s: Q4_K or IQ2_S only, got type %lld", name, (long long)type), -1;
  if (op == GGUF_OP_MUL_MAT_MMA_K && !(type == gguf::kQ4_K || type == gguf::kIQ4_XS || type == kIQ2_S))
    return fail("%s: Q4_K, IQ4_XS or IQ2_S only, got type %lld", name, (long long)type), -1;
  if (op == GGUF_OP_MUL_MAT_Q && type == kIQ1_M) return fail("%s: no MMQ for IQ1_M", name), -1;
  if (op_packed(op) && row % 16 != 0)
    return fail("%s: row=%lld must be a multiple of 16 (packed 16-row tiles)", name, (long long)row), -1;
  const int64_t k = check_inputs(W, X, type, row, op_max_rows(op), name);
  if (k < 0) return -1;
  if (x_q8) {
    const int64_t q8_bytes = X->size[0] * k / gguf::kQ81 * 36;
    if (!(x_q8->dtype == GGUF_DT_U8 && x_q8->ndim == 1 && x_q8->stride[0] == 1 && x_q8->size[0] >= q8_bytes))
      return fail("%s: x_q8 must be contiguous uint8 with at least %lld bytes", name, (long long)q8_bytes), -1;
    if (reinterpret_cast<uintptr_t>(x_q8->data) % 16 != 0) return fail("%s: x_q8 must be 16-byte aligned", name), -1;
    if (!(x_q8->device >= 0 && x_q8->device == X->device)) return fail("%s: x_q8 must be on X's device", name), -1;
  }
  return k;
}

size_t align256(size_t b) { return (b + 255) & ~(size_t)255; }

// Makes `device` current for the call when it is not already (the reference's DeviceGuard,
// lcpp_shim.cu:796), restoring the caller's device after; no device call when nothing changes,
// so a call inside stream capture makes no device switch.
struct DeviceScope {
  int prev = -1;
  hipError_t err = hipSuccess;
  explicit DeviceScope(int device) {
    int cur = -1;
    err = hipGetDevice(&cur);
    if (err == hipSuccess && cur != device) {
      err = hipSetDevice(device);
      if (err == hipSuccess) prev = cur;
    }
  }
  ~DeviceScope() {
    if (prev >= 0) (void)hipSetDevice(prev);
  }
};

}  // namespace

extern "C" {

const char* gguf_last_error(void) { return g_err.c_str(); }

const char* gguf_version(void) { return "gguf_mi355x 0.1 (gfx950)"; }

int gguf_check_op(int op, const gguf_view* W, const gguf_view* X, int64_t type, int64_t row, const gguf_view* x_q8) {
  g_err.clear();
  return check_op(op, W, X, type, row, x_q8) < 0 ? GGUF_EINVAL : GGUF_OK;
}

size_t gguf_q8_1_bytes(int64_t n, int64_t k, int mmq) {
  return mmq ? (size_t)(n * k / 128 * 144) : (size_t)(n * k / gguf::kQ81 * 36);
}

namespace {

// Decode ops (1..8 rows; the packed IQ3 op up to 32) go to the int8-MFMA GEMM from this many
// activation rows on, measured against the dot4 GEMV at the 27B-layer shapes: the GEMV's time
// grows with every row, the GEMM's is flat up to 16. IQ3_S on plain rows stays on the GEMV.
// The packed decode op quantises X inside the GEMV when the caller gives no x_q8: at one
// activation row on weights of up to 32M values (the attention projections) block by block, and
// at one or two rows on larger weights by quantising all of X into LDS first.
bool packed_fused(int op, int64_t row, int64_t k, int64_t n, bool has_x_q8) {
  return op_packed(op) && !has_x_q8 && gguf::gemv_packed_x_supported(row, k, n);
}

// A Q4_K / IQ4_XS / Q6_K decode op on the row-chunk GEMV with no x_q8 from the caller quantises X
// inside the GEMV at one or two rows where each wave's part of X is small (K <= 8192).
bool rows_fused(int op, int64_t type, int64_t row, int64_t k, int64_t n, bool has_x_q8);

// Product ops go to the 128 x 128-tile prefill GEMM from this many activation rows on (the small
// GEMMs' one-column-tile-group plans re-decode the weights once per 16..64 activation rows).
constexpr int64_t kPrefillFrom = 256;

bool xxs_packed(int op, int64_t type);

// Whether a product op runs the prefill GEMM (128 weight rows x 256 activation rows per
// workgroup; 128 on grids of fewer than 256). Its grid must hold enough workgroups: per
// workgroup it walks all of K, so on a small grid most CUs idle while the small GEMMs (16-row
// tiles) spread the same work. Measured (µs per op, graph replays, prefill / small GEMM):
//   1024 x 5120, M = 256 / 512 (8 / 16 groups): IQ3_S 106 / 109 against 26 / 38, Q6_K 113 / 114
//   against 28 / 49; M = 2048 (64 groups): IQ3_S 124 against 134, Q6_K 127 against 166;
//   6144 x 5120, M = 256 (48): IQ3_S 108 against 95, Q4_K 117 against 96; M = 512 (96): 114
//   against 168, 123 against 184; 5120 x 17408, M = 256 (40): IQ3_S 314 against 224; M = 512
//   (80): 323 against 430; 17408 x 5120, M = 256 (136): 152 against 158.
// So from 64 groups on (128 for IQ4_XS, whose prefill GEMM is the int8 one: 5120 x 6144 M = 512,
// 80 groups, 219 against 182; 17408 x 5120 M = 256, 136 groups, 242 against 263). Packed IQ3_XXS,
// whose small GEMM (the generic one) is slower, from 32 groups at 256 rows and on grids of 128
// groups from 64 rows (17408 x 5120 M = 64 / 128 / 255: 92 / 93 / 135 against 97 / 166 / 309;
// 6144 x 5120 M = 256, 48 groups: 96 against 114; 5120 x 17408 M = 128, 40 groups: 275 against
// 148).
bool prefill_route(int op, int64_t type, int64_t row, int64_t k, int64_t n) {
  if (!op_gemm(op) || n < 64) return false;
  const int64_t groups = (row + 127) / 128 * ((n + 255) / 256);
  if (xxs_packed(op, type)) return (n >= kPrefillFrom && groups >= 32) || groups >= 128;
  if (n < kPrefillFrom) return false;
  return groups >= (type == gguf::kIQ4_XS ? 128 : 64);
}

int64_t vec_mma_from(int op, int64_t type) {
  if (op_packed(op)) return 5;
  if (type == gguf::kQ4_K || type == gguf::kQ6_K) return 3;
  if (type == gguf::kIQ4_XS) return 5;
  return INT64_MAX;
}

// Bytes per 256-value block of the GGUF-row types with a row-chunk GEMV (0 for the others).
int64_t rows_block_bytes(int64_t type) {
  return type == gguf::kQ4_K ? 144 : type == gguf::kQ6_K ? 210 : type == gguf::kIQ4_XS ? 136 : 0;
}

// The MFMA decode GEMV (Q4_K / IQ4_XS / Q6_K at 2..4 rows, Q4_K / IQ4_XS at one row on long K;
// gemv_mfma4.hip) on a decode op's shape.
bool decode_mfma4(int op, int64_t type, int64_t row, int64_t k, int64_t n) {
  const int64_t bb = rows_block_bytes(type);
  return !op_gemm(op) && !op_packed(op) && bb > 0 && gguf::gemv_mfma4_supported((int)type, row, k / 256 * bb, k, n);
}

// A decode op runs the int8-MFMA small GEMM from vec_mma_from rows on, except at up to four rows
// of Q4_K / IQ4_XS / Q6_K where a GEMV takes the shape (X's q8_1 in LDS): the MFMA decode GEMV
// where it applies, else the row-chunk GEMV.
bool decode_mma(int op, int64_t type, int64_t row, int64_t k, int64_t n) {
  if (n < vec_mma_from(op, type) || decode_mfma4(op, type, row, k, n)) return false;
  const int64_t bb = rows_block_bytes(type);
  return !(op_packed(op) == false && bb > 0 && gguf::gemv_rows_supported((int)type, row, k / 256 * bb, k, n));
}

// A packed op on IQ3_XXS: the weight is in the build's IQ3_XXS unit layout (gguf_iq3_pack).
bool xxs_packed(int op, int64_t type) { return op_packed(op) && type == kIQ3_XXS; }


// A generic type's decode op with X quantised inside the stream GEMV (1-2 rows, K <= 8192).
bool generic_fused(int op, int64_t type, int64_t row, int64_t k, int64_t n) {
  if (xxs_packed(op, type)) return gguf::gemv_iq3xxs_stream_supported(row, k / 256 * 98, k, n, true);
  return gguf::gemv_generic_x_supported((int)type, row, k / 256 * gguf::block_bytes((int)type), k, n);
}

bool rows_fused(int op, int64_t type, int64_t row, int64_t k, int64_t n, bool has_x_q8) {
  if (op_gemm(op) || op_packed(op) || has_x_q8 || decode_mma(op, type, row, k, n) ||
      decode_mfma4(op, type, row, k, n))
    return false;
  const int64_t bb = rows_block_bytes(type);
  return bb > 0 && gguf::gemv_rows_x_supported((int)type, row, k / 256 * bb, k, n);
}

// The MFMA products with K <= 8192 run the fp16 small GEMM (X in the xh layout) for packed IQ3_S
// and Q4_K from 64 to 255 activation rows, and below 64 rows where its one-workgroup-per-CU range
// plan applies (4..5 row tiles per CU; 33..48 rows for IQ3_S, 17..48 for Q4_K); the rest below the
// prefill rows the int8 small GEMM (xq layout). Measured at the 27B-layer shapes: from 64 rows the fp16 GEMM's
// shared decode beats re-decoding the weights per group of 4 column tiles (17408 x 5120 IQ3_S,
// 128 rows: 84 against 134 us); over K = 17408 (68 blocks in one workgroup's loop, 320
// workgroups) the int8 GEMM's K split across waves is faster.
bool small_fp16(int op, int64_t type, int64_t row, int64_t k, int64_t n) {
  if (!op_gemm(op) || k > 8192 || !gguf::small_h_supported((int)type, op_packed(op))) return false;
  return (n >= 64 && !prefill_route(op, type, row, k, n)) || gguf::small_h_range((int)type, row, n);
}

// The int8 small GEMM on Q4_K / IQ4_XS / Q6_K rows (gemm_raw_kernel): product ops below the
// prefill rows off the fp16 GEMM's plans, and decode ops from vec_mma_from rows on.
bool raw_gemm(int op, int64_t type, int64_t row, int64_t k, int64_t n) {
  if (op_packed(op) || !(type == gguf::kQ4_K || type == gguf::kIQ4_XS || type == gguf::kQ6_K)) return false;
  if (op_gemm(op)) return !prefill_route(op, type, row, k, n) && !small_fp16(op, type, row, k, n);
  return decode_mma(op, type, row, k, n);
}

// The int8 tile GEMM on packed IQ3_S (gemm_iq3s_tile_kernel), on the same terms.
bool tile_gemm(int op, int64_t type, int64_t row, int64_t k, int64_t n) {
  if (!op_packed(op) || type != gguf::kIQ3_S) return false;
  if (op_gemm(op)) return !prefill_route(op, type, row, k, n) && !small_fp16(op, type, row, k, n);
  return decode_mma(op, type, row, k, n);
}

// Either GEMM's K split over workgroups (split_k.h): the workgroups per tile and the row tiles.
struct SplitPlan {
  int split = 1;
  int64_t tiles = 0;
};

SplitPlan split_plan(int op, int64_t type, int64_t row, int64_t k, int64_t n) {
  SplitPlan p;
  if (raw_gemm(op, type, row, k, n)) p = {gguf::raw_split((int)type, row, k, n), (row + 15) / 16};
  else if (tile_gemm(op, type, row, k, n)) p = {gguf::tile_split(row, k, n), row / 16};
  return p;
}

// Bytes after the xq copy of X that a split GEMM needs (slots, then its counters).
size_t split_ws(int op, int64_t type, int64_t row, int64_t k, int64_t n) {
  const SplitPlan p = split_plan(op, type, row, k, n);
  return gguf::split_ws_bytes(p.split, p.tiles, n);
}

}  // namespace

size_t gguf_op_workspace_bytes(int op, int64_t type, int64_t row, int64_t k, int64_t n, int has_x_q8) {
  if (n <= 0) return 0;
  if (generic(type)) {
    if (xxs_packed(op, type) && prefill_route(op, type, row, k, n)) return align256(gguf::xh_bytes(n, k));
    if (op_gemm(op)) return align256(generic_xq(type) ? gguf::xq_bytes(n, k) : gguf_q8_1_bytes(n, k, 1));
    return has_x_q8 || generic_fused(op, type, row, k, n) ? 0 : align256(gguf_q8_1_bytes(n, k, 0));
  }
  if (op_gemm(op)) {
    const bool mmq_layout = !op_packed(op) && type == gguf::kIQ3_S;
    if (!mmq_layout && ((prefill_route(op, type, row, k, n) && gguf::prefill_uses_xh((int)type, op_packed(op))) ||
                        small_fp16(op, type, row, k, n)))
      return align256(gguf::xh_bytes(n, k));
    return align256(mmq_layout ? gguf_q8_1_bytes(n, k, 1) : gguf::xq_bytes(n, k)) + split_ws(op, type, row, k, n);
  }
  if (decode_mma(op, type, row, k, n))  // x_q8 is converted into it
    return align256(gguf::xq_bytes(n, k)) + split_ws(op, type, row, k, n);
  if (packed_fused(op, row, k, n, has_x_q8 != 0) || rows_fused(op, type, row, k, n, has_x_q8 != 0)) return 0;
  return has_x_q8 ? 0 : align256(gguf_q8_1_bytes(n, k, 0));
}

}  // extern "C"

namespace {

// One product whose guards have passed (check_op returned k): the buffer checks, the plan and the
// launches. Every entry point runs the guards once and then this.
int run_checked(int op, const gguf_view* W, const gguf_view* X, int64_t type, int64_t row, const gguf_view* x_q8,
                int64_t k, void* y, size_t y_bytes, void* workspace, size_t workspace_bytes, void* stream) {
  const char* name = op_name(op);
  const int64_t n = X->size[0];
  if (n == 0) return GGUF_OK;
  if (y_bytes < (size_t)(n * row * elem_size(X->dtype))) return fail("%s: output buffer too small", name);
  const bool packed = op_packed(op);
  const bool gemm = op_gemm(op);
  hipStream_t s = (hipStream_t)stream;
  const DeviceScope scope(X->device);
  if (scope.err != hipSuccess) return hip_fail(scope.err, name, "device select");
  // sized on X's device, as the dispatch below decides (some plans depend on its CU count)
  const size_t need = gguf_op_workspace_bytes(op, type, row, k, n, x_q8 != nullptr);
  if (workspace_bytes < need || (need > 0 && !workspace))
    return fail("%s: workspace of %zu bytes needed, got %zu", name, need, workspace_bytes);
  if (reinterpret_cast<uintptr_t>(workspace) % 16 != 0) return fail("%s: workspace must be 16-byte aligned", name);
  hipError_t e;
  const int64_t s01 = n == 1 ? k : X->stride[0];
  const uint8_t* w = (const uint8_t*)W->data;
  const int64_t row_bytes = W->size[1];
  const int ydt = X->dtype;

  if (generic(type)) {
    const bool xxs = xxs_packed(op, type);
    if (xxs && prefill_route(op, type, row, k, n)) {  // IQ3_XXS unit layout: the fp16 prefill GEMM (xh layout)
      e = gguf::launch_quantize_xh(X->data, X->dtype, n, k, s01, (int)type, workspace, s);
      if (e != hipSuccess) return hip_fail(e, name, "quantize");
      e = gguf::launch_gemm_prefill((int)type, true, w, row_bytes, (int)row, (int)k, (const uint8_t*)workspace, (int)n,
                                    y, ydt, s);
      if (e != hipSuccess) return hip_fail(e, name, "gemm");
      return GGUF_OK;
    }
    if (gemm && generic_xq(type)) {  // the product ops' MMQ arithmetic in the xq layout
      e = gguf::launch_quantize_xq(X->data, X->dtype, n, k, s01, (int)type, false, workspace, s);
      if (e != hipSuccess) return hip_fail(e, name, "quantize");
      e = xxs ? gguf::launch_gemm_iq3xxs_packed(w, row_bytes, (int)row, (int)k, (const uint8_t*)workspace, (int)n, y,
                                               ydt, s)
              : gguf::launch_gemm_xq((int)type, w, row_bytes, (int)row, (int)k, (const uint8_t*)workspace, (int)n, y,
                                     ydt, true, nullptr, s);
      if (e != hipSuccess) return hip_fail(e, name, "gemm");
      return GGUF_OK;
    }
    if (xxs) {  // IQ3_XXS unit layout: the IQ3 stream GEMV
      if (!gguf::gemv_iq3xxs_stream_supported(row, row_bytes, k, 1, false))
        return fail("%s: K=%lld is past the packed IQ3_XXS GEMV's X staging", name, (long long)k);
      if (!x_q8 && generic_fused(op, type, row, k, n)) {
        e = gguf::launch_gemv_iq3xxs_stream(w, row_bytes, (int)row, (int)k, X->data, X->dtype, s01, (int)n, y, ydt, s);
        if (e != hipSuccess) return hip_fail(e, name, "gemv");
        return GGUF_OK;
      }
      const uint8_t* q8 = x_q8 ? (const uint8_t*)x_q8->data : (const uint8_t*)workspace;
      if (!x_q8) {
        e = gguf::launch_quantize(X->data, X->dtype, n, k, s01, (int)type, false, workspace, s);
        if (e != hipSuccess) return hip_fail(e, name, "quantize");
      }
      e = gguf::launch_gemv_iq3xxs_stream(w, row_bytes, (int)row, (int)k, q8, -1, 0, (int)n, y, ydt, s);
      if (e != hipSuccess) return hip_fail(e, name, "gemv");
      return GGUF_OK;
    }
    if (gemm) {  // Q2_K: the product ops' MMQ arithmetic, block_q8_1_mmq and the per-slice MFMA GEMM
      e = gguf::launch_quantize(X->data, X->dtype, n, k, s01, (int)type, true, workspace, s);
      if (e != hipSuccess) return hip_fail(e, name, "quantize");
      e = gguf::launch_gemm((int)type, w, row_bytes, (int)row, (int)k, (const uint8_t*)workspace, (int)n, y, ydt, s);
      if (e != hipSuccess) return hip_fail(e, name, "gemm");
      return GGUF_OK;
    }
    if (!x_q8 && generic_fused(op, type, row, k, n)) {  // quantisation inside the stream GEMV
      e = gguf::launch_gemv_generic_x((int)type, w, row_bytes, (int)row, (int)k, X->data, X->dtype, s01, (int)n, y,
                                      ydt, s);
      if (e != hipSuccess) return hip_fail(e, name, "gemv");
      return GGUF_OK;
    }
    const uint8_t* q8 = x_q8 ? (const uint8_t*)x_q8->data : (const uint8_t*)workspace;
    if (!x_q8) {
      e = gguf::launch_quantize(X->data, X->dtype, n, k, s01, (int)type, false, workspace, s);
      if (e != hipSuccess) return hip_fail(e, name, "quantize");
    }
    // the GEMV takes up to 8 activation rows per launch (the packed decode op allows 32)
    for (int64_t c = 0; c < n; c += 8) {
      const int64_t nc = n - c < 8 ? n - c : 8;
      e = gguf::launch_gemv_raw((int)type, w, row_bytes, (int)row, (int)k, q8 + c * (k / gguf::kQ81) * 36, (int)nc,
                                (uint8_t*)y + c * row * elem_size(X->dtype), ydt, s);
      if (e != hipSuccess) return hip_fail(e, name, "gemv");
    }
    return GGUF_OK;
  }

  // int8-MFMA GEMMs on the xq layout: the product ops with the MMQ arithmetic, the decode ops
  // (from vec_mma_from rows on, see decode_mma) with the decode ops' q8_1 arithmetic or the
  // caller's x_q8
  if ((gemm && (packed || type != gguf::kIQ3_S)) || (!gemm && decode_mma(op, type, row, k, n))) {
    const bool prefill = prefill_route(op, type, row, k, n);
    const bool fp16 = small_fp16(op, type, row, k, n);
    const bool xh = fp16 || (prefill && gguf::prefill_uses_xh((int)type, packed));
    // a K-split GEMM's slots and counters follow the xq copy; the quantise launch clears the
    // counters
    uint8_t* sws = nullptr;
    uint32_t* counters = nullptr;
    int nctr = 0;
    const SplitPlan sp = split_plan(op, type, row, k, n);
    if (sp.split > 1) {
      sws = (uint8_t*)workspace + align256(gguf::xq_bytes(n, k));
      counters = (uint32_t*)(sws + gguf::split_part_bytes(sp.split, sp.tiles, n));
      nctr = gguf::split_counters(sp.split, sp.tiles, n);
    }
    if (!gemm && x_q8)
      e = gguf::launch_q8_1_to_xq(x_q8->data, n, k, (int)type, workspace, s, counters, nctr);
    else if (xh)
      e = gguf::launch_quantize_xh(X->data, X->dtype, n, k, s01, (int)type, workspace, s);
    else
      e = gguf::launch_quantize_xq(X->data, X->dtype, n, k, s01, (int)type, !gemm, workspace, s, counters, nctr);
    if (e != hipSuccess) return hip_fail(e, name, "quantize");
    if (prefill)
      e = gguf::launch_gemm_prefill((int)type, packed, w, row_bytes, (int)row, (int)k, (const uint8_t*)workspace,
                                    (int)n, y, ydt, s);
    else if (fp16)
      e = gguf::launch_gemm_small_h((int)type, packed, w, row_bytes, (int)row, (int)k, (const uint8_t*)workspace,
                                    (int)n, y, ydt, s);
    else if (packed)
      e = gguf::launch_gemm_packed_xq(w, row_bytes, (int)row, (int)k, (const uint8_t*)workspace, (int)n, y, ydt, sws,
                                      s);
    else
      e = gguf::launch_gemm_xq((int)type, w, row_bytes, (int)row, (int)k, (const uint8_t*)workspace, (int)n, y, ydt,
                               gemm, sws, s);
    if (e != hipSuccess) return hip_fail(e, name, "gemm");
    return GGUF_OK;
  }
  if (gemm) {  // IQ3_S on plain rows: the MMQ layout and the per-slice MFMA GEMM
    e = gguf::launch_quantize(X->data, X->dtype, n, k, s01, (int)type, true, workspace, s);
    if (e != hipSuccess) return hip_fail(e, name, "quantize");
    e = gguf::launch_gemm((int)type, w, row_bytes, (int)row, (int)k, (const uint8_t*)workspace, (int)n, y, ydt, s);
    if (e != hipSuccess) return hip_fail(e, name, "gemm");
    return GGUF_OK;
  }
  if (packed_fused(op, row, k, n, x_q8 != nullptr)) {  // quantisation inside the GEMV
    e = gguf::launch_gemv_packed_x(w, row_bytes, (int)row, (int)k, X->data, X->dtype, s01, (int)n, y, ydt, s);
    if (e != hipSuccess) return hip_fail(e, name, "gemv");
    return GGUF_OK;
  }
  if (rows_fused(op, type, row, k, n, x_q8 != nullptr)) {  // quantisation inside the row-chunk GEMV
    e = gguf::launch_gemv_rows_x((int)type, w, row_bytes, (int)row, (int)k, X->data, X->dtype, s01, (int)n, y, ydt, s);
    if (e != hipSuccess) return hip_fail(e, name, "gemv");
    return GGUF_OK;
  }
  const uint8_t* q8 = (const uint8_t*)workspace;
  if (x_q8) {
    q8 = (const uint8_t*)x_q8->data;
  } else {
    e = gguf::launch_quantize(X->data, X->dtype, n, k, s01, (int)type, false, workspace, s);
    if (e != hipSuccess) return hip_fail(e, name, "quantize");
  }
  e = packed ? gguf::launch_gemv_packed(w, row_bytes, (int)row, (int)k, q8, (int)n, y, ydt, s)
             : gguf::launch_gemv_raw((int)type, w, row_bytes, (int)row, (int)k, q8, (int)n, y, ydt, s);
  if (e != hipSuccess) return hip_fail(e, name, "gemv");
  return GGUF_OK;
}

}  // namespace

extern "C" {

int gguf_mul_mat(int op, const gguf_view* W, const gguf_view* X, int64_t type, int64_t row, const gguf_view* x_q8,
                 void* y, size_t y_bytes, void* workspace, size_t workspace_bytes, void* stream) {
  g_err.clear();
  const int64_t k = check_op(op, W, X, type, row, x_q8);
  if (k < 0) return GGUF_EINVAL;
  return run_checked(op, W, X, type, row, x_q8, k, y, y_bytes, workspace, workspace_bytes, stream);
}

int gguf_mul_mat_alloc(int op, const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                       const gguf_view* x_q8, gguf_alloc_fn alloc, void* alloc_ctx, void* stream) {
  g_err.clear();
  const int64_t k = check_op(op, W, X, type, row, x_q8);
  if (k < 0) return GGUF_EINVAL;
  const char* name = op_name(op);
  if (!alloc) return fail("%s: no allocator given", name);
  const int64_t n = X->size[0];
  const size_t y_bytes = (size_t)(n * row * elem_size(X->dtype));
  void* y = alloc(alloc_ctx, GGUF_ALLOC_OUTPUT, y_bytes);
  if (!y && y_bytes) return fail("%s: the allocator returned no output buffer", name);
  if (n == 0) return GGUF_OK;
  const DeviceScope scope(X->device);
  if (scope.err != hipSuccess) return hip_fail(scope.err, name, "device select");
  const size_t need = gguf_op_workspace_bytes(op, type, row, k, n, x_q8 != nullptr);
  void* ws = nullptr;
  if (need) {
    ws = alloc(alloc_ctx, GGUF_ALLOC_WORKSPACE, need);
    if (!ws) return fail("%s: the allocator returned no workspace", name);
  }
  return run_checked(op, W, X, type, row, x_q8, k, y, y_bytes, ws, need, stream);
}

}  // extern "C"

namespace {

// The no-allocation variant's workspace: one statically sized device array per GPU, held until
// the process ends. Host code never uses the array's name as an address (on the host it is only
// a stand-in for the symbol); each device's address comes from hipGetSymbolAddress with that
// device current, once, and is kept here.
constexpr size_t kScratchBytes = GGUF_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

void* g_scratch_ptr[gguf::kMaxDevices] = {};
std::mutex g_scratch_mu;

// The current device's scratch address (the caller has made X's device current). The first call
// on a device may come inside a caller's stream capture: the symbol lookup runs with the capture
// mode relaxed (gguf::outside_capture).
hipError_t scratch_address(int device, void** out) {
  if (device < 0 || device >= gguf::kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[device]) {
    void* p = nullptr;
    hipError_t e = hipSuccess;
    gguf::outside_capture([&] { e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)); });
    if (e != hipSuccess) return e;
    g_scratch_ptr[device] = p;
  }
  *out = g_scratch_ptr[device];
  return hipSuccess;
}

}  // namespace

extern "C" {

size_t gguf_scratch_bytes(void) { return kScratchBytes; }

int gguf_mul_mat_noalloc(int op, const gguf_view* W, const gguf_view* X, int64_t type, int64_t row,
                         const gguf_view* x_q8, void* y, size_t y_bytes, void* stream) {
  g_err.clear();
  const int64_t k = check_op(op, W, X, type, row, x_q8);
  if (k < 0) return GGUF_EINVAL;
  const char* name = op_name(op);
  const int64_t n = X->size[0];
  if (n == 0) return GGUF_OK;
  const DeviceScope scope(X->device);
  if (scope.err != hipSuccess) return hip_fail(scope.err, name, "device select");
  const size_t need = gguf_op_workspace_bytes(op, type, row, k, n, x_q8 != nullptr);
  if (need > kScratchBytes)
    return fail("%s: needs a %zu-byte workspace, more than the %zu-byte static scratch of the no-allocation "
                "entry point (use gguf_mul_mat with a workspace)", name, need, kScratchBytes);
  void* ws = nullptr;
  const hipError_t e = scratch_address(X->device, &ws);
  if (e != hipSuccess) return hip_fail(e, name, "scratch address");
  return run_checked(op, W, X, type, row, x_q8, k, y, y_bytes, ws, kScratchBytes, stream);
}

#define GGUF_OP_Q8(fn, OP)                                                                                    \
  int fn(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row, const gguf_view* x_q8, void* y,   \
         size_t y_bytes, void* ws, size_t ws_bytes, void* stream) {                                           \
    return gguf_mul_mat(OP, W, X, type, row, x_q8, y, y_bytes, ws, ws_bytes, stream);                         \
  }
#define GGUF_OP_OWN(fn, OP)                                                                                  \
  int fn(const gguf_view* W, const gguf_view* X, int64_t type, int64_t row, void* y, size_t y_bytes, void* ws, \
         size_t ws_bytes, void* stream) {                                                                     \
    return gguf_mul_mat(OP, W, X, type, row, nullptr, y, y_bytes, ws, ws_bytes, stream);                      \
  }
GGUF_OP_Q8(gguf_lcpp_mul_mat_vec_q, GGUF_OP_MUL_MAT_VEC_Q)
GGUF_OP_OWN(gguf_lcpp_mul_mat_q, GGUF_OP_MUL_MAT_Q)
GGUF_OP_Q8(gguf_lcpp_mul_mat_vec_iq3, GGUF_OP_MUL_MAT_VEC_IQ3)
GGUF_OP_Q8(gguf_lcpp_mul_mat_vec_iq3_mma, GGUF_OP_MUL_MAT_VEC_IQ3_MMA)
GGUF_OP_Q8(gguf_lcpp_mul_mat_vec_own, GGUF_OP_MUL_MAT_VEC_OWN)
GGUF_OP_OWN(gguf_lcpp_mul_mat_mma_k, GGUF_OP_MUL_MAT_MMA_K)
GGUF_OP_Q8(gguf_lcpp_mul_mat_vec_iq3_mma_packed, GGUF_OP_MUL_MAT_VEC_IQ3_MMA_PACKED)
GGUF_OP_OWN(gguf_lcpp_mul_mat_iq3_packed, GGUF_OP_MUL_MAT_IQ3_PACKED)
#undef GGUF_OP_Q8
#undef GGUF_OP_OWN

int gguf_lcpp_quantize_q8_1(const gguf_view* X, int64_t type, int mmq, int vendored, void* out, size_t out_bytes,
                            void* stream) {
  g_err.clear();
  // lcpp_shim.cu:950-955: one combined guard
  if (!(X && type_served(type) && X->device >= 0 && X->ndim == 2 && X->stride[1] == 1 && X->size[1] % 512 == 0 &&
        !(mmq && type == kIQ1_M) && is_float(X->dtype)))
    return fail("lcpp_quantize_q8_1: bad arguments");
  if (vendored) return fail("lcpp_quantize_q8_1: no vendored quantizer in this build (vendored must be false)");
  const int64_t n = X->size[0], k = X->size[1];
  if (out_bytes < gguf_q8_1_bytes(n, k, mmq)) return fail("lcpp_quantize_q8_1: output buffer too small");
  if (n == 0) return GGUF_OK;
  const DeviceScope scope(X->device);
  if (scope.err != hipSuccess) return hip_fail(scope.err, "lcpp_quantize_q8_1", "device select");
  hipError_t e;
  const int64_t s01 = n == 1 ? k : X->stride[0];
  e = gguf::launch_quantize(X->data, X->dtype, n, k, s01, (int)type, mmq != 0, out, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "lcpp_quantize_q8_1", "quantize");
  return GGUF_OK;
}

size_t gguf_iq3_pack_scratch_bytes(int64_t rows, int64_t row_bytes) { return gguf::iq3_pack_scratch_bytes(rows, row_bytes); }

int gguf_dense_mul_mat(const gguf_view* W, const gguf_view* X, void* y, size_t y_bytes, void* stream) {
  g_err.clear();
  const char* name = "gguf_dense_mul_mat";
  if (!W || !X) return fail("%s: W and X must be given", name);
  if (W->ndim != 2 || X->ndim != 2) return fail("%s: W and X must be 2-D", name);
  if (!is_float(W->dtype) || X->dtype != W->dtype) return fail("%s: W and X must share one float dtype", name);
  const int64_t rows = W->size[0], k = W->size[1], n = X->size[0];
  if (X->size[1] != k) return fail("%s: X has %lld columns, W has %lld", name, (long long)X->size[1], (long long)k);
  if (!(k > 0 && k % 32 == 0 && k <= INT_MAX)) return fail("%s: K=%lld must be a positive multiple of 32", name, (long long)k);
  if (!(rows >= 1 && rows <= INT_MAX)) return fail("%s: W must have rows", name);
  if (n > 8) return fail("%s: at most 8 rows, got %lld", name, (long long)n);
  const int64_t es = elem_size(X->dtype);
  if (W->stride[1] != 1 || X->stride[1] != 1) return fail("%s: W and X inner stride must be 1", name);
  if ((rows > 1 && (W->stride[0] < k || (W->stride[0] * es) % 16)) || (n > 1 && (X->stride[0] < k || (X->stride[0] * es) % 16)))
    return fail("%s: row strides must be at least K and 16-byte multiples", name);
  if (reinterpret_cast<uintptr_t>(W->data) % 16 || reinterpret_cast<uintptr_t>(X->data) % 16)
    return fail("%s: W and X data must be 16-byte aligned", name);
  if (W->device < 0 || X->device < 0) return fail("%s: W and X must be CUDA tensors", name);
  if (W->device != X->device) return fail("%s: W and X must be on the same device", name);
  if (n == 0) return GGUF_OK;
  if (y_bytes < (size_t)(n * rows * es)) return fail("%s: output buffer too small", name);
  const DeviceScope scope(X->device);
  if (scope.err != hipSuccess) return hip_fail(scope.err, name, "device select");
  const hipError_t e = gguf::launch_dense(X->dtype, W->data, rows > 1 ? W->stride[0] : k, (int)rows, (int)k, X->data,
                                          n > 1 ? X->stride[0] : k, (int)n, y, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, name, "gemv");
  return GGUF_OK;
}

int gguf_iq3_pack(void* w, int64_t type, int64_t rows, int64_t row_bytes, int unpack, void* scratch,
                  size_t scratch_bytes, void* stream) {
  g_err.clear();
  if (type != gguf::kIQ3_S && type != kIQ3_XXS)
    return fail("gguf_iq3_pack: IQ3_S or IQ3_XXS only, got type %lld", (long long)type);
  const int64_t bs = type == kIQ3_XXS ? 98 : 110;
  if (!w || rows <= 0 || rows % 16 != 0 || row_bytes <= 0 || row_bytes % bs != 0)
    return fail("gguf_iq3_pack: rows must be a positive multiple of 16 and row bytes whole %s blocks",
                type == kIQ3_XXS ? "IQ3_XXS" : "IQ3_S");
  if (reinterpret_cast<uintptr_t>(w) % 16 != 0) return fail("gguf_iq3_pack: W data must be 16-byte aligned");
  if (scratch_bytes < gguf::iq3_pack_scratch_bytes(rows, row_bytes) || !scratch)
    return fail("gguf_iq3_pack: scratch of %zu bytes needed", gguf::iq3_pack_scratch_bytes(rows, row_bytes));
  const hipError_t e = gguf::launch_iq3_pack((int)type, (uint8_t*)w, rows, row_bytes, unpack != 0, (uint8_t*)scratch,
                                             scratch_bytes, (hipStream_t)stream);
  if (e != hipSuccess) return hip_fail(e, "gguf_iq3_pack", "pack");
  return GGUF_OK;
}

}  // extern "C"
